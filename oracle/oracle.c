/*
 * oracle.c - CPU restatement of Rapier's exact-verify MTP hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the CPU baseline timed by bench.py.  The product
 * library never links it.  Built with -ffp-contract=off so every float expression rounds exactly as written.
 *
 * Parity status (how each function is pinned; tests/test_oracle.py holds the checks):
 *   formats / Q6_K code layout  - ggml dequantize_row_q6_K element order and the mmvq:121-140 offsets; known-answer
 *                                 blocks built by hand.
 *   orc_q6k_block_dots          - closed form; cross-checked against the reference's lane-mapped dp4a form
 *                                 (orc_q6k_block_dots_lanes, mmvq:733-748) and against a float dequant dot.
 *   orc_quantize_q8_1           - closed form d = amax/127, q = roundf(x/d); sum in the 32-lane xor-tree order of
 *                                 mmvq:158-173.  Rounding mode and the fp16 finite guard live in an un-vendored Strata
 *                                 header (q8_1_finite.hpp): that part is "parity unpinned" and fixed here as
 *                                 round-half-away-from-zero and saturation to +-65504.
 *   orc_q6k_gemv / q8_0         - fp64 sum of exact integer dots; invariants (ncols=2 column == ncols=1, res ==
 *                                 plain + res, partials == sum of 4 squared rows) as in src/test_res.cpp:57-112.
 *   GDN conv / step             - closed forms of fgdn:40-133; checked against a brute-force fp64 matrix form and
 *                                 the zero-input / unit-decay special cases.
 *   attention                   - fp64 softmax(q K^T * scale) V; n_tok = 1 -> V0 and constant-K -> mean(V) cases.
 *   rms_norm_heads, rope_neox   - un-vendored in the reference (rms_norm_weighted, native_rope_apply): parity
 *                                 unpinned; the definitions follow the published RMSNorm and NEOX rotary formulas.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------------------------------------------ */
/* generators: splitmix64 finalizer over a counter, so any element can be drawn independently                   */

static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

uint64_t orc_rand_u64(uint64_t seed, uint64_t index) {
    return mix64(seed * 0xD1B54A32D192ED03ULL + (index + 1) * 0x9E3779B97F4A7C15ULL);
}

double orc_rand_unit(uint64_t seed, uint64_t index) {
    return (double) (orc_rand_u64(seed, index) >> 11) * (1.0 / 9007199254740992.0);
}

double orc_rand_normal(uint64_t seed, uint64_t index) {
    /* Box-Muller on two counter draws; u1 in (0,1] so the log is finite */
    const double u1 = 1.0 - orc_rand_unit(seed, 2 * index);
    const double u2 = orc_rand_unit(seed, 2 * index + 1);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

void orc_fill_normal(float* out, size_t n, uint64_t seed, double mean, double std) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) out[i] = (float) (mean + std * orc_rand_normal(seed, i));
}

/* one Q6_K block from its 256 codes, 16 sub-scales and super-scale (inverse of orc_q6k_code) */
static void pack_q6k(uint8_t* b, const uint8_t* codes, const int8_t* sc, uint16_t d) {
    uint8_t* ql = b;
    uint8_t* qh = b + 128;
    memset(b, 0, ORC_Q6K_BYTES);
    for (int e = 0; e < 256; ++e) {
        const int n = e / 128, r = e % 128, k = r / 32, l = r % 32;
        const int c = codes[e] & 63;
        uint8_t* lo = &ql[64 * n + (k & 1) * 32 + l];
        if (k >> 1) *lo |= (uint8_t) ((c & 15) << 4);
        else *lo |= (uint8_t) (c & 15);
        qh[32 * n + l] |= (uint8_t) ((c >> 4) << (2 * k));
    }
    memcpy(b + 192, sc, 16);
    memcpy(b + 208, &d, 2);
}

void orc_gen_q6k(uint8_t* w, size_t nblocks, uint64_t seed, double d_std) {
    const uint64_t s_codes = seed ^ 0x51ULL, s_sc = seed ^ 0x52ULL, s_d = seed ^ 0x53ULL;
#pragma omp parallel for schedule(static)
    for (size_t bi = 0; bi < nblocks; ++bi) {
        uint8_t codes[256];
        int8_t sc[16];
        for (int e = 0; e < 256; e += 8) {   /* eight 6-bit codes per 64-bit draw */
            uint64_t r = orc_rand_u64(s_codes, bi * 32 + (uint64_t) (e / 8));
            for (int m = 0; m < 8; ++m) codes[e + m] = (uint8_t) ((r >> (8 * m)) & 63);
        }
        uint64_t r0 = orc_rand_u64(s_sc, 2 * bi), r1 = orc_rand_u64(s_sc, 2 * bi + 1);
        for (int m = 0; m < 8; ++m) sc[m] = (int8_t) ((int) ((r0 >> (8 * m)) & 63) - 32);
        for (int m = 0; m < 8; ++m) sc[8 + m] = (int8_t) ((int) ((r1 >> (8 * m)) & 63) - 32);
        const uint16_t d = orc_f32_to_f16((float) fabs(d_std * orc_rand_normal(s_d, bi)));
        pack_q6k(w + bi * ORC_Q6K_BYTES, codes, sc, d);
    }
}

void orc_gen_q8_0(uint8_t* w, size_t nblocks, uint64_t seed, double d_std) {
#pragma omp parallel for schedule(static)
    for (size_t bi = 0; bi < nblocks; ++bi) {
        uint8_t* b = w + bi * ORC_Q8_0_BYTES;
        const uint16_t d = orc_f32_to_f16((float) fabs(d_std * orc_rand_normal(seed ^ 0x61ULL, bi)));
        memcpy(b, &d, 2);
        for (int m = 0; m < 4; ++m) {
            uint64_t r = orc_rand_u64(seed ^ 0x62ULL, bi * 4 + (uint64_t) m);
            for (int t = 0; t < 8; ++t) b[2 + 8 * m + t] = (uint8_t) ((r >> (8 * t)) & 0xff);
        }
    }
}

/* ------------------------------------------------------------------------------------------------------------ */
/* fp16                                                                                                          */

uint16_t orc_f32_to_f16(float x) {
    uint32_t f;
    memcpy(&f, &x, 4);
    const uint32_t sign = (f >> 16) & 0x8000u;
    const uint32_t absf = f & 0x7fffffffu;
    if (absf >= 0x7f800000u) return (uint16_t) (sign | 0x7c00u | (absf > 0x7f800000u ? 0x200u : 0u));
    if (absf >= 0x477ff000u) return (uint16_t) (sign | 0x7c00u); /* rounds to >= 65520: inf */
    if (absf < 0x38800000u) {                                   /* subnormal half (or zero) */
        if (absf < 0x33000000u) return (uint16_t) sign;          /* < 2^-25: rounds to 0 */
        const uint32_t exp = absf >> 23;
        const uint32_t mant = (absf & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - exp;                      /* 14..24 */
        uint32_t h = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (h & 1u))) ++h;
        return (uint16_t) (sign | h);
    }
    uint32_t h = ((absf - 0x38000000u) >> 13);
    const uint32_t rem = absf & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t) (sign | h);
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    uint32_t f;
    if (exp == 0) {
        if (mant == 0) f = sign;
        else {
            int e = -1;
            do { ++e; mant <<= 1; } while (!(mant & 0x400u));
            f = sign | ((uint32_t) (112 - e) << 23) | ((mant & 0x3ffu) << 13);
        }
    } else if (exp == 31) {
        f = sign | 0x7f800000u | (mant << 13);
    } else {
        f = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    float x;
    memcpy(&x, &f, 4);
    return x;
}

uint16_t orc_f16_sat(float x) {
    if (x > 65504.0f) return 0x7bffu;
    if (x < -65504.0f) return 0xfbffu;
    return orc_f32_to_f16(x);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Q8_1 quantizer (mmvq:158-173): per 32 elements, amax and sum by a 32-lane xor butterfly (offsets 16..1),     */
/* d = amax/127, q = roundf(x/d) (0 when amax == 0), ds = (fp16 d, fp16 sum) with the finite guard.            */

static float tree_sum32(const float* v) {
    float a[32], b[32];
    memcpy(a, v, sizeof a);
    for (int off = 16; off > 0; off >>= 1) {
        for (int l = 0; l < 32; ++l) b[l] = a[l] + a[l ^ off];
        memcpy(a, b, sizeof a);
    }
    return a[0];
}

static void quant_block(const float* x, uint8_t* y) {
    float amax = 0.0f;
    for (int l = 0; l < 32; ++l) amax = fmaxf(amax, fabsf(x[l]));
    const float sum = tree_sum32(x);
    const float d = amax / 127.0f;
    for (int l = 0; l < 32; ++l) {
        const int q = amax == 0.0f ? 0 : (int) roundf(x[l] / d);
        y[4 + l] = (uint8_t) (int8_t) q;
    }
    const uint16_t dh = orc_f16_sat(d), sh = orc_f16_sat(sum);
    memcpy(y, &dh, 2);
    memcpy(y + 2, &sh, 2);
}

void orc_quantize_q8_1(const float* x, uint8_t* y, int n_in, int ncols) {
    const int nb = n_in / 32 * ncols;
    for (int b = 0; b < nb; ++b) quant_block(x + 32 * b, y + ORC_Q8_1_BYTES * b);
}

void orc_dequantize_q8_1(const uint8_t* y, float* x, int n) {
    for (int b = 0; b < n / 32; ++b) {
        uint16_t dh;
        memcpy(&dh, y + ORC_Q8_1_BYTES * b, 2);
        const float d = orc_f16_to_f32(dh);
        for (int l = 0; l < 32; ++l) x[32 * b + l] = d * (float) (int8_t) y[ORC_Q8_1_BYTES * b + 4 + l];
    }
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Q6_K layout (ggml dequantize_row_q6_K; mmvq:121-140): element e of a 256-block, n = e/128, k = (e%128)/32,    */
/* l = e%32: low nibble of ql[64n + 32(k&1) + l] (high nibble when k >= 2), bits 2k..2k+1 of qh[32n + l],       */
/* sub-scale sc[8n + l/16 + 2k], weight = d * sc * (code - 32).                                                 */

int orc_q6k_code(const uint8_t* b, int e) {
    const int n = e / 128, r = e % 128, k = r / 32, l = r % 32;
    const uint8_t lo = b[64 * n + 32 * (k & 1) + l];
    const int nib = (k >> 1) ? (lo >> 4) : (lo & 15);
    const int hi = (b[128 + 32 * n + l] >> (2 * k)) & 3;
    return nib | (hi << 4);
}

static int q6k_scale(const uint8_t* b, int e) {
    const int n = e / 128, r = e % 128, k = r / 32, l = r % 32;
    return (int8_t) b[192 + 8 * n + l / 16 + 2 * k];
}

static float q6k_d(const uint8_t* b) {
    uint16_t h;
    memcpy(&h, b + 208, 2);
    return orc_f16_to_f32(h);
}

void orc_q6k_dequant_row(const uint8_t* w, float* y, int n) {
    for (int bi = 0; bi < n / 256; ++bi) {
        const uint8_t* b = w + (size_t) bi * ORC_Q6K_BYTES;
        const float d = q6k_d(b);
        for (int e = 0; e < 256; ++e)
            y[256 * bi + e] = d * (float) q6k_scale(b, e) * (float) (orc_q6k_code(b, e) - 32);
    }
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Q4_K / Q5_K (token_embd of Q5_K_M files; dequantized by strata::dequantize_q4_K / q5_K at qw:109-115, a      */
/* dependency absent from the reference tree: restated from ggml's published dequantize_row_q4_K / q5_K).       */
/* A 256-block is 8 sub-blocks of 32 with a 6-bit scale and a 6-bit min each, packed in 12 bytes: for j < 4     */
/* scale = s[j] & 63, min = s[j+4] & 63; for j >= 4 scale = (s[j+4] & 15) | (s[j-4] >> 6) << 4,                  */
/* min = (s[j+4] >> 4) | (s[j] >> 6) << 4.  weight = d * scale * q - dmin * min.                                */
/* Q4_K (144 B): d, dmin (fp16), scales[12], qs[128]; sub-block 2c takes the low nibbles of qs[32c .. 32c+31],   */
/* sub-block 2c+1 their high nibbles.  Q5_K (176 B): d, dmin, scales[12], qh[32], qs[128]; element l of          */
/* sub-block j gains bit j of qh[l] as its fifth bit (16).                                                      */

static void k4_scale_min(const uint8_t* s, int j, int* sc, int* m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

static float f16_at(const uint8_t* p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return orc_f16_to_f32(h);
}

void orc_q4k_dequant_row(const uint8_t* w, float* y, int n) {
    for (int bi = 0; bi < n / 256; ++bi) {
        const uint8_t* b = w + (size_t) bi * ORC_Q4K_BYTES;
        const float d = f16_at(b), dmin = f16_at(b + 2);
        const uint8_t* qs = b + 16;
        for (int c = 0; c < 4; ++c) {
            int s0, m0, s1, m1;
            k4_scale_min(b + 4, 2 * c, &s0, &m0);
            k4_scale_min(b + 4, 2 * c + 1, &s1, &m1);
            const float d0 = d * (float) s0, mm0 = dmin * (float) m0, d1 = d * (float) s1, mm1 = dmin * (float) m1;
            for (int l = 0; l < 32; ++l) {
                y[256 * bi + 64 * c + l] = d0 * (float) (qs[32 * c + l] & 15) - mm0;
                y[256 * bi + 64 * c + 32 + l] = d1 * (float) (qs[32 * c + l] >> 4) - mm1;
            }
        }
    }
}

void orc_q5k_dequant_row(const uint8_t* w, float* y, int n) {
    for (int bi = 0; bi < n / 256; ++bi) {
        const uint8_t* b = w + (size_t) bi * ORC_Q5K_BYTES;
        const float d = f16_at(b), dmin = f16_at(b + 2);
        const uint8_t* qh = b + 16;
        const uint8_t* qs = b + 48;
        for (int c = 0; c < 4; ++c) {
            int s0, m0, s1, m1;
            k4_scale_min(b + 4, 2 * c, &s0, &m0);
            k4_scale_min(b + 4, 2 * c + 1, &s1, &m1);
            const float d0 = d * (float) s0, mm0 = dmin * (float) m0, d1 = d * (float) s1, mm1 = dmin * (float) m1;
            for (int l = 0; l < 32; ++l) {
                const int q0 = (qs[32 * c + l] & 15) | (((qh[l] >> (2 * c)) & 1) << 4);
                const int q1 = (qs[32 * c + l] >> 4) | (((qh[l] >> (2 * c + 1)) & 1) << 4);
                y[256 * bi + 64 * c + l] = d0 * (float) q0 - mm0;
                y[256 * bi + 64 * c + 32 + l] = d1 * (float) q1 - mm1;
            }
        }
    }
}

static const int8_t* q81_qs(const uint8_t* xq, int j) { return (const int8_t*) (xq + (size_t) ORC_Q8_1_BYTES * j + 4); }
static float q81_d(const uint8_t* xq, int j) {
    uint16_t h;
    memcpy(&h, xq + (size_t) ORC_Q8_1_BYTES * j, 2);
    return orc_f16_to_f32(h);
}

void orc_q6k_block_dots(const uint8_t* w, const uint8_t* xq, int32_t* out, int n_in, int n_out) {
    const int nb = n_in / 256, nj = n_in / 32;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < n_out; ++r) {
        for (int bi = 0; bi < nb; ++bi) {
            const uint8_t* b = w + ((size_t) r * nb + bi) * ORC_Q6K_BYTES;
            for (int jj = 0; jj < 8; ++jj) {
                const int8_t* q8 = q81_qs(xq, 8 * bi + jj);
                int32_t acc = 0;
                for (int l = 0; l < 32; ++l) {
                    const int e = 32 * jj + l;
                    acc += q6k_scale(b, e) * (orc_q6k_code(b, e) - 32) * (int) q8[l];
                }
                out[(size_t) r * nj + 8 * bi + jj] = acc;
            }
        }
    }
}

/* the reference's per-lane form: lane iqs of a block, two dp4a each (mmvq:642-655, 733-748) */
static int dp4a(int a, int b) {
    int s = 0;
    for (int m = 0; m < 4; ++m) s += (int) (int8_t) (a >> (8 * m)) * (int) (int8_t) (b >> (8 * m));
    return s;
}
static int load_b2(const uint8_t* p, int i32) {
    return (int) ((uint32_t) p[4 * i32] | ((uint32_t) p[4 * i32 + 1] << 8) | ((uint32_t) p[4 * i32 + 2] << 16) |
                  ((uint32_t) p[4 * i32 + 3] << 24));
}

void orc_q6k_block_dots_lanes(const uint8_t* w, const uint8_t* xq, int32_t* out, int n_in, int n_out) {
    const int nb = n_in / 256, nj = n_in / 32;
    memset(out, 0, sizeof(int32_t) * (size_t) nj * (size_t) n_out);
    for (int r = 0; r < n_out; ++r) {
        for (int bi = 0; bi < nb; ++bi) {
            const uint8_t* b = w + ((size_t) r * nb + bi) * ORC_Q6K_BYTES;
            for (int iqs = 0; iqs < 32; ++iqs) {
                const int bq8_offset = 4 * (iqs / 16) + (iqs % 16) / 8;
                const int scale_offset = 8 * (iqs / 16) + (iqs % 16) / 4;
                const int vh_shift = 2 * ((iqs % 16) / 8);
                const int vl = load_b2(b, iqs);
                const int vh = (int) ((uint32_t) load_b2(b + 128, 8 * (iqs / 16) + iqs % 8) >> vh_shift);
                for (int i = 0; i < 2; ++i) {
                    const int sc = (int8_t) b[192 + scale_offset + 4 * i];
                    const int vil = (int) (((uint32_t) vl >> (4 * i)) & 0x0f0f0f0fu);
                    const int vih = (int) ((((uint32_t) vh >> (4 * i)) << 4) & 0x30303030u);
                    int vi = 0;
                    for (int m = 0; m < 4; ++m) {   /* bytewise (vil|vih) - 32, no saturation for codes 0..63 */
                        const int byte = (((vil | vih) >> (8 * m)) & 0xff) - 32;
                        vi |= (byte & 0xff) << (8 * m);
                    }
                    const int j = 8 * bi + bq8_offset + 2 * i;
                    const int u = load_b2((const uint8_t*) q81_qs(xq, j), iqs % 8);
                    out[(size_t) r * nj + j] += dp4a(vi, u) * sc;
                }
            }
        }
    }
}

void orc_q8_0_block_dots(const uint8_t* w, const uint8_t* xq, int32_t* out, int n_in, int n_out) {
    const int nj = n_in / 32;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < n_out; ++r) {
        for (int j = 0; j < nj; ++j) {
            const uint8_t* b = w + ((size_t) r * nj + j) * ORC_Q8_0_BYTES;
            const int8_t* q8 = q81_qs(xq, j);
            int32_t acc = 0;
            for (int l = 0; l < 32; ++l) acc += (int) (int8_t) b[2 + l] * (int) q8[l];
            out[(size_t) r * nj + j] = acc;
        }
    }
}

/* ------------------------------------------------------------------------------------------------------------ */
/* fp64 GEMVs with the residual epilogue (mmvq:3096-3140): y = acc + res, partials[g] = sum of 4 rows' y^2      */

static void gemv_epilogue(const float* res, double* y, double* partials, int n_out, int ncols) {
    const int np = (n_out + 3) / 4;
    for (int c = 0; c < ncols; ++c) {
        double* yc = y + (size_t) c * n_out;
        if (res)
            for (int r = 0; r < n_out; ++r) yc[r] += (double) res[(size_t) c * n_out + r];
        if (partials)
            for (int g = 0; g < np; ++g) {
                double p = 0.0;
                for (int r = 4 * g; r < 4 * g + 4 && r < n_out; ++r) p += yc[r] * yc[r];
                partials[(size_t) c * np + g] = p;
            }
    }
}

void orc_q6k_gemv(const uint8_t* w, const uint8_t* xq, const float* res, double* y, double* partials, int n_in,
                  int n_out, int ncols) {
    const int nb = n_in / 256, nj = n_in / 32;
    for (int c = 0; c < ncols; ++c) {
        const uint8_t* xc = xq + (size_t) c * nj * ORC_Q8_1_BYTES;
#pragma omp parallel for schedule(static)
        for (int r = 0; r < n_out; ++r) {
            double acc = 0.0;
            for (int bi = 0; bi < nb; ++bi) {
                const uint8_t* b = w + ((size_t) r * nb + bi) * ORC_Q6K_BYTES;
                double blk = 0.0;
                for (int jj = 0; jj < 8; ++jj) {
                    const int8_t* q8 = q81_qs(xc, 8 * bi + jj);
                    int32_t isum = 0;
                    for (int l = 0; l < 32; ++l) {
                        const int e = 32 * jj + l;
                        isum += q6k_scale(b, e) * (orc_q6k_code(b, e) - 32) * (int) q8[l];
                    }
                    blk += (double) q81_d(xc, 8 * bi + jj) * (double) isum;
                }
                acc += (double) q6k_d(b) * blk;
            }
            y[(size_t) c * n_out + r] = acc;
        }
    }
    gemv_epilogue(res, y, partials, n_out, ncols);
}

void orc_q8_0_gemv(const uint8_t* w, const uint8_t* xq, const float* res, double* y, double* partials, int n_in,
                   int n_out, int ncols) {
    const int nj = n_in / 32;
    for (int c = 0; c < ncols; ++c) {
        const uint8_t* xc = xq + (size_t) c * nj * ORC_Q8_1_BYTES;
#pragma omp parallel for schedule(static)
        for (int r = 0; r < n_out; ++r) {
            double acc = 0.0;
            for (int j = 0; j < nj; ++j) {
                const uint8_t* b = w + ((size_t) r * nj + j) * ORC_Q8_0_BYTES;
                uint16_t dh;
                memcpy(&dh, b, 2);
                const int8_t* q8 = q81_qs(xc, j);
                int32_t isum = 0;
                for (int l = 0; l < 32; ++l) isum += (int) (int8_t) b[2 + l] * (int) q8[l];
                acc += (double) orc_f16_to_f32(dh) * (double) q81_d(xc, j) * (double) isum;
            }
            y[(size_t) c * n_out + r] = acc;
        }
    }
    gemv_epilogue(res, y, partials, n_out, ncols);
}

/* Q4_K / Q5_K x Q8_1 GEMV (native_q4_k_mmvq / native_q5_k_mmvq, mmvq:562-640 and 185-300, with the residual
 * epilogue of mmvq:3202-3294): per weight block and Q8_1 block j (32 elements, sub-block j of the 256-block), the
 * exact integer dot sum(q u) and code sum sum(u) (vec_dot_q4_K/q5_K_q8_1_impl_vmmq's dot1 / dot2), then
 * d * sc_j * d8_j * dot1 - dmin * m_j * d8_j * dot2, accumulated in fp64. */
static void kquant_gemv(int five, const uint8_t* w, const uint8_t* xq, const float* res, double* y, double* partials,
                        int n_in, int n_out, int ncols) {
    const int nb = n_in / 256, bytes = five ? ORC_Q5K_BYTES : ORC_Q4K_BYTES;
    for (int c = 0; c < ncols; ++c) {
        const uint8_t* xc = xq + (size_t) c * (n_in / 32) * ORC_Q8_1_BYTES;
#pragma omp parallel for schedule(static)
        for (int r = 0; r < n_out; ++r) {
            double acc = 0.0;
            for (int bi = 0; bi < nb; ++bi) {
                const uint8_t* b = w + ((size_t) r * nb + bi) * bytes;
                const double d = f16_at(b), dmin = f16_at(b + 2);
                const uint8_t* qh = b + 16;
                const uint8_t* qs = b + (five ? 48 : 16);
                for (int j = 0; j < 8; ++j) {
                    int sc, m;
                    k4_scale_min(b + 4, j, &sc, &m);
                    const int8_t* u = q81_qs(xc, 8 * bi + j);
                    int32_t dot = 0, su = 0;
                    for (int l = 0; l < 32; ++l) {
                        int q = (qs[32 * (j / 2) + l] >> (4 * (j & 1))) & 15;
                        if (five) q |= ((qh[l] >> j) & 1) << 4;
                        dot += q * (int) u[l];
                        su += (int) u[l];
                    }
                    const double d8 = q81_d(xc, 8 * bi + j);
                    acc += d * sc * d8 * (double) dot - dmin * m * d8 * (double) su;
                }
            }
            y[(size_t) c * n_out + r] = acc;
        }
    }
    gemv_epilogue(res, y, partials, n_out, ncols);
}

void orc_q4k_gemv(const uint8_t* w, const uint8_t* xq, const float* res, double* y, double* partials, int n_in,
                  int n_out, int ncols) {
    kquant_gemv(0, w, xq, res, y, partials, n_in, n_out, ncols);
}

void orc_q5k_gemv(const uint8_t* w, const uint8_t* xq, const float* res, double* y, double* partials, int n_in,
                  int n_out, int ncols) {
    kquant_gemv(1, w, xq, res, y, partials, n_in, n_out, ncols);
}

/* fp32 timing build of the same GEMV: per 256-block, decode to int8, integer dots per 16 elements, then the
 * fp32 accumulation d8 * (sc * dot) as in mmvq:642-655.  Threaded over rows. */
void orc_q6k_gemv_f32_omp(const uint8_t* w, const uint8_t* xq, const float* res, float* y, float* partials,
                          int n_in, int n_out, int ncols, int threads) {
    const int nb = n_in / 256, nj = n_in / 32, np = (n_out + 3) / 4;
#pragma omp parallel for schedule(static) num_threads(threads)
    for (int r = 0; r < n_out; ++r) {
        float acc[16] = {0};
        for (int bi = 0; bi < nb; ++bi) {
            const uint8_t* b = w + ((size_t) r * nb + bi) * ORC_Q6K_BYTES;
            const uint8_t* ql = b;
            const uint8_t* qh = b + 128;
            const int8_t* sc = (const int8_t*) (b + 192);
            int8_t q[256];
            for (int n = 0; n < 2; ++n)
                for (int l = 0; l < 32; ++l) {
                    const int h = qh[32 * n + l];
                    q[128 * n + l] = (int8_t) (((ql[64 * n + l] & 15) | ((h & 3) << 4)) - 32);
                    q[128 * n + 32 + l] = (int8_t) (((ql[64 * n + 32 + l] & 15) | (((h >> 2) & 3) << 4)) - 32);
                    q[128 * n + 64 + l] = (int8_t) (((ql[64 * n + l] >> 4) | (((h >> 4) & 3) << 4)) - 32);
                    q[128 * n + 96 + l] = (int8_t) (((ql[64 * n + 32 + l] >> 4) | (((h >> 6) & 3) << 4)) - 32);
                }
            const float d = q6k_d(b);
            for (int c = 0; c < ncols; ++c) {
                const uint8_t* xc = xq + (size_t) c * nj * ORC_Q8_1_BYTES;
                float blk = 0.0f;
                for (int jj = 0; jj < 8; ++jj) {
                    const int8_t* q8 = q81_qs(xc, 8 * bi + jj);
                    const int n = jj / 4, k = jj % 4;
                    int d0 = 0, d1 = 0;
                    for (int l = 0; l < 16; ++l) d0 += q[32 * jj + l] * q8[l];
                    for (int l = 16; l < 32; ++l) d1 += q[32 * jj + l] * q8[l];
                    const int s = sc[8 * n + 2 * k] * d0 + sc[8 * n + 1 + 2 * k] * d1;
                    blk += q81_d(xc, 8 * bi + jj) * (float) s;
                }
                acc[c] += d * blk;
            }
        }
        for (int c = 0; c < ncols; ++c) {
            float v = acc[c];
            if (res) v += res[(size_t) c * n_out + r];
            y[(size_t) c * n_out + r] = v;
        }
    }
    if (partials)
        for (int c = 0; c < ncols; ++c)
            for (int g = 0; g < np; ++g) {
                float p = 0.0f;
                for (int r = 4 * g; r < 4 * g + 4 && r < n_out; ++r) p += y[(size_t) c * n_out + r] * y[(size_t) c * n_out + r];
                partials[(size_t) c * np + g] = p;
            }
}

/* ------------------------------------------------------------------------------------------------------------ */
/* epilogues (qw:602-715)                                                                                       */

void orc_row_sum_partials(const float* x, double* partials, int n) {
    for (int g = 0; g < (n + 3) / 4; ++g) {
        double p = 0.0;
        for (int r = 4 * g; r < 4 * g + 4 && r < n; ++r) p += (double) x[r] * (double) x[r];
        partials[g] = p;
    }
}

double orc_rms_inv(const double* partials, int nparts, int cols, double eps) {
    double ss = 0.0;
    for (int p = 0; p < nparts; ++p) ss += partials[p];
    return 1.0 / sqrt(ss / (double) cols + eps);
}

void orc_rms_norm_out(const float* x, const float* w, double inv, double* out, int n) {
    for (int i = 0; i < n; ++i) out[i] = (double) x[i] * (double) w[i] * inv;
}

static double silu_d(double v) { return v / (1.0 + exp(-v)); }
static double sigmoid_d(double v) { return 1.0 / (1.0 + exp(-v)); }

void orc_swiglu(const float* up, const float* gate, double* out, int n) {
    for (int i = 0; i < n; ++i) out[i] = silu_d((double) gate[i]) * (double) up[i];
}

void orc_sig_mul(const float* o, const float* g, double* out, int n) {
    for (int i = 0; i < n; ++i) out[i] = (double) o[i] * sigmoid_d((double) g[i]);
}

void orc_beta_gate(const float* beta_in, const float* alpha, const float* dt, const float* ssm_a, double* beta_out,
                   double* gate_out, int n) {
    for (int i = 0; i < n; ++i) {
        beta_out[i] = sigmoid_d((double) beta_in[i]);
        const double v = (double) alpha[i] + (double) dt[i];
        gate_out[i] = (v > 20.0 ? v : log1p(exp(v))) * (double) ssm_a[i];
    }
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Gated DeltaNet (fgdn:40-133)                                                                                 */

void orc_gdn_conv_l2(float* hist, const float* x, const float* w, double* h, int channels, int qk_heads, double eps) {
    for (int c = 0; c < channels; ++c) {
        const double sum = (double) hist[3 * c] * w[4 * c] + (double) hist[3 * c + 1] * w[4 * c + 1] +
                           (double) hist[3 * c + 2] * w[4 * c + 2] + (double) x[c] * w[4 * c + 3];
        hist[3 * c] = hist[3 * c + 1];
        hist[3 * c + 1] = hist[3 * c + 2];
        hist[3 * c + 2] = x[c];
        h[c] = silu_d(sum);
    }
    for (int hd = 0; hd < qk_heads; ++hd) {
        double ss = 0.0;
        for (int i = 0; i < 128; ++i) ss += h[128 * hd + i] * h[128 * hd + i];
        const double s = 1.0 / sqrt(ss + eps);
        for (int i = 0; i < 128; ++i) h[128 * hd + i] *= s;
    }
}

void orc_gdn_step_norm(double* state, const double* q, const double* k, const double* v, const double* gate,
                       const double* beta, const float* z, const float* gamma, double eps, double* y, int h_k,
                       int h_v) {
    const int S = 128;
    for (int hd = 0; hd < h_v; ++hd) {
        const int qh = hd % h_k;
        const double g = exp(gate[hd]);
        double o[128];
        for (int j = 0; j < S; ++j) {
            double kv = 0.0;
            for (int i = 0; i < S; ++i) kv += state[((size_t) i * h_v + hd) * S + j] * k[qh * S + i];
            const double delta = (v[hd * S + j] - g * kv) * beta[hd];
            double oj = 0.0;
            for (int i = 0; i < S; ++i) {
                double* s = &state[((size_t) i * h_v + hd) * S + j];
                *s = g * *s + k[qh * S + i] * delta;
                oj += *s * q[qh * S + i];
            }
            o[j] = oj / sqrt((double) S);
        }
        double ss = 0.0;
        for (int j = 0; j < S; ++j) ss += o[j] * o[j];
        const double scale = 1.0 / sqrt(ss / (double) S + eps);
        for (int j = 0; j < S; ++j) y[hd * S + j] = o[j] * scale * (double) gamma[j] * silu_d((double) z[hd * S + j]);
    }
}

/* ------------------------------------------------------------------------------------------------------------ */
/* attention (qw:384-442): per q-head h, kv head h / (n_head / n_kv), softmax over n_tok positions             */

void orc_gqa_decode(const float* q, const uint16_t* kc, const uint16_t* vc, double* o, int n_head, int n_kv, int hd,
                    int n_tok, double scale) {
    double* p = (double*) malloc(sizeof(double) * (size_t) n_tok);
    for (int h = 0; h < n_head; ++h) {
        const int kv = h / (n_head / n_kv);
        double m = -INFINITY;
        for (int t = 0; t < n_tok; ++t) {
            const uint16_t* kk = kc + ((size_t) t * n_kv + kv) * hd;
            double dot = 0.0;
            for (int d = 0; d < hd; ++d) dot += (double) q[h * hd + d] * (double) orc_f16_to_f32(kk[d]);
            p[t] = dot * scale;
            if (p[t] > m) m = p[t];
        }
        double sum = 0.0;
        for (int t = 0; t < n_tok; ++t) { p[t] = exp(p[t] - m); sum += p[t]; }
        for (int d = 0; d < hd; ++d) {
            double acc = 0.0;
            for (int t = 0; t < n_tok; ++t) acc += p[t] * (double) orc_f16_to_f32(vc[((size_t) t * n_kv + kv) * hd + d]);
            o[h * hd + d] = acc / sum;
        }
    }
    free(p);
}

void orc_rms_norm_heads(const float* x, const float* w, double* out, int rows, int cols, double eps) {
    for (int r = 0; r < rows; ++r) {
        double ss = 0.0;
        for (int c = 0; c < cols; ++c) ss += (double) x[r * cols + c] * (double) x[r * cols + c];
        const double inv = 1.0 / sqrt(ss / (double) cols + eps);
        for (int c = 0; c < cols; ++c) out[r * cols + c] = (double) x[r * cols + c] * inv * (double) w[c];
    }
}

void orc_rope_neox(const double* x, double* out, int heads, int hd, int n_rot, int pos, double theta) {
    const int half = n_rot / 2;
    for (int h = 0; h < heads; ++h) {
        const double* xi = x + (size_t) h * hd;
        double* yo = out + (size_t) h * hd;
        for (int d = 0; d < hd; ++d) yo[d] = xi[d];
        for (int i = 0; i < half; ++i) {
            const double ang = (double) pos * pow(theta, -2.0 * i / (double) n_rot);
            const double c = cos(ang), s = sin(ang);
            yo[i] = xi[i] * c - xi[i + half] * s;
            yo[i + half] = xi[i] * s + xi[i + half] * c;
        }
    }
}

/* YaRN RoPE as the reference configures it (qw:1991-1999: freq_base, factor, original context, ext_factor 1,
 * attn_factor 1, beta_fast 32, beta_slow 1), applied by strata's native_rope_apply (absent from the reference tree):
 * restated from the published YaRN algorithm as ggml implements it (rope_yarn, ggml_rope_yarn_corr_dims).  For pair i
 * (rotary dims i and i + n_rot/2): theta_extrap = pos * base^(-2i/n_rot), theta_interp = theta_extrap / factor,
 * ramp = 1 - clamp((i - low) / max(0.001, high - low), 0, 1) with low = max(0, floor(corr(beta_fast))),
 * high = min(n_rot - 1, ceil(corr(beta_slow))), corr(b) = n_rot ln(orig_ctx / (2 pi b)) / (2 ln base);
 * theta = theta_interp (1 - ramp ext) + theta_extrap ramp ext; cos, sin scaled by
 * attn_factor (1 + 0.1 ln factor) when ext != 0.  factor 1 is plain NEOX RoPE. */
void orc_rope_yarn(const double* x, double* out, int heads, int hd, int n_rot, int pos, double base, double factor,
                   double orig_ctx, double ext_factor, double attn_factor, double beta_fast, double beta_slow) {
    const int half = n_rot / 2;
    const double pi = 3.14159265358979323846;
    const double cf = n_rot * log(orig_ctx / (beta_fast * 2.0 * pi)) / (2.0 * log(base));
    const double cs = n_rot * log(orig_ctx / (beta_slow * 2.0 * pi)) / (2.0 * log(base));
    const double low = fmax(0.0, floor(cf)), high = fmin((double) (n_rot - 1), ceil(cs));
    const double mscale = ext_factor != 0.0 ? attn_factor * (1.0 + 0.1 * log(factor)) : attn_factor;
    for (int h = 0; h < heads; ++h) {
        const double* xi = x + (size_t) h * hd;
        double* yo = out + (size_t) h * hd;
        for (int d = 0; d < hd; ++d) yo[d] = xi[d];
        for (int i = 0; i < half; ++i) {
            const double te = (double) pos * pow(base, -2.0 * i / (double) n_rot);
            const double ti = te / factor;
            const double y = ((double) i - low) / fmax(0.001, high - low);
            const double ramp = (1.0 - fmin(1.0, fmax(0.0, y))) * ext_factor;
            const double th = ti * (1.0 - ramp) + te * ramp;
            const double c = cos(th) * mscale, s = sin(th) * mscale;
            yo[i] = xi[i] * c - xi[i + half] * s;
            yo[i + half] = xi[i] * s + xi[i + half] * c;
        }
    }
}

int orc_argmax(const float* l, int n) {
    int best = 0;
    for (int i = 1; i < n; ++i)
        if (l[i] > l[best]) best = i;
    return best;
}

/* topk_out (qw:2513-2531) restated: scan the logits once; the first k fill the list, which is then sorted by logit,
 * descending; afterwards a logit strictly greater than the list's last replaces it and moves up past every strictly
 * smaller entry.  The reference sorts the first k with std::sort, which leaves the order of equal logits among them
 * unspecified; this restatement sorts them stably (lower id first), the order the rest of the scan gives equal logits.
 * With n < k the list is never sorted (as in the reference) and holds the n logits in id order. */
int orc_topk(const float* l, int n, int k, int* ids, float* vals) {
    int m = 0;
    for (int i = 0; i < n; ++i) {
        if (m < k) {
            ids[m] = i;
            vals[m] = l[i];
            ++m;
            if (m == k) {   /* stable insertion sort, descending */
                for (int a = 1; a < k; ++a) {
                    const int id = ids[a];
                    const float v = vals[a];
                    int b = a;
                    while (b > 0 && v > vals[b - 1]) {
                        ids[b] = ids[b - 1];
                        vals[b] = vals[b - 1];
                        --b;
                    }
                    ids[b] = id;
                    vals[b] = v;
                }
            }
        } else if (l[i] > vals[k - 1]) {
            int j = k - 1;
            ids[j] = i;
            vals[j] = l[i];
            for (; j > 0 && vals[j] > vals[j - 1]; --j) {
                const int ti = ids[j];
                const float tv = vals[j];
                ids[j] = ids[j - 1];
                vals[j] = vals[j - 1];
                ids[j - 1] = ti;
                vals[j - 1] = tv;
            }
        }
    }
    return m;
}
