/*
 * cpu_round.c - the reference's ggml CPU path for one exact-verify MTP round, restated as a SIMD timing build.
 *
 * TEST INFRASTRUCTURE ONLY: bench.py times these functions on the host cores as the reported CPU baseline
 * (`cpu_baseline`, kind "port"), and tests/test_oracle.py checks them against the fp64 oracle (oracle.c).  Nothing in
 * the product library links or calls it.
 *
 * The arithmetic is the reference's (ggml's Q6_K x Q8_1 CPU dot, restated by mmvq:642-655 / 753-789 for the GPU):
 * per Q8_1 block, d8 * sum over its two 16-element sub-blocks of sc * (sum of (q6 - 32) q8), per Q6_K block times d.
 * Integer dots run on AVX2 (vpmaddubsw on the unsigned 0..63 codes, the -32 folded in through the per-16 sums of the
 * activation codes) or on AVX-512 VNNI (vpdpbusd) where the CPU has it; fp32 accumulation in vector lanes, so the
 * summation order is not the oracle's (tolerance-checked).  Rows are split over OpenMP threads.
 *   cpr_q6k_gemv        y = W x (+ res, 4-row partials) for 1 or 2 columns (mmvq:3096-3140)
 *   cpr_gdn_layer       conv + SiLU + L2, beta/gate, delta-rule step + RMSNorm * SiLU(z) for ntok tokens (fgdn:40-133,
 *                       qw:707-715), value heads over threads
 *   cpr_gqa_decode      softmax(q K^T * scale) V over an fp16 cache for ntok query tokens (qw:384-442), one pass over
 *                       K / V per KV head chunk (online softmax), then a merge
 */
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { Q6K = 210, Q81 = 36 };

static float f16_to_f32(uint16_t h) { return _cvtsh_ss(h); }

/* ---- Q6_K x Q8_1 ------------------------------------------------------------------------------------------------ */
/* the 256 unsigned codes (0..63) of a Q6_K block in element order (ggml dequantize_row_q6_K): four 32-code groups per
 * 128-element half, group g of half n = Q8_1 block 4 n + g */
static inline void q6k_codes(const uint8_t* b, __m256i q[8]) {
    const __m256i m4 = _mm256_set1_epi8(0x0f), m2 = _mm256_set1_epi8(0x03);
    for (int n = 0; n < 2; ++n) {
        const __m256i l0 = _mm256_loadu_si256((const __m256i*) (b + 64 * n));
        const __m256i l1 = _mm256_loadu_si256((const __m256i*) (b + 64 * n + 32));
        const __m256i h = _mm256_loadu_si256((const __m256i*) (b + 128 + 32 * n));
        const __m256i h0 = _mm256_slli_epi16(_mm256_and_si256(h, m2), 4);
        const __m256i h1 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 2), m2), 4);
        const __m256i h2 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 4), m2), 4);
        const __m256i h3 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 6), m2), 4);
        q[4 * n + 0] = _mm256_or_si256(_mm256_and_si256(l0, m4), h0);
        q[4 * n + 1] = _mm256_or_si256(_mm256_and_si256(l1, m4), h1);
        q[4 * n + 2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l0, 4), m4), h2);
        q[4 * n + 3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l1, 4), m4), h3);
    }
}

/* per Q8_1 block of a column: d8 and the -32 * (sum of codes) of each 16-element half, computed once per call */
typedef struct {
    float d8;
    int32_t off0, off1;
} XBlk;

static void x_blocks(const uint8_t* xq, int nblk, XBlk* out) {
    for (int j = 0; j < nblk; ++j) {
        const uint8_t* b = xq + (size_t) Q81 * j;
        uint16_t h;
        memcpy(&h, b, 2);
        int s0 = 0, s1 = 0;
        for (int l = 0; l < 16; ++l) s0 += (int8_t) b[4 + l];
        for (int l = 16; l < 32; ++l) s1 += (int8_t) b[4 + l];
        out[j].d8 = f16_to_f32(h);
        out[j].off0 = -32 * s0;
        out[j].off1 = -32 * s1;
    }
}

/* one row of one column, AVX2: returns sum over Q6_K blocks of d * sum_j d8_j * (sc0 (dot0 - 32 s0) + sc1 (...)) */
static float row_avx2(const uint8_t* w, const uint8_t* xq, const XBlk* xb, int nb) {
    __m256 acc = _mm256_setzero_ps();
    float accs = 0.0f;
    for (int bi = 0; bi < nb; ++bi) {
        const uint8_t* b = w + (size_t) bi * Q6K;
        __m256i q[8];
        q6k_codes(b, q);
        const int8_t* sc = (const int8_t*) (b + 192);
        uint16_t dh;
        memcpy(&dh, b + 208, 2);
        const float d = f16_to_f32(dh);
        __m256 blk = _mm256_setzero_ps();
        float blks = 0.0f;
        for (int g = 0; g < 8; ++g) {
            const int j = 8 * bi + g;
            const __m256i x8 = _mm256_loadu_si256((const __m256i*) (xq + (size_t) Q81 * j + 4));
            const __m256i p16 = _mm256_maddubs_epi16(q[g], x8);   /* pairs: |.| <= 2 * 63 * 127 */
            const __m256i s16 = _mm256_set_m128i(_mm_set1_epi16(sc[2 * g + 1]), _mm_set1_epi16(sc[2 * g]));
            const __m256i p32 = _mm256_madd_epi16(p16, s16);
            blk = _mm256_fmadd_ps(_mm256_set1_ps(xb[j].d8), _mm256_cvtepi32_ps(p32), blk);
            blks += xb[j].d8 * (float) (sc[2 * g] * xb[j].off0 + sc[2 * g + 1] * xb[j].off1);
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), blk, acc);
        accs += d * blks;
    }
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    s = _mm_hadd_ps(s, s);
    s = _mm_hadd_ps(s, s);
    return _mm_cvtss_f32(s) + accs;
}

/* the same on AVX-512 VNNI: two Q8_1 blocks per vpdpbusd (64 codes), sub-scales multiplied in int32 lanes */
__attribute__((target("avx512f,avx512bw,avx512vnni"))) static float row_vnni(const uint8_t* w, const uint8_t* xq,
                                                                               const XBlk* xb, int nb) {
    __m512 acc = _mm512_setzero_ps();
    float accs = 0.0f;
    for (int bi = 0; bi < nb; ++bi) {
        const uint8_t* b = w + (size_t) bi * Q6K;
        __m256i q[8];
        q6k_codes(b, q);
        const int8_t* sc = (const int8_t*) (b + 192);
        uint16_t dh;
        memcpy(&dh, b + 208, 2);
        const float d = f16_to_f32(dh);
        __m512 blk = _mm512_setzero_ps();
        float blks = 0.0f;
        for (int g = 0; g < 8; g += 2) {
            const int j = 8 * bi + g;
            const __m512i qq = _mm512_inserti64x4(_mm512_castsi256_si512(q[g]), q[g + 1], 1);
            const __m256i xa = _mm256_loadu_si256((const __m256i*) (xq + (size_t) Q81 * j + 4));
            const __m256i xc = _mm256_loadu_si256((const __m256i*) (xq + (size_t) Q81 * (j + 1) + 4));
            const __m512i x8 = _mm512_inserti64x4(_mm512_castsi256_si512(xa), xc, 1);
            const __m512i dp = _mm512_dpbusd_epi32(_mm512_setzero_si512(), qq, x8);   /* sums of 4 codes */
            const __m512i sv = _mm512_setr_epi32(sc[2 * g], sc[2 * g], sc[2 * g], sc[2 * g], sc[2 * g + 1],
                                                 sc[2 * g + 1], sc[2 * g + 1], sc[2 * g + 1], sc[2 * g + 2],
                                                 sc[2 * g + 2], sc[2 * g + 2], sc[2 * g + 2], sc[2 * g + 3],
                                                 sc[2 * g + 3], sc[2 * g + 3], sc[2 * g + 3]);
            const __m512 dv = _mm512_setr_ps(xb[j].d8, xb[j].d8, xb[j].d8, xb[j].d8, xb[j].d8, xb[j].d8, xb[j].d8,
                                             xb[j].d8, xb[j + 1].d8, xb[j + 1].d8, xb[j + 1].d8, xb[j + 1].d8,
                                             xb[j + 1].d8, xb[j + 1].d8, xb[j + 1].d8, xb[j + 1].d8);
            blk = _mm512_fmadd_ps(dv, _mm512_cvtepi32_ps(_mm512_mullo_epi32(dp, sv)), blk);
            blks += xb[j].d8 * (float) (sc[2 * g] * xb[j].off0 + sc[2 * g + 1] * xb[j].off1) +
                    xb[j + 1].d8 * (float) (sc[2 * g + 2] * xb[j + 1].off0 + sc[2 * g + 3] * xb[j + 1].off1);
        }
        acc = _mm512_fmadd_ps(_mm512_set1_ps(d), blk, acc);
        accs += d * blks;
    }
    return _mm512_reduce_add_ps(acc) + accs;
}

int cpr_simd_level(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512bw") ? 2 : 1;
}

/* y[c][r] = W x_c (+ res); partials[c][g] = sum of squares of rows 4g..4g+3 of y (when res and partials) */
void cpr_q6k_gemv(const uint8_t* w, const uint8_t* xq, const float* res, float* y, float* partials, int n_in,
                  int n_out, int ncols, int threads, int simd) {
    const int nb = n_in / 256, nblk = n_in / 32;
    XBlk* xb = (XBlk*) malloc(sizeof(XBlk) * (size_t) nblk * ncols);
    for (int c = 0; c < ncols; ++c) x_blocks(xq + (size_t) c * nblk * Q81, nblk, xb + (size_t) c * nblk);
    const int vnni = simd >= 2 && cpr_simd_level() >= 2;
#pragma omp parallel for schedule(static, 16) num_threads(threads)
    for (int r = 0; r < n_out; ++r) {
        const uint8_t* wr = w + (size_t) r * nb * Q6K;
        for (int c = 0; c < ncols; ++c) {
            const uint8_t* xc = xq + (size_t) c * nblk * Q81;
            float v = vnni ? row_vnni(wr, xc, xb + (size_t) c * nblk, nb) : row_avx2(wr, xc, xb + (size_t) c * nblk, nb);
            if (res) v += res[(size_t) c * n_out + r];
            y[(size_t) c * n_out + r] = v;
        }
    }
    free(xb);
    if (res && partials) {
        const int np = (n_out + 3) / 4;
        for (int c = 0; c < ncols; ++c)
            for (int g = 0; g < np; ++g) {
                float p = 0.0f;
                for (int r = 4 * g; r < 4 * g + 4 && r < n_out; ++r) p += y[(size_t) c * n_out + r] * y[(size_t) c * n_out + r];
                partials[(size_t) c * np + g] = p;
            }
    }
}

/* ---- Gated DeltaNet layer, ntok tokens ----------------------------------------------------------------------------- */
static float silu_f(float v) { return v / (1.0f + expf(-v)); }

/* qkvz: token t at + t * stride = [q h_k*128 | k h_k*128 | v h_v*128 | z h_v*128]; ab: token t at + t * 2 h_v =
 * [beta | alpha]; hist [channels][3] and state [128][h_v][128] updated in place; y token t at + t * h_v * 128 */
void cpr_gdn_layer(const float* qkvz, int stride, const float* ab, const float* conv_w, const float* dt,
                   const float* ssm_a, const float* gamma, float eps, float* hist, float* state, float* y, int h_k,
                   int h_v, int ntok, int threads) {
    const int S = 128, ch = (2 * h_k + h_v) * S;
    float* h = (float*) malloc(sizeof(float) * (size_t) ch * ntok);
    for (int t = 0; t < ntok; ++t) {
        const float* x = qkvz + (size_t) t * stride;
        float* ht = h + (size_t) t * ch;
#pragma omp parallel for schedule(static) num_threads(threads)
        for (int c = 0; c < ch; ++c) {
            const float s = hist[3 * c] * conv_w[4 * c] + hist[3 * c + 1] * conv_w[4 * c + 1] +
                            hist[3 * c + 2] * conv_w[4 * c + 2] + x[c] * conv_w[4 * c + 3];
            hist[3 * c] = hist[3 * c + 1];
            hist[3 * c + 1] = hist[3 * c + 2];
            hist[3 * c + 2] = x[c];
            ht[c] = silu_f(s);
        }
        for (int hd = 0; hd < 2 * h_k; ++hd) {
            float ss = 0.0f;
            for (int i = 0; i < S; ++i) ss += ht[hd * S + i] * ht[hd * S + i];
            const float inv = 1.0f / sqrtf(ss + eps);
            for (int i = 0; i < S; ++i) ht[hd * S + i] *= inv;
        }
    }
#pragma omp parallel for schedule(static) num_threads(threads)
    for (int hd = 0; hd < h_v; ++hd) {
        const int qh = hd % h_k;
        float kv[128], o[128], delta[128];
        for (int t = 0; t < ntok; ++t) {
            const float* ht = h + (size_t) t * ch;
            const float* q = ht + qh * S;
            const float* k = ht + (h_k + qh) * S;
            const float* v = ht + 2 * h_k * S + hd * S;
            const float* z = qkvz + (size_t) t * stride + ch + hd * S;
            const float b = 1.0f / (1.0f + expf(-ab[(size_t) t * 2 * h_v + hd]));
            const float av = ab[(size_t) t * 2 * h_v + h_v + hd] + dt[hd];
            const float g = expf((av > 20.0f ? av : log1pf(expf(av))) * ssm_a[hd]);
            for (int j = 0; j < S; ++j) kv[j] = 0.0f;
            for (int i = 0; i < S; ++i) {
                const float* srow = state + ((size_t) i * h_v + hd) * S;
                for (int j = 0; j < S; ++j) kv[j] += srow[j] * k[i];
            }
            for (int j = 0; j < S; ++j) delta[j] = (v[j] - g * kv[j]) * b;
            for (int j = 0; j < S; ++j) o[j] = 0.0f;
            for (int i = 0; i < S; ++i) {
                float* srow = state + ((size_t) i * h_v + hd) * S;
                for (int j = 0; j < S; ++j) {
                    srow[j] = g * srow[j] + k[i] * delta[j];
                    o[j] += srow[j] * q[i];
                }
            }
            float ss = 0.0f;
            for (int j = 0; j < S; ++j) {
                o[j] *= 0.08838834764831845f;
                ss += o[j] * o[j];
            }
            const float sc = 1.0f / sqrtf(ss / (float) S + eps);
            for (int j = 0; j < S; ++j) y[(size_t) t * h_v * S + hd * S + j] = o[j] * sc * gamma[j] * silu_f(z[j]);
        }
    }
    free(h);
}

/* ---- GQA decode over an fp16 cache [pos][n_kv][hd] ---------------------------------------------------------------- */
/* token t (position pos0 + t) of head h: q at q + (t * n_head + h) * hd, output likewise; each task is (kv head,
 * chunk of 256 positions) for every query of that kv head, keeping an online softmax per query, merged in chunk
 * order at the end */
void cpr_gqa_decode(const float* q, const uint16_t* kc, const uint16_t* vc, float* o, int n_head, int n_kv, int hd,
                    int pos0, int ntok, float scale, int threads) {
    enum { CH = 256, MAXQ = 64 };
    const int G = n_head / n_kv, nq = G * ntok, last = pos0 + ntok - 1;
    const int nchunk = last / CH + 1;
    float* rec = (float*) malloc(sizeof(float) * (size_t) nchunk * n_kv * nq * (hd + 2));
#pragma omp parallel for collapse(2) schedule(dynamic) num_threads(threads)
    for (int kv = 0; kv < n_kv; ++kv)
        for (int ck = 0; ck < nchunk; ++ck) {
            float m[MAXQ], l[MAXQ];
            float* acc = rec + ((size_t) ck * n_kv + kv) * nq * (hd + 2);
            for (int i = 0; i < nq; ++i) {
                m[i] = -INFINITY;
                l[i] = 0.0f;
                memset(acc + (size_t) i * (hd + 2) + 2, 0, sizeof(float) * hd);
            }
            float kr[1024], vr[1024];
            for (int p = ck * CH; p < (ck + 1) * CH && p <= last; ++p) {
                const uint16_t* kp = kc + ((size_t) p * n_kv + kv) * hd;
                const uint16_t* vp = vc + ((size_t) p * n_kv + kv) * hd;
                for (int d = 0; d < hd; d += 8) {
                    _mm256_storeu_ps(kr + d, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*) (kp + d))));
                    _mm256_storeu_ps(vr + d, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*) (vp + d))));
                }
                for (int i = 0; i < nq; ++i) {
                    const int t = i / G, h = kv * G + i % G;
                    if (p > pos0 + t) continue;
                    const float* qi = q + ((size_t) t * n_head + h) * hd;
                    __m256 sv = _mm256_setzero_ps();
                    for (int d = 0; d < hd; d += 8)
                        sv = _mm256_fmadd_ps(_mm256_loadu_ps(qi + d), _mm256_loadu_ps(kr + d), sv);
                    __m128 s4 = _mm_add_ps(_mm256_castps256_ps128(sv), _mm256_extractf128_ps(sv, 1));
                    s4 = _mm_hadd_ps(s4, s4);
                    s4 = _mm_hadd_ps(s4, s4);
                    const float s = _mm_cvtss_f32(s4) * scale;
                    float* a = acc + (size_t) i * (hd + 2) + 2;
                    if (s > m[i]) {
                        const float r = expf(m[i] - s);
                        l[i] *= r;
                        for (int d = 0; d < hd; ++d) a[d] *= r;
                        m[i] = s;
                    }
                    const float e = expf(s - m[i]);
                    l[i] += e;
                    for (int d = 0; d < hd; ++d) a[d] += e * vr[d];
                }
            }
            for (int i = 0; i < nq; ++i) {
                acc[(size_t) i * (hd + 2)] = m[i];
                acc[(size_t) i * (hd + 2) + 1] = l[i];
            }
        }
    for (int kv = 0; kv < n_kv; ++kv)
        for (int i = 0; i < nq; ++i) {
            const int t = i / G, h = kv * G + i % G;
            const int nc = (pos0 + t) / CH + 1;
            float M = -INFINITY;
            for (int ck = 0; ck < nc; ++ck) {
                const float mm = rec[(((size_t) ck * n_kv + kv) * nq + i) * (hd + 2)];
                if (mm > M) M = mm;
            }
            float L = 0.0f;
            float* out = o + ((size_t) t * n_head + h) * hd;
            for (int d = 0; d < hd; ++d) out[d] = 0.0f;
            for (int ck = 0; ck < nc; ++ck) {
                const float* r = rec + (((size_t) ck * n_kv + kv) * nq + i) * (hd + 2);
                const float wgt = expf(r[0] - M);
                L += r[1] * wgt;
                for (int d = 0; d < hd; ++d) out[d] += wgt * r[2 + d];
            }
            for (int d = 0; d < hd; ++d) out[d] /= L;
        }
    free(rec);
}
