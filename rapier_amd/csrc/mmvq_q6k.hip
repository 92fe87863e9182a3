// mmvq_q6k.hip - Q6_K x Q8_1 GEMV for gfx950 at ncols 1..16, with the fused residual + sum-of-squares epilogue.
//
// Reference behaviour: src/native_mmvq.cu native_q6_k_mmvq (3627-3660), native_mmvq_multi_kernel (1261-1356),
// native_q6_k_mmvq_res_kernel (3096-3140), integer core q6_q8_dot_impl (642-655).
//
// Design (memory-bound GEMV, no MFMA):
//  * A workgroup of 256 lanes (4 wave64) owns R output rows.  It walks the rows' bytes in chunks of CB Q6_K blocks
//    (R * CB = 128, so a chunk is always 26880 bytes), loading each chunk with 16-byte fully coalesced loads into
//    registers one chunk ahead and parking it in LDS.  Rows are 16-byte aligned because n_in % (256 * CB) == 0.
//  * Q8_1 activation blocks are staged in LDS, re-laid as 32 code bytes plus a record {-32 * sum(q8) per 16
//    elements, d8}, so the "code - 32" of Q6_K is folded into the dot's accumulator.  Rows of at most 4096 elements
//    are staged whole, once per workgroup, while the first weight chunks are in flight; longer rows chunk by chunk.
//  * Lane (row, half-block) decodes 128 weights once (aligned LDS dwords + v_alignbyte for the odd blocks' 2-byte
//    offset) and applies them to every column with v_dot4_i32_i8: an exact int32 per 16 elements, then
//    acc = fma(d8, float(sc0 * dot0 + sc1 * dot1), acc) per Q8_1 block and tot = fma(d, acc, tot) per half-block.
//  * A row's lanes are reduced by a fixed xor butterfly.  The lane <-> half-block ownership and the reduction tree
//    depend only on (n_in, n_out), never on ncols, so every column of an ncols >= 2 call is bitwise the ncols = 1
//    result, and the residual variant is bitwise plain + res.
#include "rmi_common.h"

#include <algorithm>
#include <cstdlib>

namespace rmi {
namespace {

constexpr int kThreads = 256;
constexpr int kTileBytes = 128 * kQ6KBytes;          // R * CB * 210 = 26880
constexpr int kTileVec = kTileBytes / 16;             // 1680 16-byte loads per chunk
constexpr int kLoadsPerThread = (kTileVec + kThreads - 1) / kThreads;   // 7

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// ---- shared decode: 128 weights of one half-block (n = 0/1) from realigned dwords --------------------------------
// ql[16] = ql bytes [64n, 64n+64), qh[8] = qh bytes [32n, 32n+32), sc[2] = sub-scales [8n, 8n+8).
// Element l (0..31) of sub-block k (0..3): low nibble of ql[32(k&1) + l] (high when k >= 2) | qh bits 2k..2k+1.
__device__ __forceinline__ int q6_codes4(const uint32_t (&ql)[16], const uint32_t (&qh)[8], int k, int w) {
    const uint32_t lo = (ql[(k & 1) * 8 + w] >> ((k >> 1) * 4)) & 0x0f0f0f0fu;
    const uint32_t hi = ((qh[w] >> (2 * k)) & 0x03030303u) << 4;
    return static_cast<int>(lo | hi);
}

__device__ __forceinline__ int sc_byte(const uint32_t (&sc)[2], int i) {
    return static_cast<int>(static_cast<int8_t>((sc[i >> 2] >> (8 * (i & 3))) & 0xffu));
}

// exact integer of sub-block k against one Q8_1 block: sc_lo * sum(q6 - 32)q8 [0,16) + sc_hi * ... [16,32)
__device__ __forceinline__ int q6_subblock_dot(const int (&v)[8], const int (&u)[8], int corr0, int corr1, int sc0,
                                               int sc1) {
    int d0 = corr0, d1 = corr1;
#pragma unroll
    for (int w = 0; w < 4; ++w) d0 = sdot4(v[w], u[w], d0);
#pragma unroll
    for (int w = 4; w < 8; ++w) d1 = sdot4(v[w], u[w], d1);
    // |sc| <= 32 and |d| <= 16 * 32 * 127: both fit 24 bits, so the full-rate 24-bit multiplies are exact
    return __mul24(sc0, d0) + __mul24(sc1, d1);
}

// 4-byte little-endian word from a 2-byte aligned global address (two u16 loads)
__device__ __forceinline__ uint32_t ldg_u32_b2(const uint8_t* p) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
    return static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16);
}

// ---- activation staging: Q8_1 block -> {32 code bytes (two 16-B units), record {corr0, corr1, d8 bits, 0}} ----------
// 16-B units are xor-swizzled inside aligned groups of 8 so the 16 lanes of a row (which read blocks 4m + k) hit
// distinct bank groups.
__device__ __forceinline__ int swz(int u) { return u ^ ((u >> 3) & 7); }

struct XRegs {
    uint32_t w[9];
};

__device__ __forceinline__ void load_x_block(const uint8_t* __restrict__ xb, XRegs& r) {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(xb);
#pragma unroll
    for (int i = 0; i < 9; ++i) r.w[i] = p[i];   // re-read by every workgroup: keep it cached
}

// block j of a chunk slice: codes at lq[swz(2j)], lq[swz(2j + 1)], record at lrec[swz(j)]
__device__ __forceinline__ void stage_codes(const uint32_t (&cw)[8], uint32_t d_bits, int j, uint4* lq, uint4* lrec) {
    int s0 = 0, s1 = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) s0 = sdot4(static_cast<int>(cw[i]), 0x01010101, s0);
#pragma unroll
    for (int i = 4; i < 8; ++i) s1 = sdot4(static_cast<int>(cw[i]), 0x01010101, s1);
    const float d8 = half_bits_to_float(d_bits);
    lq[swz(2 * j)] = make_uint4(cw[0], cw[1], cw[2], cw[3]);
    lq[swz(2 * j + 1)] = make_uint4(cw[4], cw[5], cw[6], cw[7]);
    lrec[swz(j)] = make_uint4(static_cast<uint32_t>(-32 * s0), static_cast<uint32_t>(-32 * s1), __float_as_uint(d8), 0u);
}

__device__ __forceinline__ void stage_x_block(const XRegs& r, int j, uint4* lq, uint4* lrec) {
    const uint32_t cw[8] = {r.w[1], r.w[2], r.w[3], r.w[4], r.w[5], r.w[6], r.w[7], r.w[8]};
    stage_codes(cw, r.w[0], j, lq, lrec);
}

// Activation staging.  XM 0: a chunk's Q8_1 blocks are loaded one step ahead with the weights and staged per step;
// XM 1: the whole row (n_in <= kFullMaxIn) is staged once per workgroup, in the same per-chunk layout, while the
// first weight chunks are in flight.  Same staged values either way.
constexpr int kFullMaxIn = 4096;

// ---- the tiled kernel ------------------------------------------------------------------------------------------------
// Persistent: workgroup g owns row tiles g, g + G, g + 2G, ... and walks the flat sequence of (tile, chunk) steps with
// DEPTH chunks of loads in flight in registers, across tile boundaries, so a workgroup never idles on a fresh tile's
// first load.  Each step: park the oldest chunk in LDS, refill its registers with the chunk DEPTH steps ahead, decode.
template <int R, int NCOLS, bool RES, int DEPTH, int XM>
__global__ __launch_bounds__(kThreads) void q6k_gemv_tiled(const uint8_t* __restrict__ w,
                                                           const uint8_t* __restrict__ x, float* y,
                                                           const float* res, float* partials, int n_in, int n_out) {
    constexpr int CB = 128 / R;            // Q6_K blocks per row per chunk
    constexpr int TPR = kThreads / R;      // lanes per row = half-blocks per row per chunk
    constexpr int NB = CB * 8;             // Q8_1 blocks per chunk per column
    constexpr int U = CB * kQ6KBytes / 16; // 16-byte units per row per chunk
    // LDS dwords per tile row: 16-byte aligned (the staging stores are 128-bit) and padded so that the decode's
    // dword reads of the wave's rows spread over the banks (at most 2-way; checked exhaustively for both tiles)
    constexpr int ROWW = CB * kQ6KBytes / 4 + (R == 16 ? 4 : 12);
    constexpr int XS = XM == 0 ? NCOLS * NB : 0;   // activation blocks to stage per chunk
    constexpr int XP = XS ? (XS + kThreads - 1) / kThreads : 1;
    constexpr int XBLK = XM == 0 ? NB : kFullMaxIn / 32;   // staged blocks per column

    __shared__ __attribute__((aligned(16))) uint32_t lw[R * ROWW];
    __shared__ uint4 lq[NCOLS * 2 * XBLK];
    __shared__ uint4 lrec[NCOLS * XBLK];
    __shared__ float vout[NCOLS][R];

    const int t = threadIdx.x;
    const uint32_t rowbytes = static_cast<uint32_t>(n_in / 256) * kQ6KBytes;
    const int nch = n_in / (256 * CB);
    const int ntiles = (n_out + R - 1) / R;
    const int G = gridDim.x;
    const int my_tiles = (ntiles - static_cast<int>(blockIdx.x) + G - 1) / G;
    const int nsteps = my_tiles * nch;
    const int xcol_blocks = n_in / 32;
    const int xcs = XM == 0 ? NB : nch * NB;   // staged blocks between columns

    u32x4 wreg[DEPTH][kLoadsPerThread];
    XRegs xreg[DEPTH][XP];

    // per-thread load / store slots, fixed for every step: 16-byte unit i = t + 256 m is tile row i / U, unit i % U
    uint32_t goff[kLoadsPerThread];   // byte offset from the chunk's first row (UINT32_MAX: slot unused)
    uint32_t lrow[kLoadsPerThread];   // tile row of the slot
#pragma unroll
    for (int m = 0; m < kLoadsPerThread; ++m) {
        const int i = t + kThreads * m;
        const int tr = i / U, u = i - tr * U;
        lrow[m] = static_cast<uint32_t>(tr);
        goff[m] = i < kTileVec ? static_cast<uint32_t>(tr) * rowbytes + static_cast<uint32_t>(u * 16) : 0xffffffffu;
    }

    // step f -> (tile, chunk)
    auto issue = [&](int f, u32x4 (&wr)[kLoadsPerThread], XRegs (&xr)[XP]) {
        const int q = f / nch;
        const int c = f - q * nch;
        const int row0 = (static_cast<int>(blockIdx.x) + q * G) * R;
        const uint8_t* base = w + static_cast<size_t>(row0) * rowbytes + static_cast<size_t>(c) * (CB * kQ6KBytes);
        const uint32_t rows_left = static_cast<uint32_t>(n_out - row0);
#pragma unroll
        for (int m = 0; m < kLoadsPerThread; ++m)
            if (goff[m] != 0xffffffffu && lrow[m] < rows_left)
                wr[m] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + goff[m]));
#pragma unroll
        for (int p = 0; p < XP; ++p) {
            const int sidx = t + kThreads * p;
            if (sidx < XS) {
                const int col = sidx / NB, jb = sidx - col * NB;
                load_x_block(x + (static_cast<size_t>(col) * xcol_blocks + static_cast<size_t>(c) * NB + jb) *
                                     kQ8_1Bytes,
                             xr[p]);
            }
        }
    };

    // lane ownership: row ri, half-block hb of the chunk (block b, half n)
    const int ri = t / TPR, hb = t - ri * TPR;
    const int b = hb >> 1, n = hb & 1;
    const int wbase = ri * (ROWW * 4) + b * kQ6KBytes;   // byte offset of the lane's block in the LDS tile
    const int mis = wbase & 3;                           // 0 or 2 (odd blocks of a 210-byte stride)
    const int wd = wbase >> 2;

    float tot[NCOLS];
#pragma unroll
    for (int c = 0; c < NCOLS; ++c) tot[c] = 0.0f;

#pragma unroll
    for (int s = 0; s < DEPTH; ++s)
        if (s < nsteps) issue(s, wreg[s], xreg[s]);

    // whole-row activations, staged once while the first weight chunks are in flight (published by the first
    // step's barrier).  Chunk c of column col occupies blocks [col * xcs + c * NB, + NB) in the per-chunk layout.
    if constexpr (XM == 1) {
        for (int J = t; J < NCOLS * xcol_blocks; J += kThreads) {
            const int col = J / xcol_blocks, jb = J - col * xcol_blocks;
            const int c = jb / NB, j = jb - c * NB;
            XRegs r;
            load_x_block(x + static_cast<size_t>(J) * kQ8_1Bytes, r);
            stage_x_block(r, j, lq + 2 * (col * xcs + c * NB), lrec + col * xcs + c * NB);
        }
    }

    for (int f0 = 0; f0 < nsteps; f0 += DEPTH) {
#pragma unroll
        for (int s = 0; s < DEPTH; ++s) {
            const int f = f0 + s;
            if (f >= nsteps) break;   // uniform across the workgroup
            const int q = f / nch;
            const int c = f - q * nch;
            if (f > 0) __syncthreads();
#pragma unroll
            for (int m = 0; m < kLoadsPerThread; ++m) {
                const int i = t + kThreads * m;
                const int tr = i / U, u = i - tr * U;   // compile-time U: a multiply-shift, hoisted by the compiler
                if (i < kTileVec) *reinterpret_cast<u32x4*>(&lw[tr * ROWW + u * 4]) = wreg[s][m];
            }
#pragma unroll
            for (int p = 0; p < XP; ++p) {
                const int sidx = t + kThreads * p;
                if (sidx < XS) {
                    const int col = sidx / NB, jb = sidx - col * NB;
                    stage_x_block(xreg[s][p], jb, lq + 2 * col * NB, lrec + col * NB);
                }
            }
            const uint4* lqc = lq + (XM == 0 ? 0 : 2 * c * NB);   // this chunk's slice of every column
            const uint4* lrc = lrec + (XM == 0 ? 0 : c * NB);
            __syncthreads();
            if (f + DEPTH < nsteps) issue(f + DEPTH, wreg[s], xreg[s]);

            // decode the lane's half-block: qh and the scales once, ql per nibble pair (sub-blocks k, k + 2)
            uint32_t qh[8], sc[2];
            {
                uint32_t th[9];
#pragma unroll
                for (int i = 0; i < 9; ++i) th[i] = lw[wd + 32 + 8 * n + i];
#pragma unroll
                for (int i = 0; i < 8; ++i) qh[i] = __builtin_amdgcn_alignbyte(th[i + 1], th[i], mis);
                const uint32_t s0 = lw[wd + 48 + 2 * n], s1 = lw[wd + 49 + 2 * n], s2 = lw[wd + 50 + 2 * n];
                sc[0] = __builtin_amdgcn_alignbyte(s1, s0, mis);
                sc[1] = __builtin_amdgcn_alignbyte(s2, s1, mis);
            }
            const float d = half_bits_to_float(lw[wd + 52] >> (8 * mis));
            float acc[NCOLS];
#pragma unroll
            for (int col = 0; col < NCOLS; ++col) acc[col] = 0.0f;
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                uint32_t ql8[8];
                {
                    uint32_t tq[9];
#pragma unroll
                    for (int i = 0; i < 9; ++i) tq[i] = lw[wd + 16 * n + 8 * kk + i];
#pragma unroll
                    for (int i = 0; i < 8; ++i) ql8[i] = __builtin_amdgcn_alignbyte(tq[i + 1], tq[i], mis);
                }
#pragma unroll
                for (int kh = 0; kh < 2; ++kh) {
                    const int k = kk + 2 * kh;
                    int v[8];
#pragma unroll
                    for (int ww = 0; ww < 8; ++ww)
                        v[ww] = static_cast<int>(((ql8[ww] >> (4 * kh)) & 0x0f0f0f0fu) |
                                                 (((qh[ww] >> (2 * k)) & 0x03030303u) << 4));
                    const int sc0 = sc_byte(sc, 2 * k), sc1 = sc_byte(sc, 2 * k + 1);
                    const int j = 8 * b + 4 * n + k;
#pragma unroll
                    for (int col = 0; col < NCOLS; ++col) {
                        const uint4 qa = lqc[2 * col * xcs + swz(2 * j)];
                        const uint4 qb = lqc[2 * col * xcs + swz(2 * j + 1)];
                        const uint4 rec = lrc[col * xcs + swz(j)];
                        const int u[8] = {static_cast<int>(qa.x), static_cast<int>(qa.y), static_cast<int>(qa.z),
                                          static_cast<int>(qa.w), static_cast<int>(qb.x), static_cast<int>(qb.y),
                                          static_cast<int>(qb.z), static_cast<int>(qb.w)};
                        const int sdot = q6_subblock_dot(v, u, static_cast<int>(rec.x), static_cast<int>(rec.y), sc0, sc1);
                        acc[col] = __builtin_fmaf(__uint_as_float(rec.z), static_cast<float>(sdot), acc[col]);
                    }
                }
            }
#pragma unroll
            for (int col = 0; col < NCOLS; ++col) tot[col] = __builtin_fmaf(d, acc[col], tot[col]);

            if (c == nch - 1) {
                // the tile's rows are complete: reduce each row's TPR lanes, then the epilogue
                const int row0 = (static_cast<int>(blockIdx.x) + q * G) * R;
#pragma unroll
                for (int col = 0; col < NCOLS; ++col) {
                    const float sum = group_sum<TPR>(tot[col]);
                    if (hb == 0) vout[col][ri] = sum;
                    tot[col] = 0.0f;
                }
                __syncthreads();
                if (t < NCOLS * R) {
                    const int col = t / R, r = t - col * R;
                    const int row = row0 + r;
                    if (row < n_out) {
                        float v = vout[col][r];
                        if constexpr (RES) v += res[static_cast<size_t>(col) * n_out + row];
                        y[static_cast<size_t>(col) * n_out + row] = v;
                        if constexpr (RES) vout[col][r] = v;
                    }
                }
                if constexpr (RES) {
                    __syncthreads();
                    constexpr int GR = R / 4;
                    if (t < NCOLS * GR) {
                        const int col = t / GR, g = t - col * GR;
                        const int np = (n_out + 3) / 4;
                        const int grow = row0 / 4 + g;
                        if (grow < np) {
                            float p = 0.0f;
#pragma unroll
                            for (int i = 0; i < 4; ++i)
                                if (row0 + 4 * g + i < n_out)
                                    p = __builtin_fmaf(vout[col][4 * g + i], vout[col][4 * g + i], p);
                            partials[static_cast<size_t>(col) * np + grow] = p;
                        }
                    }
                }
            }
        }
    }
}

// ---- generic kernel: any n_in % 256 == 0, any 2-byte aligned weight pointer --------------------------------------------
// One wave per row (4 rows per workgroup); lane l owns half-blocks l, l+64, ...; decode straight from global memory.
template <int NCOLS, bool RES>
__global__ __launch_bounds__(kThreads) void q6k_gemv_generic(const uint8_t* __restrict__ w,
                                                             const uint8_t* __restrict__ x, float* y,
                                                             const float* res, float* partials, int n_in, int n_out) {
    __shared__ float vout[NCOLS][4];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int row = blockIdx.x * 4 + wv;
    const int nb = n_in / 256;
    const int xcol_blocks = n_in / 32;
    float tot[NCOLS];
#pragma unroll
    for (int c = 0; c < NCOLS; ++c) tot[c] = 0.0f;
    if (row < n_out) {
        for (int hbi = lane; hbi < 2 * nb; hbi += 64) {
            const int bi = hbi >> 1, n = hbi & 1;
            const uint8_t* blk = w + (static_cast<size_t>(row) * nb + bi) * kQ6KBytes;
            uint32_t ql[16], qh[8], sc[2];
#pragma unroll
            for (int i = 0; i < 16; ++i) ql[i] = ldg_u32_b2(blk + 64 * n + 4 * i);
#pragma unroll
            for (int i = 0; i < 8; ++i) qh[i] = ldg_u32_b2(blk + 128 + 32 * n + 4 * i);
            sc[0] = ldg_u32_b2(blk + 192 + 8 * n);
            sc[1] = ldg_u32_b2(blk + 196 + 8 * n);
            const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(blk + 208));
            float acc[NCOLS];
#pragma unroll
            for (int col = 0; col < NCOLS; ++col) acc[col] = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                int v[8];
#pragma unroll
                for (int ww = 0; ww < 8; ++ww) v[ww] = q6_codes4(ql, qh, k, ww);
                const int sc0 = sc_byte(sc, 2 * k), sc1 = sc_byte(sc, 2 * k + 1);
                const int j = 8 * bi + 4 * n + k;
#pragma unroll
                for (int col = 0; col < NCOLS; ++col) {
                    const uint32_t* xb = reinterpret_cast<const uint32_t*>(
                        x + (static_cast<size_t>(col) * xcol_blocks + j) * kQ8_1Bytes);
                    int u[8];
                    int s0 = 0, s1 = 0;
#pragma unroll
                    for (int i = 0; i < 8; ++i) u[i] = static_cast<int>(xb[1 + i]);
#pragma unroll
                    for (int i = 0; i < 4; ++i) s0 = sdot4(u[i], 0x01010101, s0);
#pragma unroll
                    for (int i = 4; i < 8; ++i) s1 = sdot4(u[i], 0x01010101, s1);
                    const int s = q6_subblock_dot(v, u, -32 * s0, -32 * s1, sc0, sc1);
                    acc[col] = __builtin_fmaf(half_bits_to_float(xb[0]), static_cast<float>(s), acc[col]);
                }
            }
#pragma unroll
            for (int col = 0; col < NCOLS; ++col) tot[col] = __builtin_fmaf(d, acc[col], tot[col]);
        }
    }
#pragma unroll
    for (int col = 0; col < NCOLS; ++col) {
        float s = group_sum<64>(tot[col]);
        if (row < n_out) {
            if constexpr (RES) s += res[static_cast<size_t>(col) * n_out + row];
            if (lane == 0) {
                y[static_cast<size_t>(col) * n_out + row] = s;
                vout[col][wv] = s;
            }
        }
    }
    if constexpr (RES) {
        __syncthreads();
        if (threadIdx.x < NCOLS) {
            const int col = threadIdx.x;
            float p = 0.0f;
            for (int i = 0; i < 4; ++i)
                if (blockIdx.x * 4 + i < n_out) p = __builtin_fmaf(vout[col][i], vout[col][i], p);
            partials[static_cast<size_t>(col) * ((n_out + 3) / 4) + blockIdx.x] = p;
        }
    }
}

// ---- integer block dots: one lane per (row, half-block), same decode as the GEMVs -----------------------------------
__global__ __launch_bounds__(kThreads) void q6k_block_dots_kernel(const uint8_t* __restrict__ w,
                                                                  const uint8_t* __restrict__ x,
                                                                  int32_t* __restrict__ out, int n_in, int n_out) {
    const int nb = n_in / 256;
    const size_t gid = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (gid >= static_cast<size_t>(n_out) * 2 * nb) return;
    const int row = static_cast<int>(gid / (2 * nb));
    const int hbi = static_cast<int>(gid - static_cast<size_t>(row) * 2 * nb);
    const int bi = hbi >> 1, n = hbi & 1;
    const uint8_t* blk = w + (static_cast<size_t>(row) * nb + bi) * kQ6KBytes;
    uint32_t ql[16], qh[8], sc[2];
    for (int i = 0; i < 16; ++i) ql[i] = ldg_u32_b2(blk + 64 * n + 4 * i);
    for (int i = 0; i < 8; ++i) qh[i] = ldg_u32_b2(blk + 128 + 32 * n + 4 * i);
    sc[0] = ldg_u32_b2(blk + 192 + 8 * n);
    sc[1] = ldg_u32_b2(blk + 196 + 8 * n);
    for (int k = 0; k < 4; ++k) {
        int v[8], u[8];
        for (int ww = 0; ww < 8; ++ww) v[ww] = q6_codes4(ql, qh, k, ww);
        const int j = 8 * bi + 4 * n + k;
        const uint32_t* xb = reinterpret_cast<const uint32_t*>(x + static_cast<size_t>(j) * kQ8_1Bytes);
        int s0 = 0, s1 = 0;
        for (int i = 0; i < 8; ++i) u[i] = static_cast<int>(xb[1 + i]);
        for (int i = 0; i < 4; ++i) s0 = sdot4(u[i], 0x01010101, s0);
        for (int i = 4; i < 8; ++i) s1 = sdot4(u[i], 0x01010101, s1);
        out[static_cast<size_t>(row) * (n_in / 32) + j] =
            q6_subblock_dot(v, u, -32 * s0, -32 * s1, sc_byte(sc, 2 * k), sc_byte(sc, 2 * k + 1));
    }
}

// ---- dispatch ----------------------------------------------------------------------------------------------------------
// Row tile: 16 rows x 8 blocks per chunk, or 8 rows x 16 blocks when that is the only way to reach enough
// workgroups.  The choice depends on the shape only (never on ncols).
int pick_rows(int n_in, int n_out, const void* w) {
    const bool a16 = (reinterpret_cast<uintptr_t>(w) & 15u) == 0;
    if (!a16 || n_in % 2048 != 0) return 0;
    // 8-row tiles (16 blocks per chunk) for long rows or too few 16-row tiles to fill the chip (measured on MI355X)
    if (n_in % 4096 == 0 && (n_in > 4096 || (n_out + 15) / 16 < 512)) return 8;
    return 16;
}

struct TileCfg {
    int rows;    // 16 or 8 (0: generic kernel)
    int depth;   // chunks of loads in flight per workgroup
    int per_cu;  // persistent workgroups per CU (0: one workgroup per tile)
};

int env_int(const char* name, int def) {
    const char* v = std::getenv(name);
    return v && *v ? std::atoi(v) : def;
}

int cu_count() {
    static int n = [] {
        int dev = 0, c = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            c = 256;
        return c > 0 ? c : 256;
    }();
    return n;
}

TileCfg pick_cfg(int n_in, int n_out, const void* w) {
    static const int depth = env_int("RMI_GEMV_DEPTH", 1);
    static const int per_cu = env_int("RMI_GEMV_PER_CU", 3);
    static const int force_rows = env_int("RMI_GEMV_ROWS", 0);
    TileCfg cfg{pick_rows(n_in, n_out, w), depth == 1 ? 1 : 2, per_cu};
    if (cfg.rows && (force_rows == 8 || force_rows == 16) && n_in % (256 * (128 / force_rows)) == 0)
        cfg.rows = force_rows;
    return cfg;
}

template <int R, int NCOLS, bool RES, int DEPTH, int XM>
void launch_tiled(const uint8_t* w, const uint8_t* x, float* y, const float* res, float* partials, int n_in, int n_out,
                  int per_cu, hipStream_t s) {
    const int ntiles = (n_out + R - 1) / R;
    int grid = ntiles;
    if (per_cu > 0) grid = std::min(ntiles, per_cu * cu_count());
    hipLaunchKernelGGL((q6k_gemv_tiled<R, NCOLS, RES, DEPTH, XM>), dim3(grid), dim3(kThreads), 0, s, w, x, y, res,
                       partials, n_in, n_out);
}

template <int R, int NCOLS, bool RES, int XM>
void launch_depth(const uint8_t* w, const uint8_t* x, float* y, const float* res, float* partials, int n_in, int n_out,
                  const TileCfg& cfg, hipStream_t s) {
    if (cfg.depth == 1) launch_tiled<R, NCOLS, RES, 1, XM>(w, x, y, res, partials, n_in, n_out, cfg.per_cu, s);
    else launch_tiled<R, NCOLS, RES, 2, XM>(w, x, y, res, partials, n_in, n_out, cfg.per_cu, s);
}

// whole-row staging for rows of at most kFullMaxIn elements (shape-only choice; the staged values are the same)
bool full_row(int n_in) {
    static const bool on = env_int("RMI_GEMV_XFULL", 1) != 0;
    return on && n_in <= kFullMaxIn;
}

template <int NCOLS, bool RES>
void launch_cols(const uint8_t* w, const uint8_t* x, float* y, const float* res, float* partials, int n_in, int n_out,
                 hipStream_t s) {
    // rows of 4096 / 8192 / 12288: the stream kernel (every column, including the passes of ncols > 4, bitwise its
    // one-column result and the packed kernels'); RMI_GGUF_STREAM=0 measures the tiled kernel instead
    static const bool stream_on = env_int("RMI_GGUF_STREAM", 1) != 0;
    if (NCOLS <= 4 && stream_on &&
        gguf_stream_gemv(w, x, y, RES ? res : nullptr, RES ? partials : nullptr, n_in, n_out, NCOLS, s) == RMI_OK)
        return;
    const TileCfg cfg = pick_cfg(n_in, n_out, w);
    const bool full = full_row(n_in);
    if (cfg.rows == 16) {
        if (full) launch_depth<16, NCOLS, RES, 1>(w, x, y, res, partials, n_in, n_out, cfg, s);
        else launch_depth<16, NCOLS, RES, 0>(w, x, y, res, partials, n_in, n_out, cfg, s);
    } else if (cfg.rows == 8) {
        if (full) launch_depth<8, NCOLS, RES, 1>(w, x, y, res, partials, n_in, n_out, cfg, s);
        else launch_depth<8, NCOLS, RES, 0>(w, x, y, res, partials, n_in, n_out, cfg, s);
    } else {
        hipLaunchKernelGGL((q6k_gemv_generic<NCOLS, RES>), dim3((n_out + 3) / 4), dim3(kThreads), 0, s, w, x, y, res,
                           partials, n_in, n_out);
    }
}

template <bool RES>
int launch(const void* wv, const void* xv, float* y, const float* res, float* partials, int n_in, int n_out,
           int ncols, hipStream_t s) {
    const auto* w = static_cast<const uint8_t*>(wv);
    const auto* x = static_cast<const uint8_t*>(xv);
    switch (ncols) {
        case 1: launch_cols<1, RES>(w, x, y, res, partials, n_in, n_out, s); break;
        case 2: launch_cols<2, RES>(w, x, y, res, partials, n_in, n_out, s); break;
        case 3: launch_cols<3, RES>(w, x, y, res, partials, n_in, n_out, s); break;
        case 4: launch_cols<4, RES>(w, x, y, res, partials, n_in, n_out, s); break;
        default: {   // 5..16: passes of at most 4 columns over the same weights (each column unchanged)
            const size_t xcol = static_cast<size_t>(n_in / 32) * kQ8_1Bytes;
            const size_t pcol = static_cast<size_t>((n_out + 3) / 4);
            for (int j = 0; j < ncols; j += 4) {
                const int nj = ncols - j < 4 ? ncols - j : 4;
                const int rc = launch<RES>(w, x + j * xcol, y + static_cast<size_t>(j) * n_out,
                                           RES ? res + static_cast<size_t>(j) * n_out : nullptr,
                                           RES ? partials + j * pcol : nullptr, n_in, n_out, nj, s);
                if (rc != RMI_OK) return rc;
            }
            return RMI_OK;
        }
    }
    return launch_status("native_q6_k_mmvq");
}

int validate(const void* w, const void* x, const float* y, int n_in, int n_out, int ncols, void* stream) {
    if (n_in <= 0 || n_in % 256 != 0)
        return fail(RMI_ERR_SHAPE, "native MMVQ requires n_in > 0 and divisible by its block element count");
    if (ncols < 1 || ncols > kMaxCols) return fail(RMI_ERR_SHAPE, "native MMVQ requires 1 <= ncols <= 16");
    if (n_out <= 0) return fail(RMI_ERR_SHAPE, "native MMVQ requires n_out > 0");
    if (!aligned4(w) || !aligned4(x) || !aligned4(y))
        return fail(RMI_ERR_POINTER, "native MMVQ requires non-null 4-byte aligned device pointers");
    if (!stream) return fail(RMI_ERR_STREAM, "native MMVQ requires an explicit non-null CUDA stream");
    return RMI_OK;
}

}  // namespace
}  // namespace rmi

using namespace rmi;

extern "C" int rmi_native_q6_k_mmvq(const void* w, const void* x_q8_1, float* y, int n_in, int n_out, int ncols,
                                    void* stream) {
    if (int rc = validate(w, x_q8_1, y, n_in, n_out, ncols, stream)) return rc;
    // a library-owned packed copy of these weights first, as the reference looks up its registry (mmvq:3629)
    if (const int rc = registry_mmvq(w, x_q8_1, y, nullptr, nullptr, n_in, n_out, ncols, stream); rc >= 0) return rc;
    return launch<false>(w, x_q8_1, y, nullptr, nullptr, n_in, n_out, ncols, static_cast<hipStream_t>(stream));
}

extern "C" int rmi_native_q6_k_mmvq_res_n(const void* w, const void* x_q8_1, float* y, const float* res,
                                          float* partials, int n_in, int n_out, int ncols, void* stream) {
    if (int rc = validate(w, x_q8_1, y, n_in, n_out, ncols, stream)) return rc;
    if (!aligned4(res) || !aligned4(partials))
        return fail(RMI_ERR_POINTER, "native MMVQ requires non-null 4-byte aligned device pointers");
    if (const int rc = registry_mmvq(w, x_q8_1, y, res, partials, n_in, n_out, ncols, stream); rc >= 0) return rc;
    return launch<true>(w, x_q8_1, y, res, partials, n_in, n_out, ncols, static_cast<hipStream_t>(stream));
}

extern "C" int rmi_native_q6_k_mmvq_res(const void* w, const void* x_q8_1, float* y, const float* res,
                                        float* partials, int n_in, int n_out, void* stream) {
    return rmi_native_q6_k_mmvq_res_n(w, x_q8_1, y, res, partials, n_in, n_out, 1, stream);
}

extern "C" int rmi_q6_k_block_dots(const void* w, const void* x_q8_1, int32_t* out, int n_in, int n_out,
                                   void* stream) {
    if (int rc = validate(w, x_q8_1, reinterpret_cast<const float*>(out), n_in, n_out, 1, stream)) return rc;
    const size_t lanes = static_cast<size_t>(n_out) * 2 * (n_in / 256);
    hipLaunchKernelGGL(q6k_block_dots_kernel, dim3(static_cast<unsigned>((lanes + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(w),
                       static_cast<const uint8_t*>(x_q8_1), out, n_in, n_out);
    return launch_status("q6_k_block_dots");
}

