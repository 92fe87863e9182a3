// mmvq_q6k_packed.hip - Q6_K x Q8_1 GEMV over a wave-tiled copy of the weights (caller-owned), for gfx950.
//
// Reference: the reference keeps an opt-in packed copy of a Q6_K matrix in a registry (native_q6_k_pack,
// src/native_mmvq.cu:2930-3040; used by native_q6_k_mmvq at mmvq:3629 when STRATA_Q6_PACKED=1).  Here the caller
// owns the packed buffer (rmi_q6_k_packed_bytes / rmi_q6_k_pack) and calls the packed GEMV on it directly.
//
// Packed layout.  Rows are grouped in quads (4 rows; the last quad zero-padded) and each row is cut in chunks of 8
// Q6_K blocks (2048 elements).  The 6720 bytes of one (quad, chunk) wave tile are re-laid so that lane l = 4 hb + r
// (row r of the quad, half-block hb: block hb / 2, half hb % 2) finds its half-block in registers after fully
// coalesced loads:
//     [    0, 4096)  ql: 16-byte unit u (0..3) of lane l at u * 1024 + 16 l   (ql bytes [64 n + 16 u, +16))
//     [ 4096, 6144)  qh: unit u (0..1) of lane l at 4096 + u * 1024 + 16 l    (qh bytes [32 n + 16 u, +16))
//     [ 6144, 6656)  sc: lane l's 8 sub-scales at 6144 + 8 l                  (sc bytes [8 n, +8))
//     [ 6656, 6720)  d:  block (r, b)'s fp16 scale at 6656 + 2 (4 b + r)
// The four rows of a half-block sit in four adjacent lanes: that is the operand layout of the 16-block 4x4x4 int8
// MFMA (block = half-block, A row = quad row), which the 8 / 16-column ingest kernel runs on.
// Wave tiles are stored quad-major: tile (q, c) at (q * nch + c) * 6720.
//
// Kernel: every wave streams its own quads (no workgroup barrier after the activation staging): the (quad, chunk)
// steps of its quads are loaded D steps ahead straight into registers (8 loads per step per lane, each a contiguous
// 1 KB / 512 B wave access), decoded as in the tiled kernel (v_dot4 with the "-32" folded into the staged record),
// and a row's 16 lanes are reduced by the same xor butterfly (over hb: lane offsets 32, 16, 8, 4).  Lane ownership, per-lane accumulation order and the
// reduction tree are those of the 16-row tiled kernel, so the results are bitwise the same, every column of an
// ncols >= 2 call is bitwise the ncols = 1 result, and the residual variant is bitwise plain + res.
//
// Rows of 4096, 8192 and 12288 (two, four and six chunks) run a stream variant: one wave per quad (two quads per wave
// for the lm_head's 62080 quads), in straight-line code with the tiles issued behind the activation loads, two tiles
// ahead of the step - the same bits, more loads in flight.
#include "rmi_common.h"

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <mutex>
#include <string>
#include <unordered_map>

namespace rmi {
namespace {

constexpr int kThreads = 256;
constexpr int kQuad = 4;                                  // rows per wave tile
constexpr int kChunkBlocks = 8;                           // Q6_K blocks per row per chunk
constexpr int kChunkElems = kChunkBlocks * 256;           // 2048
constexpr int kWaveTile = kQuad * kChunkBlocks * kQ6KBytes;   // 6720
constexpr int kNB = kChunkElems / 32;                     // Q8_1 blocks per chunk per column (64)
constexpr int kMaxStageBytes = 64 * 1024;                 // activation LDS per workgroup, up to 4 columns
constexpr int kWideStageBytes = 160 * 1024;               // 8 / 16 columns: the whole LDS of a CU (gfx950)
constexpr int kWideWaves = 8;                             // waves per workgroup sharing one wide activation stage

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int sc_byte2(uint32_t s0, uint32_t s1, int i) {
    const uint32_t w = i < 4 ? s0 : s1;
    return static_cast<int>(static_cast<int8_t>((w >> (8 * (i & 3))) & 0xffu));
}

__device__ __forceinline__ int subblock_dot(const int (&v)[8], const int (&u)[8], int corr0, int corr1, int sc0,
                                            int sc1) {
    int d0 = corr0, d1 = corr1;
#pragma unroll
    for (int w = 0; w < 4; ++w) d0 = sdot4(v[w], u[w], d0);
#pragma unroll
    for (int w = 4; w < 8; ++w) d1 = sdot4(v[w], u[w], d1);
    return __mul24(sc0, d0) + __mul24(sc1, d1);   // |sc|, |d| < 2^23: exact
}

// sum over the 16 half-blocks of a row (lanes 4 hb + r): the xor butterfly over hb with offsets 8, 4, 2, 1, the tree
// of the 16-row tiled kernel's row sum
__device__ __forceinline__ float hb_sum(float v) {
    v += xor_lane<32>(v);
    v += xor_lane<16>(v);
    v += xor_lane<8>(v);
    v += xor_lane<4>(v);
    return v;
}

// ---- pack: one thread per (quad, chunk, lane) --------------------------------------------------------------------------
// SwiGLU row order of an up||gate matrix ([up ff rows | gate ff rows] in the source): packed rows 64 G .. 64 G + 31 are
// gate rows 32 G .., rows 64 G + 32 .. 64 G + 63 up rows 32 G .., so a 16-quad group holds both inputs of 32 outputs
__host__ __device__ __forceinline__ int swiglu_src_row(int p, int ff) {
    const int g = p >> 6, j = p & 63;
    return j < 32 ? ff + 32 * g + j : 32 * g + j - 32;
}

// ff = 0: rows in source order; ff > 0: the SwiGLU order above (n_out = 2 ff, ff % 32 == 0)
__global__ __launch_bounds__(kThreads) void q6k_pack_kernel(const uint8_t* __restrict__ w, uint8_t* __restrict__ wp,
                                                            int n_in, int n_out, size_t nslots, int ff) {
    const size_t gid = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (gid >= nslots) return;
    const int nch = n_in / kChunkElems, nb = n_in / 256;
    const int l = static_cast<int>(gid & 63);
    const size_t tile = gid >> 6;                         // q * nch + c
    const int q = static_cast<int>(tile / nch), c = static_cast<int>(tile - static_cast<size_t>(q) * nch);
    const int r = l & 3, hb = l >> 2, b = hb >> 1, n = hb & 1;
    const int row = kQuad * q + r;
    uint8_t* dst = wp + tile * kWaveTile;
    const bool live = row < n_out;
    const int srow = ff > 0 && live ? swiglu_src_row(row, ff) : row;
    const uint8_t* src = w + (static_cast<size_t>(srow) * nb + static_cast<size_t>(c) * kChunkBlocks + b) * kQ6KBytes;
    for (int u = 0; u < 4; ++u)
        for (int i = 0; i < 16; ++i) dst[u * 1024 + 16 * l + i] = live ? src[64 * n + 16 * u + i] : 0;
    for (int u = 0; u < 2; ++u)
        for (int i = 0; i < 16; ++i) dst[4096 + u * 1024 + 16 * l + i] = live ? src[128 + 32 * n + 16 * u + i] : 0;
    for (int i = 0; i < 8; ++i) dst[6144 + 8 * l + i] = live ? src[192 + 8 * n + i] : 0;
    if (n == 0) {
        dst[6656 + 2 * (4 * b + r)] = live ? src[208] : 0;
        dst[6656 + 2 * (4 * b + r) + 1] = live ? src[209] : 0;
    }
}

// ---- GEMV ---------------------------------------------------------------------------------------------------------------
struct WTile {
    u32x4 ql[4];
    u32x4 qh[2];
    uint2 sc;
    uint32_t d;   // the dword holding the lane's fp16 block scale (half lane & 1)
};

// ---- shared pieces -------------------------------------------------------------------------------------------------
// The activation stage: whole-row activations, staged once per workgroup while the first weight steps are in flight,
// in three regions of NCOLS * nbt uint4 - codes 0..15 of a Q8_1 block | codes 16..31 | its record {-32 sum(codes
// 0..15), -32 sum(codes 16..31), d8, 0}.  Block jb = 64 c + 4 hb + k of column col (chunk c, sub-step k, the
// half-block hb that reads it) sits at slot ((4 c + k) NCOLS + col) 16 + hb of each region: the 16 half-blocks of a
// wave's read take 256 contiguous bytes (every LDS bank once), and a lane's 24 reads of a step are immediate offsets
// from one address per chunk, so the step spends no VALU on LDS addresses.
template <int NCOLS>
__device__ __forceinline__ int stage_slot(int col, int jb) {
    const int c = jb >> 6, j = jb & 63;
    return (((4 * c + (j & 3)) * NCOLS + col) << 4) + (j >> 2);
}

// block J (column J / nbt, block J % nbt of the column) into the stage st
template <int NCOLS>
__device__ __forceinline__ void stage_one(const uint32_t (&wv)[9], int J, int nbt, uint4* st) {
    const int col = J / nbt, jb = J - col * nbt;
    int s0 = 0, s1 = 0;
#pragma unroll
    for (int i = 1; i <= 4; ++i) s0 = sdot4(static_cast<int>(wv[i]), 0x01010101, s0);
#pragma unroll
    for (int i = 5; i <= 8; ++i) s1 = sdot4(static_cast<int>(wv[i]), 0x01010101, s1);
    const int rs = NCOLS * nbt, i = stage_slot<NCOLS>(col, jb);
    st[i] = make_uint4(wv[1], wv[2], wv[3], wv[4]);
    st[rs + i] = make_uint4(wv[5], wv[6], wv[7], wv[8]);
    st[2 * rs + i] = make_uint4(static_cast<uint32_t>(-32 * s0), static_cast<uint32_t>(-32 * s1),
                                __float_as_uint(half_bits_to_float(wv[0])), 0u);
}

// Blocks are taken up to 4 per lane at a time, every load of a batch issued before the first is used (768 blocks of a
// 12288-row at two columns: one batch per lane).  Measured against one block per iteration: 12288 x 4096 residual
// 12.1 -> 12.0 us, 4096 x 4096 residual 7.1 -> 6.9 us (the weight loads issued before the staging hide most of it).
template <int NCOLS>
__device__ __forceinline__ void stage_activations(const uint8_t* __restrict__ x, int nblocks, int nbt, uint4* st, int t,
                                                  int nthreads) {
    constexpr int B = 4;
    for (int J0 = t; J0 < nblocks; J0 += B * nthreads) {
        uint32_t wv[B][9];
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int J = J0 + b * nthreads;
            if (J < nblocks) {
                const uint32_t* p = reinterpret_cast<const uint32_t*>(x + static_cast<size_t>(J) * kQ8_1Bytes);
#pragma unroll
                for (int i = 0; i < 9; ++i) wv[b][i] = p[i];
            }
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int J = J0 + b * nthreads;
            if (J < nblocks) stage_one<NCOLS>(wv[b], J, nbt, st);
        }
    }
}

// a lane's read addresses into the stage: the three regions at its half-block (add kNB * NCOLS per chunk)
struct StageLane {
    const uint4* a;
    const uint4* b;
    const uint4* r;
};
template <int NCOLS>
__device__ __forceinline__ StageLane stage_lane(const uint4* st, int nbt, int lane) {
    const uint4* a = st + (lane >> 2);
    return {a, a + NCOLS * nbt, a + 2 * NCOLS * nbt};
}

// ---- a normed vector quantized straight into the stage ------------------------------------------------------------
// The GEMV's input as rms_quant_apply makes it (qw:627-655): Q8_1 of (x * w) * inv per column, inv = rsqrt(sum of x's
// 4-row partials / n + eps) by the norm kernels' tree (rmi_common.h), quantized into the activation stage instead of
// HBM.  The codes, the fp16 block scale and the stage record are those of rms_quant_apply followed by stage_one, bit
// for bit, and the norm's own launch (a graph node and a dependent memory level) is gone.  Two lanes per Q8_1 block,
// 16 elements each: the block's amax and the second half's code sum cross by one lane exchange, and q8_round_fast
// replaces the block's divides.  norm_issue loads ahead of the weight tiles, norm_stage computes after they are issued.
struct NormIn {
    const float* x;      // NCOLS columns of n_in (column c at + c n_in), 16-byte aligned
    const float* w;      // the norm weights (n_in), 16-byte aligned
    const float* part;   // x's 4-row partials (column c at + c n_in / 4)
    float eps;
};

template <int NCOLS, int NCH, int NW>
struct NormLanes {
    static constexpr int kNbt = NCH * kNB;                              // Q8_1 blocks per column
    static constexpr int kHalves = 2 * NCOLS * kNbt;                     // half-blocks of the stage
    static constexpr int kHPL = (kHalves + 64 * NW - 1) / (64 * NW);     // half-blocks per lane
    static constexpr int kTreeCols = NW >= 8 ? 1 : NCOLS;                // columns a lane's four-wave group reduces
    static constexpr int kNp = NCH * kChunkElems / 4;                    // partial slots per column
    static constexpr int kPL = kNp / 256;                                // partial slots per tree lane
    float pv[kTreeCols][kPL];
    float4 xv[kHPL][4], wv[kHPL][4];
};

// the norm tree runs on 256 lanes per column: waves 0..3 (column 0) and 4..7 (column 1) of a workgroup of 8 or more
// waves, or waves 0..3 for every column of a 4-wave one
template <int NCOLS, int NCH, int NW>
__device__ __forceinline__ void norm_issue(NormLanes<NCOLS, NCH, NW>& L, const NormIn& ni, int t) {
    static_assert(NW == 4 || NW % 8 == 0, "the norm tree takes four waves per column");
    using NL = NormLanes<NCOLS, NCH, NW>;
    static_assert(NL::kNp % 256 == 0, "whole tree lanes");
    constexpr int n = NCH * kChunkElems;
    const int tt = t & 255;
#pragma unroll
    for (int k = 0; k < NL::kTreeCols; ++k) {
        const int col = NW >= 8 ? min(t >> 8, NCOLS - 1) : k;
        const float* p = ni.part + static_cast<size_t>(col) * NL::kNp;
#pragma unroll
        for (int i = 0; i < NL::kPL; ++i) L.pv[k][i] = p[tt + 256 * i];
    }
#pragma unroll
    for (int h = 0; h < NL::kHPL; ++h) {
        const int g = min(t + 64 * NW * h, NL::kHalves - 1);
        const int J = g >> 1, col = J / NL::kNbt, blk = J - col * NL::kNbt;
        const int e0 = 32 * blk + 16 * (g & 1);
        const float4* xp = reinterpret_cast<const float4*>(ni.x + static_cast<size_t>(col) * n + e0);
        const float4* wp = reinterpret_cast<const float4*>(ni.w + e0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            L.xv[h][i] = xp[i];
            L.wv[h][i] = wp[i];
        }
    }
}

// inv per column, then every half-block into the stage; red: NCOLS x 4 floats of LDS.  Ends before the caller's
// stage barrier (it contains one barrier of its own, after the tree).  The products x * w and their block maximum
// are formed while the tree's partials are summed: the block's amax, max |RN((x * w) * inv)|, is RN(max |x * w| * inv)
// (rounding is monotonic), so only the scaling waits for inv.
template <int NCOLS, int NCH, int NW>
__device__ __forceinline__ void norm_stage(const NormLanes<NCOLS, NCH, NW>& L, const NormIn& ni, uint4* st, int t,
                                           float (*red)[4]) {
    using NL = NormLanes<NCOLS, NCH, NW>;
    constexpr int n = NCH * kChunkElems;
#pragma unroll
    for (int k = 0; k < NL::kTreeCols; ++k) {
        const int col = NW >= 8 ? t >> 8 : k;
        if (col < NCOLS && (NW >= 8 || t < 256)) {   // whole waves
            float sw = 0.0f;   // the lane's slots in order, then the wave's butterfly (norm_wave_sum)
#pragma unroll
            for (int i = 0; i < NL::kPL; ++i) sw += L.pv[k][i];
            sw = group_sum<64>(sw);
            if ((t & 63) == 0) red[col][(t >> 6) & 3] = sw;
        }
    }
    float xw[NL::kHPL][16], mx[NL::kHPL];
#pragma unroll
    for (int h = 0; h < NL::kHPL; ++h) {
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xw[h][4 * i + 0] = L.xv[h][i].x * L.wv[h][i].x;
            xw[h][4 * i + 1] = L.xv[h][i].y * L.wv[h][i].y;
            xw[h][4 * i + 2] = L.xv[h][i].z * L.wv[h][i].z;
            xw[h][4 * i + 3] = L.xv[h][i].w * L.wv[h][i].w;
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) m = fmaxf(m, fabsf(xw[h][e]));
        mx[h] = fmaxf(m, xor_lane<1>(m));
    }
    __syncthreads();
    float inv[NCOLS];
#pragma unroll
    for (int c = 0; c < NCOLS; ++c) inv[c] = norm_inv(red[c], n, ni.eps);
    const int rs = NCOLS * NL::kNbt;
#pragma unroll
    for (int h = 0; h < NL::kHPL; ++h) {
        const int g0 = t + 64 * NW * h;
        const bool live = g0 < NL::kHalves;   // pairs (2 J, 2 J + 1) are live together
        const int g = min(g0, NL::kHalves - 1);
        const int J = g >> 1, col = J / NL::kNbt, blk = J - col * NL::kNbt, half = g & 1;
        const float iv = inv[col];
        const float am = mx[h] * iv;
        const float d = am / 127.0f;
        const float inv_d = 1.0f / d;
        float v[16], r[16];
        uint32_t slow = 0;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            v[e] = xw[h][e] * iv;
            bool sl;
            r[e] = q8_round_fast(v[e], d, inv_d, sl);
            slow |= static_cast<uint32_t>(sl) << e;
        }
        if (__builtin_amdgcn_ballot_w64(slow != 0)) {   // rare: roundf of the true quotient for the flagged values
#pragma unroll
            for (int e = 0; e < 16; ++e)
                if (slow >> e & 1u) r[e] = roundf(v[e] / d);
        }
        uint32_t dw[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t word = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int q = am == 0.0f ? 0 : static_cast<int>(r[4 * i + e]);
                word |= (static_cast<uint32_t>(q) & 0xffu) << (8 * e);
            }
            dw[i] = word;
        }
        int sc = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) sc = sdot4(static_cast<int>(dw[i]), 0x01010101, sc);
        const int sc_other = static_cast<int>(xor_lane<1>(static_cast<uint32_t>(sc)));
        if (live) {
            const int slot = stage_slot<NCOLS>(col, blk);
            st[half * rs + slot] = make_uint4(dw[0], dw[1], dw[2], dw[3]);
            if (half == 0)
                st[2 * rs + slot] = make_uint4(static_cast<uint32_t>(-32 * sc), static_cast<uint32_t>(-32 * sc_other),
                                               __float_as_uint(half_bits_to_float(float_to_half_sat(d))), 0u);
        }
    }
}

// Marks the point where a tile's registers are first used: no computation on them moves above it and no load moves
// across it, so the wait placed here covers this tile and the loads issued before it only (loads complete in issue
// order), and the previous step's arithmetic stays above it (the running sums pass through the asm).  Without it the
// compiler converts a tile's scale right after its load, or hoists the wait for this tile above the previous step's
// compute, and the wait stalls later loads.
template <int NCOLS>
__device__ __forceinline__ void pin_tile_after(WTile& w, float (&tot)[NCOLS]) {
    static_assert(NCOLS == 1 || NCOLS == 2, "one or two columns");
    if constexpr (NCOLS == 1)
        asm volatile("" : "+v"(w.ql[0]), "+v"(w.ql[1]), "+v"(w.ql[2]), "+v"(w.ql[3]), "+v"(w.qh[0]), "+v"(w.qh[1]),
                     "+v"(w.sc), "+v"(w.d), "+v"(tot[0])::"memory");
    else
        asm volatile("" : "+v"(w.ql[0]), "+v"(w.ql[1]), "+v"(w.ql[2]), "+v"(w.ql[3]), "+v"(w.qh[0]), "+v"(w.qh[1]),
                     "+v"(w.sc), "+v"(w.d), "+v"(tot[0]), "+v"(tot[1])::"memory");
}

// one wave tile step of lane l: its half-block (row l / 16, half-block l % 16) against every column's staged chunk c
// (sl: the lane's stage addresses, c: the chunk; the tile's block scale d is returned, the lane's sum in acc[col]);
// the step adds fma(d, acc[col], tot[col])
template <int NCOLS>
__device__ __forceinline__ float step_acc(const WTile& wt, int lane, const StageLane& sl, int c, float (&acc)[NCOLS]) {
    uint32_t Q[16], H[8];
#pragma unroll
    for (int i = 0; i < 16; ++i) Q[i] = wt.ql[i >> 2][i & 3];
#pragma unroll
    for (int i = 0; i < 8; ++i) H[i] = wt.qh[i >> 2][i & 3];
    const uint32_t S0 = wt.sc.x, S1 = wt.sc.y;
    const int cb = c * kNB * NCOLS;
    const uint4* pa = sl.a + cb;
    const uint4* pb = sl.b + cb;
    const uint4* pr = sl.r + cb;

#pragma unroll
    for (int col = 0; col < NCOLS; ++col) acc[col] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
            const int k = kk + 2 * kh;
            int v[8];
#pragma unroll
            for (int ww = 0; ww < 8; ++ww)
                v[ww] = static_cast<int>(((Q[8 * kk + ww] >> (4 * kh)) & 0x0f0f0f0fu) |
                                         (((H[ww] >> (2 * k)) & 0x03030303u) << 4));
            const int sc0 = sc_byte2(S0, S1, 2 * k), sc1 = sc_byte2(S0, S1, 2 * k + 1);
#pragma unroll
            for (int col = 0; col < NCOLS; ++col) {
                const int o = (k * NCOLS + col) * 16;
                const uint4 qa = pa[o];
                const uint4 qb = pb[o];
                const uint4 rec = pr[o];
                const int u[8] = {static_cast<int>(qa.x), static_cast<int>(qa.y), static_cast<int>(qa.z),
                                  static_cast<int>(qa.w), static_cast<int>(qb.x), static_cast<int>(qb.y),
                                  static_cast<int>(qb.z), static_cast<int>(qb.w)};
                const int sd = subblock_dot(v, u, static_cast<int>(rec.x), static_cast<int>(rec.y), sc0, sc1);
                acc[col] = __builtin_fmaf(__uint_as_float(rec.z), static_cast<float>(sd), acc[col]);
            }
        }
    }
    return half_bits_to_float((lane & 1) ? wt.d >> 16 : wt.d & 0xffffu);
}

template <int NCOLS>
__device__ __forceinline__ void accumulate_step(const WTile& wt, int lane, const StageLane& sl, int c,
                                                float (&tot)[NCOLS]) {
    float acc[NCOLS];
    const float d = step_acc<NCOLS>(wt, lane, sl, c, acc);
#pragma unroll
    for (int col = 0; col < NCOLS; ++col) tot[col] = __builtin_fmaf(d, acc[col], tot[col]);
}

// the finished quad q (lane 4 hb + r holds row 4 q + r's half-block sums): row sums, the residual, y and the quad's
// sum of squares
// the residual of quad q's rows for this lane (row 4 q + lane % 4), loaded from a clamped row so that the load can go
// out with the kernel's first loads (in the epilogue it would wait behind every tile issued before it)
template <int NCOLS>
__device__ __forceinline__ void load_residual(float (&rv)[NCOLS], const float* res, int lane, int q, int n_out) {
    const int row = min(kQuad * q + (lane & 3), n_out - 1);
#pragma unroll
    for (int col = 0; col < NCOLS; ++col) rv[col] = res[static_cast<size_t>(col) * n_out + row];
}

template <int NCOLS, bool RES>
__device__ __forceinline__ void quad_epilogue(float (&tot)[NCOLS], int lane, int q, float* y, const float* res,
                                              float* partials, int n_out, const float* rv = nullptr) {
    const int r = lane & 3, hb = lane >> 2;
    const int row = kQuad * q + r;
    const int np = (n_out + 3) / 4;
#pragma unroll
    for (int col = 0; col < NCOLS; ++col) {
        float v = hb_sum(tot[col]);
        tot[col] = 0.0f;
        if constexpr (RES) {
            if (row < n_out) v += rv ? rv[col] : res[static_cast<size_t>(col) * n_out + row];
        }
        if (hb == 0 && row < n_out) y[static_cast<size_t>(col) * n_out + row] = v;
        if constexpr (RES) {
            // partial of the quad: squares of its rows in row order (lanes 0, 1, 2, 3)
            const float v0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
            const float v1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 1));
            const float v2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 2));
            const float v3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 3));
            if (lane == 0) {
                const int row0 = kQuad * q;
                float p = __builtin_fmaf(v0, v0, 0.0f);
                if (row0 + 1 < n_out) p = __builtin_fmaf(v1, v1, p);
                if (row0 + 2 < n_out) p = __builtin_fmaf(v2, v2, p);
                if (row0 + 3 < n_out) p = __builtin_fmaf(v3, v3, p);
                partials[static_cast<size_t>(col) * np + q] = p;
            }
        }
    }
}

// NW waves per workgroup share the staged activations: 4 for up to 4 columns (several workgroups per CU), 8 for the
// 8 / 16-column ingest passes, whose stage fills most of the CU's LDS (one workgroup per CU)
template <int NCOLS, bool RES, int D, int NW>
__global__ __launch_bounds__(64 * NW) void q6k_packed_gemv(const uint8_t* __restrict__ wp,
                                                           const uint8_t* __restrict__ x, float* y,
                                                           const float* res, float* partials, int n_in, int n_out) {
    extern __shared__ uint4 smem[];
    const int t = threadIdx.x, lane = t & 63;
    const int nch = n_in / kChunkElems;
    const int nbt = n_in / 32;                   // Q8_1 blocks per column
    uint4* st = smem;                            // the activation stage (stage_slot)
    const StageLane sl = stage_lane<NCOLS>(st, nbt, lane);
    const int nq = (n_out + kQuad - 1) / kQuad;
    const int GW = static_cast<int>(gridDim.x) * NW;
    const int gw = static_cast<int>(blockIdx.x) * NW + (t >> 6);
    const int my_quads = gw < nq ? (nq - 1 - gw) / GW + 1 : 0;
    const int nsteps = my_quads * nch;

    WTile buf[D];
    auto issue = [&](int f, WTile& b) {
        const int qi = f / nch, c = f - qi * nch;
        const uint8_t* base = wp + (static_cast<size_t>(gw + qi * GW) * nch + c) * kWaveTile;
#pragma unroll
        for (int u = 0; u < 4; ++u)
            b.ql[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + u * 1024 + 16 * lane));
#pragma unroll
        for (int u = 0; u < 2; ++u)
            b.qh[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + 4096 + u * 1024 + 16 * lane));
        b.sc = *reinterpret_cast<const uint2*>(base + 6144 + 8 * lane);
        b.d = *reinterpret_cast<const uint32_t*>(base + 6656 + 4 * (2 * (lane >> 3) + ((lane & 3) >> 1)));
    };
#pragma unroll
    for (int s = 0; s < D; ++s)
        if (s < nsteps) issue(s, buf[s]);

    stage_activations<NCOLS>(x, NCOLS * nbt, nbt, st, t, 64 * NW);
    __syncthreads();

    float tot[NCOLS];
#pragma unroll
    for (int col = 0; col < NCOLS; ++col) tot[col] = 0.0f;

    for (int f0 = 0; f0 < nsteps; f0 += D) {
#pragma unroll
        for (int s = 0; s < D; ++s) {
            const int f = f0 + s;
            if (f >= nsteps) break;   // uniform across the wave
            const int qi = f / nch, c = f - qi * nch;
            const WTile cur = buf[s];
            if (f + D < nsteps) issue(f + D, buf[s]);
            accumulate_step<NCOLS>(cur, lane, sl, c, tot);

            if (c == nch - 1)
                quad_epilogue<NCOLS, RES>(tot, lane, gw + qi * GW, y, res, partials, n_out);
        }
    }
}

// Stream variant: one wave per quad and QPW quads per wave (quads q, q + G, q + 2G, ... with G the grid's wave count),
// all in straight-line code with PD tiles in flight ahead of the step that uses them.  Every wave is resident from the
// start (a wave per quad would leave a tail of waves waiting for slots), and the per-quad arithmetic is that of
// q6k_packed_gemv: the same bits.  NORM: the input is a normed vector quantized in the stage (norm_stage; x unused).
template <int NCOLS, bool RES, int NCH, int QPW, int NW, int PD, bool NORM = false>
__global__ __launch_bounds__(64 * NW) void q6k_packed_gemv_stream(const uint8_t* __restrict__ wp,
                                                                  const uint8_t* __restrict__ x, float* y,
                                                                  const float* res, float* partials, int n_in,
                                                                  int n_out, NormIn ni) {
    extern __shared__ uint4 smem[];
    __shared__ float nred[NORM ? NCOLS : 1][4];
    const int t = threadIdx.x, lane = t & 63;
    const int nbt = n_in / 32;
    uint4* st = smem;   // the activation stage (stage_slot)
    const StageLane sl = stage_lane<NCOLS>(st, nbt, lane);
    const int nq = (n_out + kQuad - 1) / kQuad;
    const int G = static_cast<int>(gridDim.x) * NW;
    const int q0 = static_cast<int>(blockIdx.x) * NW + (t >> 6);

    // activation loads first (a wave's loads return in issue order), clamped so that none sits in a branch
    // activation blocks per lane loaded ahead of the tiles: the whole row where four per lane hold it, else four
    constexpr int SB = NORM ? 0 : std::min(4, (NCOLS * NCH * kNB + 64 * NW - 1) / (64 * NW));
    const int nblocks = NCOLS * nbt;
    uint32_t sv[SB > 0 ? SB : 1][9];
#pragma unroll
    for (int b = 0; b < SB; ++b) {
        const int J = min(t + b * 64 * NW, nblocks - 1);
        const uint32_t* p = reinterpret_cast<const uint32_t*>(x + static_cast<size_t>(J) * kQ8_1Bytes);
#pragma unroll
        for (int i = 0; i < 9; ++i) sv[b][i] = p[i];
    }
    NormLanes<NCOLS, NCH, NW> nl;
    if constexpr (NORM) norm_issue<NCOLS, NCH, NW>(nl, ni, t);
    float rv[QPW][NCOLS];
    if constexpr (RES) {
#pragma unroll
        for (int j = 0; j < QPW; ++j) load_residual<NCOLS>(rv[j], res, lane, min(q0 + j * G, nq - 1), n_out);
    }
    __builtin_amdgcn_sched_barrier(0);

    // tile i = (quad j = i / NCH, chunk i % NCH); a quad past the last reads the last quad's tiles and discards them
    constexpr int T = QPW * NCH;
    WTile buf[T];
    auto issue = [&](int i) {
        const int j = i / NCH, c = i - j * NCH;
        const int qq = min(q0 + j * G, nq - 1);
        const uint8_t* base = wp + (static_cast<size_t>(qq) * NCH + c) * kWaveTile;
#pragma unroll
        for (int u = 0; u < 4; ++u)
            buf[i].ql[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + u * 1024 + 16 * lane));
#pragma unroll
        for (int u = 0; u < 2; ++u)
            buf[i].qh[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + 4096 + u * 1024 + 16 * lane));
        buf[i].sc = *reinterpret_cast<const uint2*>(base + 6144 + 8 * lane);
        buf[i].d = *reinterpret_cast<const uint32_t*>(base + 6656 + 4 * (2 * (lane >> 3) + ((lane & 3) >> 1)));
    };
#pragma unroll
    for (int i = 0; i < PD && i < T; ++i) {
        issue(i);
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (NORM) {
        norm_stage<NCOLS, NCH, NW>(nl, ni, st, t, nred);
    } else {
        // unconditional (lanes past the last block rewrite its slot with the same bytes): under a branch the compiler
        // sinks the stage's loads into it, behind the first tiles, and the stage then waits for those
#pragma unroll
        for (int b = 0; b < SB; ++b) stage_one<NCOLS>(sv[b], min(t + b * 64 * NW, nblocks - 1), nbt, st);
        for (int J = t + SB * 64 * NW; J < nblocks; J += 64 * NW) {
            const uint32_t* p = reinterpret_cast<const uint32_t*>(x + static_cast<size_t>(J) * kQ8_1Bytes);
            uint32_t wv[9];
#pragma unroll
            for (int i = 0; i < 9; ++i) wv[i] = p[i];
            stage_one<NCOLS>(wv, J, nbt, st);
        }
    }
    __syncthreads();

    float tot[NCOLS];
#pragma unroll
    for (int col = 0; col < NCOLS; ++col) tot[col] = 0.0f;
#pragma unroll
    for (int i = 0; i < T; ++i) {
        const int j = i / NCH, c = i - (i / NCH) * NCH;
        pin_tile_after<NCOLS>(buf[i], tot);
        float acc[NCOLS];
        const float d = step_acc<NCOLS>(buf[i], lane, sl, c, acc);
#pragma unroll
        for (int col = 0; col < NCOLS; ++col) tot[col] = __builtin_fmaf(d, acc[col], tot[col]);
        if (i + PD < T) {
            __builtin_amdgcn_sched_barrier(0);
            issue(i + PD);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (c == NCH - 1 && q0 + j * G < nq)
            quad_epilogue<NCOLS, RES>(tot, lane, q0 + j * G, y, res, partials, n_out, rv[j]);
    }
}

// ---- the same stream kernel over the GGUF layout (the drop-in entry points' weights) ------------------------------
// A wave tile is the quad's 4 rows x 8 blocks of one chunk: four 1680-byte row segments, 16-byte aligned when the row
// length is a multiple of 2048 (rows of 8k blocks are 1680k bytes).  The lane loads 7 of the tile's 420 16-byte units
// (unit i = lane + 64 m: row i / 105, unit i % 105), fully coalesced per row segment, two tiles ahead in registers.
// At its step the wave parks the tile in its own LDS rows (no workgroup barrier: only the wave reads them) and each
// lane reads its half-block (row lane % 4, half-block lane / 4, the packed kernel's ownership) back as aligned dwords
// realigned with v_alignbyte for the odd blocks' 2-byte offset.  The per-lane arithmetic is step_acc's, so the result
// is bitwise the packed kernels' (and the 16-row tiled kernel's) on the same matrix.
constexpr int kGgufUnits = 4 * kChunkBlocks * kQ6KBytes / 16;   // 420 16-byte units per wave tile
constexpr int kGgufRowUnits = kGgufUnits / 4;                   // 105 per row segment
constexpr int kGgufLoads = (kGgufUnits + 63) / 64;              // 7 per lane
constexpr int kGgufRowDw = kChunkBlocks * kQ6KBytes / 4 + 4;    // 424 dwords per parked row (16-byte multiple)
constexpr int kGgufWaveDw = 4 * kGgufRowDw;                     // 6784 bytes of LDS per wave

struct GTile {
    u32x4 u[kGgufLoads];
};

__device__ __forceinline__ void lds_wave_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// pin_tile_after for a raw GGUF tile: its wait covers this tile and the loads issued before it only, and the previous
// step's arithmetic stays above it
template <int NCOLS>
__device__ __forceinline__ void pin_gtile_after(GTile& g, float (&tot)[NCOLS]) {
#pragma unroll
    for (int c = 0; c < NCOLS; ++c) asm volatile("" : "+v"(tot[c])::"memory");
    asm volatile("" : "+v"(g.u[0]), "+v"(g.u[1]), "+v"(g.u[2]), "+v"(g.u[3]), "+v"(g.u[4]), "+v"(g.u[5]),
                 "+v"(g.u[6])::"memory");
}

// the lane's half-block of a parked tile as the packed kernel's registers
__device__ __forceinline__ void gguf_unpack(const GTile& g, uint32_t* lw, int lane, WTile& wt) {
#pragma unroll
    for (int m = 0; m < kGgufLoads; ++m) {
        const int i = min(lane + 64 * m, kGgufUnits - 1);   // lanes past the last unit rewrite it with the same bytes
        const int r = i / kGgufRowUnits, u = i - r * kGgufRowUnits;
        *reinterpret_cast<u32x4*>(lw + r * kGgufRowDw + 4 * u) = g.u[m];
    }
    lds_wave_fence();
    const int r = lane & 3, hb = lane >> 2, b = hb >> 1, n = hb & 1;
    const int row = r * kGgufRowDw * 4 + b * kQ6KBytes;   // byte offset of the lane's block in the parked rows
    const int mis = row & 3;                              // 0, or 2 for odd blocks
    const int q0 = (row + 64 * n) >> 2, h0 = (row + 128 + 32 * n) >> 2, s0 = (row + 192 + 8 * n) >> 2;
    uint32_t tq[17], th[9], ts[3];
#pragma unroll
    for (int k = 0; k < 17; ++k) tq[k] = lw[q0 + k];
#pragma unroll
    for (int k = 0; k < 9; ++k) th[k] = lw[h0 + k];
#pragma unroll
    for (int k = 0; k < 3; ++k) ts[k] = lw[s0 + k];
    const int dbyte = row + 208;
    const uint32_t dw = lw[dbyte >> 2];
#pragma unroll
    for (int k = 0; k < 16; ++k) wt.ql[k >> 2][k & 3] = __builtin_amdgcn_alignbyte(tq[k + 1], tq[k], mis);
#pragma unroll
    for (int k = 0; k < 8; ++k) wt.qh[k >> 2][k & 3] = __builtin_amdgcn_alignbyte(th[k + 1], th[k], mis);
    wt.sc.x = __builtin_amdgcn_alignbyte(ts[1], ts[0], mis);
    wt.sc.y = __builtin_amdgcn_alignbyte(ts[2], ts[1], mis);
    const uint32_t d16 = (dw >> (8 * (dbyte & 3))) & 0xffffu;
    wt.d = (lane & 1) ? d16 << 16 : d16;   // where step_acc takes the lane's scale from
}

template <int NCOLS, bool RES, int NCH, int QPW, int NW, int PD>
__global__ __launch_bounds__(64 * NW) void q6k_gguf_stream(const uint8_t* __restrict__ w, const uint8_t* __restrict__ x,
                                                           float* y, const float* res, float* partials, int n_in,
                                                           int n_out) {
    extern __shared__ uint4 smem[];
    const int t = threadIdx.x, lane = t & 63;
    const int nbt = n_in / 32;
    uint4* st = smem;   // the activation stage (stage_slot)
    const StageLane sl = stage_lane<NCOLS>(st, nbt, lane);
    uint32_t* lw = reinterpret_cast<uint32_t*>(st + 3 * NCOLS * nbt) + (t >> 6) * kGgufWaveDw;
    const int nq = (n_out + kQuad - 1) / kQuad;
    const int G = static_cast<int>(gridDim.x) * NW;
    const int q0 = static_cast<int>(blockIdx.x) * NW + (t >> 6);
    const size_t rowbytes = static_cast<size_t>(n_in / 256) * kQ6KBytes;

    // activation blocks per lane loaded ahead of the tiles: the whole row where four per lane hold it, else four
    constexpr int SB = std::min(4, (NCOLS * NCH * kNB + 64 * NW - 1) / (64 * NW));
    const int nblocks = NCOLS * nbt;
    uint32_t sv[SB][9];
#pragma unroll
    for (int b = 0; b < SB; ++b) {
        const int J = min(t + b * 64 * NW, nblocks - 1);
        const uint32_t* p = reinterpret_cast<const uint32_t*>(x + static_cast<size_t>(J) * kQ8_1Bytes);
#pragma unroll
        for (int i = 0; i < 9; ++i) sv[b][i] = p[i];
    }
    float rv[QPW][NCOLS];
    if constexpr (RES) {
#pragma unroll
        for (int j = 0; j < QPW; ++j) load_residual<NCOLS>(rv[j], res, lane, min(q0 + j * G, nq - 1), n_out);
    }
    __builtin_amdgcn_sched_barrier(0);

    // tile i = (quad j = i / NCH, chunk i % NCH); rows past the last are read from the last row and discarded
    constexpr int T = QPW * NCH;
    GTile buf[T];
    auto issue = [&](int i) {
        const int j = i / NCH, c = i - j * NCH;
        const int row0 = kQuad * min(q0 + j * G, nq - 1);
#pragma unroll
        for (int m = 0; m < kGgufLoads; ++m) {
            const int u = min(lane + 64 * m, kGgufUnits - 1);
            const int r = u / kGgufRowUnits, uu = u - r * kGgufRowUnits;
            const uint8_t* p = w + static_cast<size_t>(min(row0 + r, n_out - 1)) * rowbytes +
                               static_cast<size_t>(c) * (kChunkBlocks * kQ6KBytes) + 16 * uu;
            buf[i].u[m] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
        }
    };
#pragma unroll
    for (int i = 0; i < PD && i < T; ++i) {
        issue(i);
        __builtin_amdgcn_sched_barrier(0);
    }
    // unconditional (lanes past the last block rewrite its slot with the same bytes): under a branch the compiler sinks
    // the stage's loads into it, behind the first tiles, and the stage then waits for those
#pragma unroll
    for (int b = 0; b < SB; ++b) stage_one<NCOLS>(sv[b], min(t + b * 64 * NW, nblocks - 1), nbt, st);
    for (int J = t + SB * 64 * NW; J < nblocks; J += 64 * NW) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(x + static_cast<size_t>(J) * kQ8_1Bytes);
        uint32_t wv[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) wv[i] = p[i];
        stage_one<NCOLS>(wv, J, nbt, st);
    }
    __syncthreads();

    float tot[NCOLS];
#pragma unroll
    for (int col = 0; col < NCOLS; ++col) tot[col] = 0.0f;
#pragma unroll
    for (int i = 0; i < T; ++i) {
        const int j = i / NCH, c = i - (i / NCH) * NCH;
        pin_gtile_after<NCOLS>(buf[i], tot);
        WTile wt;
        gguf_unpack(buf[i], lw, lane, wt);
        float acc[NCOLS];
        const float d = step_acc<NCOLS>(wt, lane, sl, c, acc);
#pragma unroll
        for (int col = 0; col < NCOLS; ++col) tot[col] = __builtin_fmaf(d, acc[col], tot[col]);
        if (i + PD < T) {
            __builtin_amdgcn_sched_barrier(0);
            issue(i + PD);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (c == NCH - 1 && q0 + j * G < nq)
            quad_epilogue<NCOLS, RES>(tot, lane, q0 + j * G, y, res, partials, n_out, rv[j]);
    }
}

// up||gate GEMV with the SwiGLU + Q8_1 epilogue, over a matrix packed in the SwiGLU row order (rows of 4096: two
// chunks).  A 16-quad group holds the gate and up rows of 32 outputs; workgroup b (NW waves) owns GPW = NW QPW / 16
// consecutive groups and wave w takes QPW of their quads as the stream kernel takes its quads, two tiles ahead (same
// per-row arithmetic, so the same row sums as the plain GEMV), parks the row sums in LDS, and one 32-lane group per
// (group, column) forms silu(gate) * up and its Q8_1 block with the quantizer of swiglu_quant: bitwise the GEMV +
// swiglu_quant pair, one launch and no fp32 round trip.
// The engine's shape runs 8 waves and two groups per workgroup: 192 workgroups at n_ff 12288, one per CU.  With one
// group per 4-wave workgroup (384) half the CUs hold two, and the second's activation stage queues behind the first's
// weight tiles in the CU's memory pipeline (per-wave clock stamps: stage at 5.3 us against 1.6 us, its waves last to
// finish): 24576 x 4096 at two columns 17.2 -> 16.0 us.  Deeper prefetch (3 or 4 tiles ahead) and 16 waves of two
// quads were slower (17.2, 18.4, 29.6 us).
// NORM: the input is a normed vector quantized in the stage (norm_stage; x unused).
template <int NCOLS, int NW = 4, int QPW = 4, int PD = 2, bool NORM = false>
__global__ __launch_bounds__(64 * NW) void q6k_packed_swiglu(const uint8_t* __restrict__ wp,
                                                             const uint8_t* __restrict__ x, uint8_t* __restrict__ out,
                                                             int n_in, int ff, NormIn ni) {
    constexpr int NCH = 2, T = QPW * NCH;
    constexpr int GPW = NW * QPW / 16;   // 16-quad groups per workgroup
    static_assert(GPW * 16 == NW * QPW && GPW >= 1, "whole groups per workgroup");
    extern __shared__ uint4 smem[];
    __shared__ float nred[NORM ? NCOLS : 1][4];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int nbt = n_in / 32;
    uint4* st = smem;   // the activation stage (stage_slot)
    const StageLane sl = stage_lane<NCOLS>(st, nbt, lane);
    float* lrow = reinterpret_cast<float*>(st + 3 * NCOLS * nbt);   // [group][col][64 rows of the group]
    const int q0 = static_cast<int>(blockIdx.x) * 16 * GPW + QPW * w;

    const int nblocks = NCOLS * nbt;   // <= 2 x 128: one block per lane at most
    static_assert(64 * NW >= 2 * 128, "one staged block per lane");
    uint32_t sv[9];
    NormLanes<NCOLS, NCH, NW> nl;
    if constexpr (NORM) {
        norm_issue<NCOLS, NCH, NW>(nl, ni, t);
    } else {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(x + static_cast<size_t>(min(t, nblocks - 1)) * kQ8_1Bytes);
#pragma unroll
        for (int i = 0; i < 9; ++i) sv[i] = p[i];
    }
    __builtin_amdgcn_sched_barrier(0);
    WTile buf[T];
    auto issue = [&](int i) {
        const int j = i / NCH, c = i - j * NCH;
        const uint8_t* base = wp + (static_cast<size_t>(q0 + j) * NCH + c) * kWaveTile;
#pragma unroll
        for (int u = 0; u < 4; ++u)
            buf[i].ql[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + u * 1024 + 16 * lane));
#pragma unroll
        for (int u = 0; u < 2; ++u)
            buf[i].qh[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + 4096 + u * 1024 + 16 * lane));
        buf[i].sc = *reinterpret_cast<const uint2*>(base + 6144 + 8 * lane);
        buf[i].d = *reinterpret_cast<const uint32_t*>(base + 6656 + 4 * (2 * (lane >> 3) + ((lane & 3) >> 1)));
    };
#pragma unroll
    for (int i = 0; i < PD; ++i) {
        issue(i);
        __builtin_amdgcn_sched_barrier(0);
    }
    // unconditional (lanes past the last block rewrite its slot with the same bytes): under a branch the compiler sinks
    // the stage's loads into it, behind the first tiles, and the stage then waits for those
    if constexpr (NORM) norm_stage<NCOLS, NCH, NW>(nl, ni, st, t, nred);
    else stage_one<NCOLS>(sv, min(t, nblocks - 1), nbt, st);
    __syncthreads();

    float tot[NCOLS];
#pragma unroll
    for (int col = 0; col < NCOLS; ++col) tot[col] = 0.0f;
#pragma unroll
    for (int i = 0; i < T; ++i) {
        const int j = i / NCH, c = i - (i / NCH) * NCH;
        pin_tile_after<NCOLS>(buf[i], tot);
        float acc[NCOLS];
        const float d = step_acc<NCOLS>(buf[i], lane, sl, c, acc);
#pragma unroll
        for (int col = 0; col < NCOLS; ++col) tot[col] = __builtin_fmaf(d, acc[col], tot[col]);
        if (i + PD < T) {
            __builtin_amdgcn_sched_barrier(0);
            issue(i + PD);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (c == NCH - 1) {
            const int lqd = QPW * w + j;   // the quad within the workgroup: group lqd / 16, rows 4 (lqd % 16) + r
#pragma unroll
            for (int col = 0; col < NCOLS; ++col) {
                const float v = hb_sum(tot[col]);
                tot[col] = 0.0f;
                if (lane < kQuad) lrow[((lqd >> 4) * NCOLS + col) * 64 + 4 * (lqd & 15) + lane] = v;
            }
        }
    }
    __syncthreads();
    // wave g: lanes 32 c .. 32 c + 31 quantize column c's 32 outputs of group g
    if (w < GPW && (lane >> 5) < NCOLS) {
        const int col = lane >> 5, i = lane & 31;
        const float* rows = lrow + (w * NCOLS + col) * 64;
        const float a = silu(rows[i]) * rows[32 + i];
        q8_1_store_lane(a, out + (static_cast<size_t>(col) * (ff / 32) + GPW * blockIdx.x + w) * kQ8_1Bytes);
    }
}

// ---- ingest GEMM: 8 / 16 columns on the 16-block 4x4x4 int8 MFMA -------------------------------------------------
// Same wave tiles, lane ownership and fp32 arithmetic as q6k_packed_gemv, with the integer dot products on the matrix
// cores.  MFMA block b = half-block hb (lanes 4 hb .. 4 hb + 3), A row i = quad row i (the lane's own unpacked
// weights), B column j = activation column 4 cg + j, and D[i][j] lands in lane 4 hb + j, register i (layout of
// v_mfma_i32_4x4x4_16b_i8).  One 16-element sub-block is four MFMAs over its four K-quads starting from 0: the exact
// int32 sum the sdot4 chain forms.  The epilogue then repeats the decode kernel's operations in its order - corr + sum,
// the two sub-scales by __mul24, fma(d8, sd, acc) over k = 0, 2, 1, 3, fma(d, acc, tot) per tile, the hb butterfly -
// so every column is bitwise the single-column GEMV.  The quad's sub-scales and block scales reach the column lanes by
// quad broadcasts.
//
// Stage: per (column group cg, block jb) 13 uint4 = [codes 0..15 of columns 4 cg + 0..3 | codes 16..31 | records
// {-32 sum(q[0:16]), -32 sum(q[16:32]), d8, 0} | pad]; the pad makes a half-block step 832 bytes, so the 16 lanes of
// one LDS pass (4 half-blocks x 4 columns) hit distinct banks.
constexpr int kMStride = 13;   // uint4 per (cg, block)

// one Q8_1 block (its 9 dwords) into the MFMA stage at (column col, staged block jb), nbs staged blocks per column
__device__ __forceinline__ void stage_one_mfma(const uint32_t (&wv)[9], int col, int jb, int nbs, uint4* st) {
    int s0 = 0, s1 = 0;
#pragma unroll
    for (int i = 1; i <= 4; ++i) s0 = sdot4(static_cast<int>(wv[i]), 0x01010101, s0);
#pragma unroll
    for (int i = 5; i <= 8; ++i) s1 = sdot4(static_cast<int>(wv[i]), 0x01010101, s1);
    uint4* q = st + static_cast<size_t>((col >> 2) * nbs + jb) * kMStride + (col & 3);
    q[0] = make_uint4(wv[1], wv[2], wv[3], wv[4]);
    q[4] = make_uint4(wv[5], wv[6], wv[7], wv[8]);
    q[8] = make_uint4(static_cast<uint32_t>(-32 * s0), static_cast<uint32_t>(-32 * s1),
                      __float_as_uint(half_bits_to_float(wv[0])), 0u);
}

// KP = 2: the second half of the blocks, held in registers (up to kPhaseRegs blocks per lane) until the phase switch
constexpr int kPhaseRegs = 6;

// value of lane 4 (l / 4) + i (a broadcast inside each group of four lanes)
template <int I>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), I | (I << 2) | (I << 4) | (I << 6), 0xf,
                                                          0xf, false));
}

// CS = 2: the two waves of a pair share a quad and split its columns (each runs NCG / 2 column groups over the same
// weight tiles, the second load an L2 hit), so a shape with fewer quads than the grid's waves still fills every CU;
// a column's arithmetic is unchanged.
// KP = 2: the stage holds half of the row (a 16-column stage of a 12288-wide row is 320 KB against the CU's 160 KB).
// Each wave pair owns one quad (clamped past the last, its stores skipped), runs the first half's chunks, and at the
// half every wave of the workgroup meets at a barrier, the second half (loaded into registers at the start) replaces
// the first in the stage, and the chunks go on: one weight pass for 16 columns where two 8-column passes read the
// weights twice, and the fma chain over the chunks runs in the same order.
// LE: the quad's row sums through LDS - each lane parks its 4 x NCW (row, column group) sums of its half-block, and
// lane (row i, group g, column jj) adds its 16 half-blocks in the xor butterfly's tree (bitwise hb_sum), then owns one
// output: ~60 instructions per quad where the 16 in-register butterflies take ~300.  Needs 4 KB x NCW of LDS per wave:
// after the stage, or with two K halves the stage itself once every wave is past its last chunk.
template <int NCG, bool RES, int D, int CS = 1, int KP = 1, int NCHK = 0, bool LE = false>
__global__ __launch_bounds__(64 * kWideWaves) void q6k_packed_mfma(const uint8_t* __restrict__ wp,
                                                                   const uint8_t* __restrict__ x, float* y,
                                                                   const float* res, float* partials, int n_in,
                                                                   int n_out) {
    typedef int i32x4 __attribute__((ext_vector_type(4)));
    static_assert(CS == 1 || CS == 2, "column split: one or two waves per quad");
    static_assert(KP == 1 || (KP == 2 && CS == 2 && NCHK % 2 == 0 && NCHK > 0), "two K halves: a wave pair per quad");
    static_assert(!LE || NCG / CS <= 4, "LDS row sums: at most 64 outputs per wave");
    constexpr int NCW = NCG / CS;            // column groups of this wave
    constexpr int PG = NCW >= 2 ? 2 : 1;     // column groups per MFMA batch
    extern __shared__ uint4 smem[];   // the stage may take all 160 KB of the CU's LDS: no static LDS
    const int t = threadIdx.x, lane = t & 63;
    const int nch = n_in / kChunkElems;
    const int nbt = n_in / 32;
    const int nq = (n_out + kQuad - 1) / kQuad;
    const int wv = t >> 6, half = CS == 1 ? 0 : (wv & 1);
    const int GW = static_cast<int>(gridDim.x) * (kWideWaves / CS);
    const int gw = static_cast<int>(blockIdx.x) * (kWideWaves / CS) + (CS == 1 ? wv : (wv >> 1));
    // KP = 2: every wave runs one quad's chunks (a pair past the last quad reads the last one's tiles and stores
    // nothing), so every wave meets the phase barrier
    const int my_quads = KP == 2 ? 1 : gw < nq ? (nq - 1 - gw) / GW + 1 : 0;
    const int nsteps = my_quads * nch;
    const int nbs = nbt / KP, cpp = KP == 2 ? NCHK / 2 : nch;   // staged blocks per column, chunks per phase

    // the first kStageRegs activation blocks of each lane go out ahead of the weight tiles (a wave's loads return in
    // issue order: a stage loaded after the tiles waits for them)
    constexpr int kStageRegs = 4;
    const int nb_stage = 4 * NCG * (KP == 2 ? nbs : nbt);
    const int nbs_stage = KP == 2 ? nbs : nbt;
    uint32_t sv[kStageRegs][9];
#pragma unroll
    for (int m = 0; m < kStageRegs; ++m) {
        const int J = min(t + 64 * kWideWaves * m, nb_stage - 1);
        const int col = J / nbs_stage, jb = J - col * nbs_stage;
        const uint32_t* p = reinterpret_cast<const uint32_t*>(x + static_cast<size_t>(col * nbt + jb) * kQ8_1Bytes);
#pragma unroll
        for (int i = 0; i < 9; ++i) sv[m][i] = p[i];
    }
    __builtin_amdgcn_sched_barrier(0);

    WTile buf[D];
    auto issue = [&](int f, WTile& b) {
        const int qi = f / nch, c = f - qi * nch;
        const int qq = KP == 2 ? min(gw, nq - 1) : min(gw + qi * GW, nq - 1);   // clamped: the prefetch below
        const uint8_t* base = wp + (static_cast<size_t>(qq) * nch + c) * kWaveTile;
#pragma unroll
        for (int u = 0; u < 4; ++u)
            b.ql[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + u * 1024 + 16 * lane));
#pragma unroll
        for (int u = 0; u < 2; ++u)
            b.qh[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + 4096 + u * 1024 + 16 * lane));
        b.sc = *reinterpret_cast<const uint2*>(base + 6144 + 8 * lane);
        b.d = *reinterpret_cast<const uint16_t*>(base + 6656 + 2 * (4 * (lane >> 3) + (lane & 3)));
    };
    // unconditional (a wave with fewer steps re-reads its last, or the grid's last quad's, tile and discards it): with
    // the loads under a branch the wait for the staged blocks below would also cover the tiles
#pragma unroll
    for (int s = 0; s < D; ++s) issue(min(s, max(nsteps - 1, 0)), buf[s]);

    // the blocks held in registers (lanes past the last block rewrite its slot with the same bytes), then the rest
#pragma unroll
    for (int m = 0; m < kStageRegs; ++m) {
        const int J = min(t + 64 * kWideWaves * m, nb_stage - 1);
        const int col = J / nbs_stage, jb = J - col * nbs_stage;
        stage_one_mfma(sv[m], col, jb, nbs_stage, smem);
    }
    for (int J = t + 64 * kWideWaves * kStageRegs; J < nb_stage; J += 64 * kWideWaves) {
        const int col = J / nbs_stage, jb = J - col * nbs_stage;
        const uint32_t* p = reinterpret_cast<const uint32_t*>(x + static_cast<size_t>(col * nbt + jb) * kQ8_1Bytes);
        uint32_t wv[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) wv[i] = p[i];
        stage_one_mfma(wv, col, jb, nbs_stage, smem);
    }
    // KP = 2: the second half's blocks, loaded one step before the switch (into registers the tiles leave free) and
    // staged at the switch
    uint32_t pb[KP == 2 ? kPhaseRegs : 1][9];
    auto load_half = [&]() {
        const int nb = 4 * NCG * nbs;
#pragma unroll
        for (int m = 0; m < kPhaseRegs; ++m) {
            const int J = min(t + 64 * kWideWaves * m, nb - 1);
            const int col = J / nbs, jb = J - col * nbs;
            const uint32_t* p =
                reinterpret_cast<const uint32_t*>(x + static_cast<size_t>(col * nbt + nbs + jb) * kQ8_1Bytes);
#pragma unroll
            for (int i = 0; i < 9; ++i) pb[m][i] = p[i];
        }
    };
    __syncthreads();

    const int jj = lane & 3, hb = lane >> 2, b = hb >> 1, n = hb & 1;
    // stage offsets (uint4 units, 32-bit): the wave's column group g (group NCW half + g of the stage) at goff[g], the
    // lane's column and half-block at lbase
    int goff[NCW];
#pragma unroll
    for (int g = 0; g < NCW; ++g) goff[g] = (NCW * half + g) * nbs * kMStride;
    const int lbase = (8 * b + 4 * n) * kMStride + jj;
    // LE: this wave's row-sum scratch, after the stage; with two K halves, the stage itself once every wave is past
    // its last chunk (the rows complete at the last step of the straight-line chunk order, the same for every wave)
    constexpr bool LEA = LE && KP == 2;
    float* lescr = reinterpret_cast<float*>(smem + (LEA ? 0 : static_cast<size_t>(NCG) * nbs * kMStride)) +
                   wv * (64 * 4 * NCW);
    float tot[4][NCW];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int g = 0; g < NCW; ++g) tot[i][g] = 0.0f;

    // one (quad, chunk) step on tile buffer s
    auto step = [&](const int f, const int s) {
        const int qi = f / nch, c = f - qi * nch;
        const int cs = KP == 2 && c >= cpp ? c - cpp : c;   // the chunk within the staged half
        const WTile wt = buf[s];
        if (f + D < nsteps) issue(f + D, buf[s]);

        uint32_t Q[16], H[8];
#pragma unroll
        for (int i = 0; i < 16; ++i) Q[i] = wt.ql[i >> 2][i & 3];
#pragma unroll
        for (int i = 0; i < 8; ++i) H[i] = wt.qh[i >> 2][i & 3];
        // the quad's four rows: sub-scale words and block scales
        uint32_t S0[4], S1[4];
        float dr[4];
        S0[0] = quad_bcast<0>(wt.sc.x); S0[1] = quad_bcast<1>(wt.sc.x);
        S0[2] = quad_bcast<2>(wt.sc.x); S0[3] = quad_bcast<3>(wt.sc.x);
        S1[0] = quad_bcast<0>(wt.sc.y); S1[1] = quad_bcast<1>(wt.sc.y);
        S1[2] = quad_bcast<2>(wt.sc.y); S1[3] = quad_bcast<3>(wt.sc.y);
        dr[0] = half_bits_to_float(quad_bcast<0>(wt.d)); dr[1] = half_bits_to_float(quad_bcast<1>(wt.d));
        dr[2] = half_bits_to_float(quad_bcast<2>(wt.d)); dr[3] = half_bits_to_float(quad_bcast<3>(wt.d));

        float acc[4][NCW];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int g = 0; g < NCW; ++g) acc[i][g] = 0.0f;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
            for (int kh = 0; kh < 2; ++kh) {
                const int k = kk + 2 * kh;
                int v[8];
#pragma unroll
                for (int ww = 0; ww < 8; ++ww)
                    v[ww] = static_cast<int>(((Q[8 * kk + ww] >> (4 * kh)) & 0x0f0f0f0fu) |
                                             (((H[ww] >> (2 * k)) & 0x03030303u) << 4));
                // two column groups at a time: their codes and records first, then the four independent MFMA
                // chains interleaved, then the epilogues (no chain waits on its own loads or results)
                const int lo = lbase + (cs * kNB + k) * kMStride;
#pragma unroll
                for (int g0 = 0; g0 < NCW; g0 += PG) {
                    uint4 qa[PG], qb[PG], rec[PG];
#pragma unroll
                    for (int h = 0; h < PG; ++h) {
                        qa[h] = smem[goff[g0 + h] + lo];
                        qb[h] = smem[goff[g0 + h] + lo + 4];
                        rec[h] = smem[goff[g0 + h] + lo + 8];
                    }
                    i32x4 d0[PG], d1[PG];
#pragma unroll
                    for (int h = 0; h < PG; ++h) d0[h] = d1[h] = i32x4{0, 0, 0, 0};
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq) {
#pragma unroll
                        for (int h = 0; h < PG; ++h) {
                            d0[h] = __builtin_amdgcn_mfma_i32_4x4x4i8(v[qq], static_cast<int>(qa[h][qq]), d0[h], 0,
                                                                      0, 0);
                            d1[h] = __builtin_amdgcn_mfma_i32_4x4x4i8(v[4 + qq], static_cast<int>(qb[h][qq]), d1[h],
                                                                      0, 0, 0);
                        }
                    }
#pragma unroll
                    for (int h = 0; h < PG; ++h) {
                        const float d8 = __uint_as_float(rec[h].z);
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int sc0 = sc_byte2(S0[i], S1[i], 2 * k), sc1 = sc_byte2(S0[i], S1[i], 2 * k + 1);
                            const int sd = __mul24(sc0, d0[h][i] + static_cast<int>(rec[h].x)) +
                                           __mul24(sc1, d1[h][i] + static_cast<int>(rec[h].y));
                            acc[i][g0 + h] = __builtin_fmaf(d8, static_cast<float>(sd), acc[i][g0 + h]);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int g = 0; g < NCW; ++g) tot[i][g] = __builtin_fmaf(dr[i], acc[i][g], tot[i][g]);

        if constexpr (LEA) {
            if (c == nch - 1) __syncthreads();   // the stage's last reads are done: the row sums may overwrite it
        }
        if (c == nch - 1 && (KP == 1 || gw < nq)) {   // the quad's rows are complete
            const int q = gw + qi * GW;
            const int np = (n_out + 3) / 4;
            if constexpr (LE) {
                constexpr int R = 4 * NCW;   // the lane's sums: [row i][group g] at i NCW + g
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int g = 0; g < NCW; ++g) {
                        lescr[lane * R + i * NCW + g] = tot[i][g];
                        tot[i][g] = 0.0f;
                    }
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                // lane o: row io = o / R, group go = (o / 4) % NCW, column jo = o % 4 (lanes past 16 NCW idle)
                const bool live = lane < 4 * R;
                const int oo = live ? lane : 0;
                const int io = oo / R, go = (oo >> 2) % NCW, jo = oo & 3;
                float hv[16];
#pragma unroll
                for (int h = 0; h < 16; ++h) hv[h] = lescr[(4 * h + jo) * R + io * NCW + go];
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // read out before the next quad's sums land
                // the xor butterfly of hb_sum (partners hb ^ 8, ^ 4, ^ 2, ^ 1), evaluated for half-block 0
                float a8[8], a4[4], a2[2];
#pragma unroll
                for (int h = 0; h < 8; ++h) a8[h] = hv[h] + hv[h + 8];
#pragma unroll
                for (int h = 0; h < 4; ++h) a4[h] = a8[h] + a8[h + 4];
#pragma unroll
                for (int h = 0; h < 2; ++h) a2[h] = a4[h] + a4[h + 2];
                float v = a2[0] + a2[1];
                const int row = kQuad * q + io, col = 4 * (NCW * half + go) + jo;
                if constexpr (RES) {
                    if (live && row < n_out) v += res[static_cast<size_t>(col) * n_out + row];
                }
                if (live && row < n_out) y[static_cast<size_t>(col) * n_out + row] = v;
                if constexpr (RES) {
                    // the quad's four rows of this column sit R lanes apart: squares in row order
                    const float v1 = xor_lane<R>(v);
                    const float v2 = xor_lane<2 * R>(v);
                    const float v3 = xor_lane<2 * R>(v1);
                    if (live && io == 0) {
                        const int row0 = kQuad * q;
                        float p = __builtin_fmaf(v, v, 0.0f);
                        if (row0 + 1 < n_out) p = __builtin_fmaf(v1, v1, p);
                        if (row0 + 2 < n_out) p = __builtin_fmaf(v2, v2, p);
                        if (row0 + 3 < n_out) p = __builtin_fmaf(v3, v3, p);
                        partials[static_cast<size_t>(col) * np + q] = p;
                    }
                }
            } else {
#pragma unroll
                for (int g = 0; g < NCW; ++g) {
                    const int col = 4 * (NCW * half + g) + jj;
                    float v[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        v[i] = hb_sum(tot[i][g]);
                        tot[i][g] = 0.0f;
                        const int row = kQuad * q + i;
                        if constexpr (RES) {
                            if (row < n_out) v[i] += res[static_cast<size_t>(col) * n_out + row];
                        }
                        if (hb == 0 && row < n_out) y[static_cast<size_t>(col) * n_out + row] = v[i];
                    }
                    if constexpr (RES) {
                        if (hb == 0) {   // squares of the quad's rows in row order
                            const int row0 = kQuad * q;
                            float p = __builtin_fmaf(v[0], v[0], 0.0f);
                            if (row0 + 1 < n_out) p = __builtin_fmaf(v[1], v[1], p);
                            if (row0 + 2 < n_out) p = __builtin_fmaf(v[2], v[2], p);
                            if (row0 + 3 < n_out) p = __builtin_fmaf(v[3], v[3], p);
                            partials[static_cast<size_t>(col) * np + q] = p;
                        }
                    }
                }
            }
        }
    };
    if constexpr (KP == 1) {
        for (int f0 = 0; f0 < nsteps; f0 += D) {
#pragma unroll
            for (int s = 0; s < D; ++s) {
                const int f = f0 + s;
                if (f >= nsteps) break;   // uniform across the wave
                step(f, s);
            }
        }
    } else {
        // NCHK chunks in straight-line code: the second half's registers are live only across the last step of the
        // first half
#pragma unroll
        for (int f = 0; f < NCHK; ++f) {
            if (f == NCHK / 2 - 1) load_half();
            if (f == NCHK / 2) {
                __syncthreads();   // the first half's stage is read out
                const int nb = 4 * NCG * nbs;
#pragma unroll
                for (int m = 0; m < kPhaseRegs; ++m) {
                    const int J = t + 64 * kWideWaves * m;
                    if (J < nb) stage_one_mfma(pb[m], J / nbs, J - (J / nbs) * nbs, nbs, smem);
                }
                __syncthreads();
            }
            step(f, f % D);
        }
    }
}

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

// waves: at most per_cu workgroups per CU, and an even split of the quads over them.  32 gives every matrix up to
// 32768 quads one quad per wave (all its tiles in flight from the start; the lm_head gets two): measured in the 9B
// round, 4 -> 8 -> 32 workgroups per CU took it from 2758 to 2727 to 2712 us.
int packed_grid(int nq) {
    static const int per_cu = env_int("RMI_PACKED_PER_CU", 32);
    const int max_waves = std::max(1, per_cu) * cu_count() * (kThreads / 64);
    const int qpw = (nq + max_waves - 1) / max_waves;
    const int waves = (nq + qpw - 1) / qpw;
    return (waves + 3) / 4;
}

// Kernel choice for one or two columns (more columns, and shapes without an entry, run the pipelined loop kernel).
// Measured per launch at two columns (one column in brackets) against the loop kernel:
//   n_in 4096:  the stream kernel, one quad per wave up to 4096 quads: 4096 rows 6.80 -> 4.93 us, 12288 rows one
//               column with the residual 8.9 -> 8.6 us against a form that split a quad's two chunks over two waves
//               (once the staged blocks were loaded outside a branch; 10240 / 12352 rows two columns the same either
//               way); 24576 rows 16.6 -> 16.1 us (15.5 -> 14.8) and the 248320-row lm_head 123.9 -> 117.7 us (two
//               quads per wave, both tiles of the next quad issued while the current one is summed; three: 16.2 us)
//   n_in 8192:  4096 rows 9.15 -> 8.19 us (stream, one quad per wave, two tiles ahead: one workgroup per CU; a quad's
//               four chunks on two waves of one workgroup, two workgroups per CU, 8.64 us)
//   n_in 12288: 4096 rows 11.8 -> 10.4 us (10.5 -> 9.6) (stream, one quad per wave, two tiles ahead; three ahead
//               10.8 us, all six 13.2 us, two quads per wave 13.8 us, a quad on two waves 11.2 us)
// RMI_PACKED_KERNEL=loop runs the loop kernel for every shape.
struct PackedCfg {
    enum Kind { kLoop, kStream } kind;
};

PackedCfg packed_cfg(int n_in, int n_out, int ncols) {
    static const bool loop_only = [] {
        const char* v = std::getenv("RMI_PACKED_KERNEL");
        return v && std::string(v) == "loop";
    }();
    const int nch = n_in / kChunkElems;
    if (loop_only || ncols > 2) return {PackedCfg::kLoop};
    if (nch == 2 || nch == 4 || nch == 6) return {PackedCfg::kStream};
    return {PackedCfg::kLoop};
}

template <int NCOLS, bool RES, int NCH, int QPW, int NW, int PD>
void launch_stream(const uint8_t* wp, const uint8_t* x, float* y, const float* res, float* partials, int n_in,
                   int n_out, hipStream_t s) {
    const int nq = (n_out + kQuad - 1) / kQuad;
    const dim3 grid((nq + NW * QPW - 1) / (NW * QPW)), block(64 * NW);
    hipLaunchKernelGGL((q6k_packed_gemv_stream<NCOLS, RES, NCH, QPW, NW, PD>), grid, block,
                       static_cast<size_t>(NCOLS) * (n_in / 32) * 48, s, wp, x, y, res, partials, n_in, n_out, NormIn{});
}

template <int NCOLS, bool RES>
void launch_packed(const uint8_t* wp, const uint8_t* x, float* y, const float* res, float* partials, int n_in,
                   int n_out, hipStream_t s) {
    static const int depth = env_int("RMI_PACKED_DEPTH", 2);
    if constexpr (NCOLS <= 2) {
        const PackedCfg c = packed_cfg(n_in, n_out, NCOLS);
        if (c.kind == PackedCfg::kStream) {
            if (n_in / kChunkElems == 2) {   // one quad per wave up to 4096 quads, two above (the lm_heads)
                if ((n_out + kQuad - 1) / kQuad <= 4096)
                    return launch_stream<NCOLS, RES, 2, 1, 4, 2>(wp, x, y, res, partials, n_in, n_out, s);
                return launch_stream<NCOLS, RES, 2, 2, 4, 2>(wp, x, y, res, partials, n_in, n_out, s);
            }
            if (n_in / kChunkElems == 4)
                return launch_stream<NCOLS, RES, 4, 1, 4, 2>(wp, x, y, res, partials, n_in, n_out, s);
            return launch_stream<NCOLS, RES, 6, 1, 4, 2>(wp, x, y, res, partials, n_in, n_out, s);
        }
    }
    const int nq = (n_out + kQuad - 1) / kQuad;
    const size_t lds = static_cast<size_t>(NCOLS) * (n_in / 32) * 48;
    const dim3 grid(packed_grid(nq)), block(kThreads);
    if (depth >= 4)
        hipLaunchKernelGGL((q6k_packed_gemv<NCOLS, RES, 4, 4>), grid, block, lds, s, wp, x, y, res, partials, n_in,
                           n_out);
    else if (depth == 3)
        hipLaunchKernelGGL((q6k_packed_gemv<NCOLS, RES, 3, 4>), grid, block, lds, s, wp, x, y, res, partials, n_in,
                           n_out);
    else
        hipLaunchKernelGGL((q6k_packed_gemv<NCOLS, RES, 2, 4>), grid, block, lds, s, wp, x, y, res, partials, n_in,
                           n_out);
}

// LDS of the ingest stage: kMStride uint4 per (4-column group, block)
size_t wide_stage_bytes(int n_in, int ncols) {
    return static_cast<size_t>(ncols / 4) * (n_in / 32) * kMStride * 16;
}

// 16 columns whose stage is too wide for the LDS in two K halves (q6k_packed_mfma KP = 2): an even chunk count, half
// the stage in the LDS and the other half in kPhaseRegs blocks per lane, a wave pair per quad at most
bool wide_halves(int n_in, int n_out) {
    const int nch = n_in / kChunkElems, nq = (n_out + kQuad - 1) / kQuad;
    static const bool on = env_int("RMI_WIDE_HALVES", 1) != 0;
    return on && (nch == 4 || nch == 6) && wide_stage_bytes(n_in, 16) / 2 <= kWideStageBytes &&
           16 * (n_in / 64) <= 64 * kWideWaves * kPhaseRegs && nq <= cu_count() * (kWideWaves / 2);
}

// the widest ingest pass (16 or 8 columns) whose stage fits kWideStageBytes (16 also in two K halves), or 0
int wide_cols(int n_in, int n_out, int remaining) {
    if (remaining >= 16 && (wide_stage_bytes(n_in, 16) <= kWideStageBytes || wide_halves(n_in, n_out))) return 16;
    if (remaining >= 8 && wide_stage_bytes(n_in, 8) <= kWideStageBytes) return 8;
    return 0;
}

// 8 / 16 columns in one weight pass on the MFMA ingest kernel: one 8-wave workgroup per CU (the stage takes up to
// 160 KB of LDS), the quads split evenly over the waves
// workgroups of a grid whose quad units (one per wave, or per pair of waves at CS = 2) spread evenly over the CUs
int wide_grid(int nq, int units_per_wg) {
    const int max_units = cu_count() * units_per_wg;
    const int qpu = (nq + max_units - 1) / max_units;
    const int units = (nq + qpu - 1) / qpu;
    return (units + units_per_wg - 1) / units_per_wg;
}

template <int NCOLS, bool RES>
int launch_packed_wide(const uint8_t* wp, const uint8_t* x, float* y, const float* res, float* partials, int n_in,
                       int n_out, hipStream_t s) {
    constexpr int D = 3;
    constexpr int NCG = NCOLS / 4;
    auto kern = q6k_packed_mfma<NCG, RES, D>;
    auto kern2 = q6k_packed_mfma<NCG, RES, D, 2>;
    auto kernl = q6k_packed_mfma<NCG, RES, D, 1, 1, 0, true>;
    auto kern2l = q6k_packed_mfma<NCG, RES, D, 2, 1, 0, true>;
    auto lds_attr = [](auto k) {
        return hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                                   kWideStageBytes) == hipSuccess;
    };
    static const bool attr = lds_attr(kern) && lds_attr(kern2) && lds_attr(kernl) && lds_attr(kern2l);
    if (!attr) return fail(RMI_ERR_LAUNCH, "native_q6_k_mmvq_packed: wide LDS stage not available");
    // the LDS row sums (LE) where their scratch, 4 KB per column group of a wave, fits after the stage
    static const bool le_on = env_int("RMI_WIDE_LE", 1) != 0;
    auto le_bytes = [](int ncw) { return static_cast<size_t>(kWideWaves) * 64 * 4 * ncw * sizeof(float); };
    const int nq = (n_out + kQuad - 1) / kQuad;
    const size_t lds = wide_stage_bytes(n_in, NCOLS);
    if (lds > kWideStageBytes) {
        if constexpr (NCOLS == 16) {
            // two K halves, a wave pair per quad (the second half's blocks take 54 registers: one tile fewer in flight)
            // (the LDS row sums reuse the stage after the last chunk)
            auto kh4 = q6k_packed_mfma<4, RES, 2, 2, 2, 4, true>;
            auto kh6 = q6k_packed_mfma<4, RES, 2, 2, 2, 6, true>;
            static const bool attr_h = lds_attr(kh4) && lds_attr(kh6);
            if (!attr_h) return fail(RMI_ERR_LAUNCH, "native_q6_k_mmvq_packed: wide LDS stage not available");
            if (wide_halves(n_in, n_out)) {
                const dim3 grid((nq + kWideWaves / 2 - 1) / (kWideWaves / 2)), block(64 * kWideWaves);
                if (lds / 2 < le_bytes(2)) return fail(RMI_ERR_SHAPE, "native_q6_k_mmvq_packed: half stage too small");
                if (n_in / kChunkElems == 4)
                    hipLaunchKernelGGL(kh4, grid, block, lds / 2, s, wp, x, y, res, partials, n_in, n_out);
                else if (n_in / kChunkElems == 6)
                    hipLaunchKernelGGL(kh6, grid, block, lds / 2, s, wp, x, y, res, partials, n_in, n_out);
                else
                    return fail(RMI_ERR_SHAPE, "native_q6_k_mmvq_packed: wide stage exceeds the LDS");
                return RMI_OK;
            }
        }
        return fail(RMI_ERR_SHAPE, "native_q6_k_mmvq_packed: wide stage exceeds the LDS");
    }
    // a wave per quad unit; when that leaves CUs idle (fewer quads than the CUs' waves: the 4096-row outputs), the
    // column-split form, a pair of waves per quad, on up to twice the workgroups
    static const bool split_on = env_int("RMI_WIDE_SPLIT", 1) != 0;
    const int g1 = wide_grid(nq, kWideWaves), g2 = wide_grid(nq, kWideWaves / 2);
    const dim3 block(64 * kWideWaves);
    if (split_on && 4 * g1 < 3 * cu_count() && g2 > g1) {
        const size_t l2 = lds + le_bytes(NCG / 2);
        if (le_on && NCG >= 2 && l2 <= kWideStageBytes)
            hipLaunchKernelGGL(kern2l, dim3(g2), block, l2, s, wp, x, y, res, partials, n_in, n_out);
        else
            hipLaunchKernelGGL(kern2, dim3(g2), block, lds, s, wp, x, y, res, partials, n_in, n_out);
    } else {
        const size_t l1 = lds + le_bytes(NCG);
        if (le_on && l1 <= kWideStageBytes)
            hipLaunchKernelGGL(kernl, dim3(g1), block, l1, s, wp, x, y, res, partials, n_in, n_out);
        else
            hipLaunchKernelGGL(kern, dim3(g1), block, lds, s, wp, x, y, res, partials, n_in, n_out);
    }
    return RMI_OK;
}

// columns per narrow pass: at most 4, and the pass's staged activations within kMaxStageBytes
int cols_per_pass(int n_in) {
    const int per = kMaxStageBytes / ((n_in / 32) * 48);
    return std::max(1, std::min(4, per));
}

// Columns are cut into passes (16 or 8 wide, then up to 4); each pass reads the weights once.  The pass width never
// changes a column's result: lane ownership and reduction order depend on the shape only.
template <bool RES>
int run_packed(const void* wpv, const void* xv, float* y, const float* res, float* partials, int n_in, int n_out,
               int ncols, hipStream_t s) {
    const auto* wp = static_cast<const uint8_t*>(wpv);
    const auto* x = static_cast<const uint8_t*>(xv);
    const int per = cols_per_pass(n_in);
    const size_t xcol = static_cast<size_t>(n_in / 32) * kQ8_1Bytes;
    const size_t pcol = static_cast<size_t>((n_out + 3) / 4);
    for (int j = 0; j < ncols;) {
        const int wide = wide_cols(n_in, n_out, ncols - j);
        const int nj = wide ? wide : std::min(per, ncols - j);
        const uint8_t* xj = x + j * xcol;
        float* yj = y + static_cast<size_t>(j) * n_out;
        const float* rj = RES ? res + static_cast<size_t>(j) * n_out : nullptr;
        float* pj = RES ? partials + j * pcol : nullptr;
        switch (nj) {
            case 1: launch_packed<1, RES>(wp, xj, yj, rj, pj, n_in, n_out, s); break;
            case 2: launch_packed<2, RES>(wp, xj, yj, rj, pj, n_in, n_out, s); break;
            case 3: launch_packed<3, RES>(wp, xj, yj, rj, pj, n_in, n_out, s); break;
            case 4: launch_packed<4, RES>(wp, xj, yj, rj, pj, n_in, n_out, s); break;
            case 8:
                if (const int rc = launch_packed_wide<8, RES>(wp, xj, yj, rj, pj, n_in, n_out, s)) return rc;
                break;
            default:
                if (const int rc = launch_packed_wide<16, RES>(wp, xj, yj, rj, pj, n_in, n_out, s)) return rc;
                break;
        }
        if (const int rc = launch_status("native_q6_k_mmvq_packed")) return rc;
        j += nj;
    }
    return RMI_OK;
}

int validate_packed(const void* wp, const void* x, const float* y, int n_in, int n_out, int ncols, void* stream) {
    if (n_in <= 0 || n_in % kChunkElems != 0 || (n_in / 32) * 48 > kMaxStageBytes)
        return fail(RMI_ERR_SHAPE, "packed Q6_K GEMV requires n_in a multiple of 2048 and at most 43690");
    if (ncols < 1 || ncols > kMaxCols) return fail(RMI_ERR_SHAPE, "native MMVQ requires 1 <= ncols <= 16");
    if (n_out <= 0) return fail(RMI_ERR_SHAPE, "native MMVQ requires n_out > 0");
    if (!aligned16(wp) || !aligned4(x) || !aligned4(y))
        return fail(RMI_ERR_POINTER, "packed Q6_K GEMV requires a 16-byte aligned packed matrix and 4-byte aligned x, y");
    if (!stream) return fail(RMI_ERR_STREAM, "native MMVQ requires an explicit non-null CUDA stream");
    return RMI_OK;
}

}  // namespace
}  // namespace rmi

using namespace rmi;

namespace rmi {
namespace {
template <int NCOLS, bool RES, int NCH, int QPW, int NW>
void launch_gguf(const uint8_t* w, const uint8_t* x, float* y, const float* res, float* partials, int n_in, int n_out,
                 hipStream_t s) {
    constexpr int PD = 2;
    const int nq = (n_out + kQuad - 1) / kQuad;
    const size_t lds = static_cast<size_t>(NCOLS) * (n_in / 32) * 48 + static_cast<size_t>(NW) * kGgufWaveDw * 4;
    hipLaunchKernelGGL((q6k_gguf_stream<NCOLS, RES, NCH, QPW, NW, PD>), dim3((nq + NW * QPW - 1) / (NW * QPW)),
                       dim3(64 * NW), lds, s, w, x, y, res, partials, n_in, n_out);
}

// One quad per wave (two tiles in flight), 4-wave workgroups, 8 above 4096 quads.  Measured at two columns (one for
// the config-1 shape) against the 16-row / 8-row tiled kernel: up||gate 24576 x 4096 18.8 us (tiled 19.9-21.3),
// FFN down 4096 x 12288 + residual 12.2 us (13.7), 12288 x 4096 + residual 10.3 us (10.8-11.0).  Two or three quads
// per wave were slower on every shape (with fewer waves the wave's LDS round trips per tile are not hidden).
template <int NCOLS, bool RES, int NCH>
void gguf_nch(const uint8_t* w, const uint8_t* x, float* y, const float* res, float* partials, int n_in, int n_out,
              hipStream_t s) {
    if ((n_out + kQuad - 1) / kQuad > 4096) return launch_gguf<NCOLS, RES, NCH, 1, 8>(w, x, y, res, partials, n_in, n_out, s);
    return launch_gguf<NCOLS, RES, NCH, 1, 4>(w, x, y, res, partials, n_in, n_out, s);
}

template <int NCOLS, bool RES>
int gguf_cols(const uint8_t* w, const uint8_t* x, float* y, const float* res, float* partials, int n_in, int n_out,
              hipStream_t s) {
    const int nch = n_in / kChunkElems;
    if (nch == 2) gguf_nch<NCOLS, RES, 2>(w, x, y, res, partials, n_in, n_out, s);
    else if (nch == 4) gguf_nch<NCOLS, RES, 4>(w, x, y, res, partials, n_in, n_out, s);
    else gguf_nch<NCOLS, RES, 6>(w, x, y, res, partials, n_in, n_out, s);
    return RMI_OK;
}
}  // namespace

// The drop-in entry points' stream kernel over GGUF-layout weights: rows of 2, 4 or 6 chunks (4096, 8192, 12288
// elements), one to four columns, a 16-byte aligned matrix.  Returns -1, launching nothing, for any other shape.
int gguf_stream_gemv(const uint8_t* w, const uint8_t* x, float* y, const float* res, float* partials, int n_in,
                     int n_out, int ncols, hipStream_t s) {
    const int nch = n_in / kChunkElems;
    if (n_in % kChunkElems || (reinterpret_cast<uintptr_t>(w) & 15u) || ncols < 1 || ncols > 4 ||
        !(nch == 2 || nch == 4 || nch == 6))
        return -1;
    switch (ncols) {
        case 1: return res ? gguf_cols<1, true>(w, x, y, res, partials, n_in, n_out, s)
                           : gguf_cols<1, false>(w, x, y, res, partials, n_in, n_out, s);
        case 2: return res ? gguf_cols<2, true>(w, x, y, res, partials, n_in, n_out, s)
                           : gguf_cols<2, false>(w, x, y, res, partials, n_in, n_out, s);
        case 3: return res ? gguf_cols<3, true>(w, x, y, res, partials, n_in, n_out, s)
                           : gguf_cols<3, false>(w, x, y, res, partials, n_in, n_out, s);
        default: return res ? gguf_cols<4, true>(w, x, y, res, partials, n_in, n_out, s)
                            : gguf_cols<4, false>(w, x, y, res, partials, n_in, n_out, s);
    }
}
}  // namespace rmi

extern "C" size_t rmi_q6_k_packed_bytes(int n_in, int n_out) {
    if (n_in <= 0 || n_in % kChunkElems != 0 || n_out <= 0) {
        set_error("q6_k_packed_bytes: n_in must be a positive multiple of 2048 and n_out positive");
        return 0;
    }
    return static_cast<size_t>((n_out + kQuad - 1) / kQuad) * (n_in / kChunkElems) * kWaveTile;
}

namespace rmi {
namespace {
int pack(const void* w, void* w_packed, int n_in, int n_out, int ff, void* stream) {
    const size_t nslots = static_cast<size_t>((n_out + kQuad - 1) / kQuad) * (n_in / kChunkElems) * 64;
    hipLaunchKernelGGL(q6k_pack_kernel, dim3(static_cast<unsigned>((nslots + kThreads - 1) / kThreads)), dim3(kThreads),
                       0, static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(w),
                       static_cast<uint8_t*>(w_packed), n_in, n_out, nslots, ff);
    return launch_status("q6_k_pack");
}
}  // namespace
}  // namespace rmi

extern "C" int rmi_q6_k_pack(const void* w, void* w_packed, int n_in, int n_out, void* stream) {
    if (n_in <= 0 || n_in % kChunkElems != 0 || n_out <= 0)
        return fail(RMI_ERR_SHAPE, "q6_k_pack: n_in must be a positive multiple of 2048 and n_out positive");
    if (!w || !aligned16(w_packed)) return fail(RMI_ERR_POINTER, "q6_k_pack: null weights or misaligned packed buffer");
    return pack(w, w_packed, n_in, n_out, 0, stream);
}

extern "C" int rmi_q6_k_pack_swiglu(const void* w, void* w_packed, int n_in, int n_ff, void* stream) {
    if (n_in <= 0 || n_in % kChunkElems != 0 || n_ff <= 0 || n_ff % 32 != 0)
        return fail(RMI_ERR_SHAPE, "q6_k_pack_swiglu: n_in must be a positive multiple of 2048, n_ff of 32");
    if (!w || !aligned16(w_packed))
        return fail(RMI_ERR_POINTER, "q6_k_pack_swiglu: null weights or misaligned packed buffer");
    return pack(w, w_packed, n_in, 2 * n_ff, n_ff, stream);
}

namespace rmi {
namespace {
// norm: the normed-input form (x_q8_1 unused)
int swiglu_packed(const void* w_packed, const void* x_q8_1, void* y_q8_1, int n_in, int n_ff, int ncols,
                  const NormIn* norm, void* stream) {
    if (n_in != 2 * kChunkElems || n_ff <= 0 || n_ff % 32 != 0 || ncols < 1 || ncols > 2)
        return fail(RMI_ERR_SHAPE, "q6_k_swiglu_packed: n_in must be 4096, n_ff a positive multiple of 32, ncols 1 or 2");
    if (!aligned16(w_packed) || !(norm || aligned4(x_q8_1)) || !aligned4(y_q8_1))
        return fail(RMI_ERR_POINTER, "q6_k_swiglu_packed: null or misaligned pointer");
    if (!stream) return fail(RMI_ERR_STREAM, "native MMVQ requires an explicit non-null CUDA stream");
    const auto* wp = static_cast<const uint8_t*>(w_packed);
    const auto* x = static_cast<const uint8_t*>(x_q8_1);
    auto* y = static_cast<uint8_t*>(y_q8_1);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    // two 32-output groups per 8-wave workgroup (192 workgroups at n_ff 12288: one per CU) when n_ff allows, else one
    // per 4-wave workgroup
    auto go = [&](auto kern, int gpw, int nw) {
        const size_t lds = static_cast<size_t>(ncols) * (n_in / 32) * 48 + static_cast<size_t>(gpw) * ncols * 64 * 4;
        hipLaunchKernelGGL(kern, dim3(n_ff / 32 / gpw), dim3(64 * nw), lds, s, wp, x, y, n_in, n_ff,
                           norm ? *norm : NormIn{});
    };
    const bool two = n_ff % 64 == 0;
    if (norm) {
        if (ncols == 1) two ? go(q6k_packed_swiglu<1, 8, 4, 2, true>, 2, 8) : go(q6k_packed_swiglu<1, 4, 4, 2, true>, 1, 4);
        else two ? go(q6k_packed_swiglu<2, 8, 4, 2, true>, 2, 8) : go(q6k_packed_swiglu<2, 4, 4, 2, true>, 1, 4);
    } else if (ncols == 1) {
        if (two) go(q6k_packed_swiglu<1, 8, 4>, 2, 8);
        else go(q6k_packed_swiglu<1>, 1, 4);
    } else {
        if (two) go(q6k_packed_swiglu<2, 8, 4>, 2, 8);
        else go(q6k_packed_swiglu<2>, 1, 4);
    }
    return launch_status(norm ? "q6_k_swiglu_packed_norm" : "q6_k_swiglu_packed");
}

// the normed-input packed GEMV: rows of 4096, one or two columns, one 8-wave workgroup per 8 QPW quads
template <int NCOLS, int QPW, int NW = 8>
void launch_norm_gemv(const uint8_t* wp, float* y, int n_out, const NormIn& ni, hipStream_t s) {
    const int nq = (n_out + kQuad - 1) / kQuad;
    hipLaunchKernelGGL((q6k_packed_gemv_stream<NCOLS, false, 2, QPW, NW, 2, true>), dim3((nq + NW * QPW - 1) / (NW * QPW)),
                       dim3(64 * NW), static_cast<size_t>(NCOLS) * (2 * kChunkElems / 32) * 48, s, wp, nullptr, y,
                       nullptr, nullptr, 2 * kChunkElems, n_out, ni);
}

// 4-wave workgroups for the normed GEMV where 8-wave ones would leave a quarter of the CUs idle (the attention qkv,
// 10240 rows: 214 workgroups of 3 quads per wave instead of 160 of 2); RMI_NORM_NW4=0 keeps the 8-wave form
bool norm_nw4(int nq) {
    static const bool on = env_int("RMI_NORM_NW4", 1) != 0;
    const int qpw8 = (nq + 8 * cu_count() - 1) / (8 * cu_count());
    const int wgs8 = (nq + 8 * qpw8 - 1) / (8 * qpw8);
    return on && 4 * wgs8 < 3 * cu_count() && (nq + 4 * cu_count() - 1) / (4 * cu_count()) <= 4;
}

}  // namespace
}  // namespace rmi

extern "C" int rmi_native_q6_k_swiglu_packed(const void* w_packed, const void* x_q8_1, void* y_q8_1, int n_in, int n_ff,
                                             int ncols, void* stream) {
    return swiglu_packed(w_packed, x_q8_1, y_q8_1, n_in, n_ff, ncols, nullptr, stream);
}

namespace {
int check_norm_in(const float* x, const float* w_norm, const float* partials) {
    if (!aligned16(x) || !aligned16(w_norm) || !aligned4(partials))
        return fail(RMI_ERR_POINTER, "normed-input GEMV: x and the norm weights 16-byte aligned, partials 4-byte aligned");
    return RMI_OK;
}
}  // namespace

extern "C" int rmi_native_q6_k_swiglu_packed_norm(const void* w_packed, const float* x, const float* w_norm,
                                                  const float* partials, float eps, void* y_q8_1, int n_in, int n_ff,
                                                  int ncols, void* stream) {
    if (int rc = check_norm_in(x, w_norm, partials)) return rc;
    const NormIn ni{x, w_norm, partials, eps};
    return swiglu_packed(w_packed, nullptr, y_q8_1, n_in, n_ff, ncols, &ni, stream);
}

// Whether the normed-input GEMV is the faster way to run norm + GEMV at this shape.  It runs one 8-wave workgroup per
// 16 quads (a CU each), so rows that leave many CUs idle lose to the two launches: measured in pairs led by a residual
// GEMV (graph replay, two columns), 12352 rows 17.6 against 18.2 us, 10240 rows 17.6 against 17.2 us (160 of 256 CUs).
extern "C" int rmi_q6_k_packed_norm_preferred(int n_in, int n_out, int ncols) {
    if (n_in != 2 * kChunkElems || ncols < 1 || ncols > 2 || n_out <= 0 || n_out > 4 * 8 * 4 * 256) return 0;
    const int nq = (n_out + kQuad - 1) / kQuad, qpw = (nq + 8 * cu_count() - 1) / (8 * cu_count());
    const int wgs = (nq + 8 * qpw - 1) / (8 * qpw);
    return 4 * wgs >= 3 * cu_count() || norm_nw4(nq) ? 1 : 0;
}

extern "C" int rmi_native_q6_k_mmvq_packed_norm(const void* w_packed, const float* x, const float* w_norm,
                                                const float* partials, float eps, float* y, int n_in, int n_out,
                                                int ncols, void* stream) {
    if (n_in != 2 * kChunkElems || ncols < 1 || ncols > 2 || n_out <= 0 || n_out > 4 * 8 * 4 * 256)
        return fail(RMI_ERR_SHAPE, "q6_k_mmvq_packed_norm: n_in must be 4096, ncols 1 or 2, 0 < n_out <= 32768");
    if (!aligned16(w_packed) || !aligned4(y)) return fail(RMI_ERR_POINTER, "q6_k_mmvq_packed_norm: null or misaligned pointer");
    if (int rc = check_norm_in(x, w_norm, partials)) return rc;
    if (!stream) return fail(RMI_ERR_STREAM, "native MMVQ requires an explicit non-null CUDA stream");
    const NormIn ni{x, w_norm, partials, eps};
    const auto* wp = static_cast<const uint8_t*>(w_packed);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    // quads per wave: every quad's wave resident at once on the CUs' 8-wave workgroups (one per CU up to 2048 quads)
    const int nq = (n_out + kQuad - 1) / kQuad, qpw = (nq + 8 * cu_count() - 1) / (8 * cu_count());
    auto go = [&](auto one, auto two) { ncols == 1 ? one() : two(); };
    if (norm_nw4(nq)) {
        const int q4 = (nq + 4 * cu_count() - 1) / (4 * cu_count());
        if (q4 <= 1) go([&] { launch_norm_gemv<1, 1, 4>(wp, y, n_out, ni, s); }, [&] { launch_norm_gemv<2, 1, 4>(wp, y, n_out, ni, s); });
        else if (q4 == 2) go([&] { launch_norm_gemv<1, 2, 4>(wp, y, n_out, ni, s); }, [&] { launch_norm_gemv<2, 2, 4>(wp, y, n_out, ni, s); });
        else if (q4 == 3) go([&] { launch_norm_gemv<1, 3, 4>(wp, y, n_out, ni, s); }, [&] { launch_norm_gemv<2, 3, 4>(wp, y, n_out, ni, s); });
        else go([&] { launch_norm_gemv<1, 4, 4>(wp, y, n_out, ni, s); }, [&] { launch_norm_gemv<2, 4, 4>(wp, y, n_out, ni, s); });
        return launch_status("q6_k_mmvq_packed_norm");
    }
    if (qpw <= 1) go([&] { launch_norm_gemv<1, 1>(wp, y, n_out, ni, s); }, [&] { launch_norm_gemv<2, 1>(wp, y, n_out, ni, s); });
    else if (qpw == 2) go([&] { launch_norm_gemv<1, 2>(wp, y, n_out, ni, s); }, [&] { launch_norm_gemv<2, 2>(wp, y, n_out, ni, s); });
    else if (qpw == 3) go([&] { launch_norm_gemv<1, 3>(wp, y, n_out, ni, s); }, [&] { launch_norm_gemv<2, 3>(wp, y, n_out, ni, s); });
    else go([&] { launch_norm_gemv<1, 4>(wp, y, n_out, ni, s); }, [&] { launch_norm_gemv<2, 4>(wp, y, n_out, ni, s); });
    return launch_status("q6_k_mmvq_packed_norm");
}

extern "C" int rmi_native_q6_k_mmvq_packed(const void* w_packed, const void* x_q8_1, float* y, int n_in, int n_out,
                                           int ncols, void* stream) {
    if (int rc = validate_packed(w_packed, x_q8_1, y, n_in, n_out, ncols, stream)) return rc;
    return run_packed<false>(w_packed, x_q8_1, y, nullptr, nullptr, n_in, n_out, ncols,
                             static_cast<hipStream_t>(stream));
}

extern "C" int rmi_native_q6_k_mmvq_packed_res_n(const void* w_packed, const void* x_q8_1, float* y, const float* res,
                                                 float* partials, int n_in, int n_out, int ncols, void* stream) {
    if (int rc = validate_packed(w_packed, x_q8_1, y, n_in, n_out, ncols, stream)) return rc;
    if (!aligned4(res) || !aligned4(partials))
        return fail(RMI_ERR_POINTER, "native MMVQ requires non-null 4-byte aligned device pointers");
    return run_packed<true>(w_packed, x_q8_1, y, res, partials, n_in, n_out, ncols, static_cast<hipStream_t>(stream));
}

// ---- packed copies owned by the library, behind the drop-in entry points -----------------------------------------------
// The reference keeps an opt-in registry of re-laid Q6_K copies keyed by the GGUF weight pointer (native_q6_k_pack,
// mmvq:2930-2960; native_q6_k_mmvq looks it up first, mmvq:2752-2770 and 3629; native_q6_k_unpack frees, mmvq:3042-3048).
// Here the copy is the packed wave-tile layout, and rmi_native_q6_k_mmvq / _res / _res_n run the packed kernels on it:
// the same bits as the GGUF-layout kernels (every kernel of both layouts gives the 16-row tiled kernel's results).
namespace rmi {
namespace {
struct PackedCopy {
    void* packed;
    int n_in, n_out;
};
std::mutex g_reg_mu;
std::unordered_map<const void*, PackedCopy> g_reg;
std::atomic<int> g_reg_size{0};   // an empty registry costs the hot path one relaxed load
}  // namespace

int registry_mmvq(const void* w, const void* x_q8_1, float* y, const float* res, float* partials, int n_in, int n_out,
                  int ncols, void* stream) {
    if (g_reg_size.load(std::memory_order_relaxed) == 0) return -1;
    void* packed = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_reg_mu);
        const auto it = g_reg.find(w);
        if (it == g_reg.end() || it->second.n_in != n_in || it->second.n_out != n_out) return -1;
        packed = it->second.packed;
    }
    const auto s = static_cast<hipStream_t>(stream);
    return res ? run_packed<true>(packed, x_q8_1, y, res, partials, n_in, n_out, ncols, s)
               : run_packed<false>(packed, x_q8_1, y, nullptr, nullptr, n_in, n_out, ncols, s);
}
}  // namespace rmi

extern "C" int rmi_native_q6_k_pack_copy(const void* w, int n_in, int n_out) {
    if (n_in <= 0 || n_in % kChunkElems != 0 || n_out <= 0)
        return fail(RMI_ERR_UNSUPPORTED, "native_q6_k_pack: n_in must be a positive multiple of 2048 and n_out positive");
    if (!aligned4(w)) return fail(RMI_ERR_POINTER, "native_q6_k_pack: null or misaligned weights");
    std::lock_guard<std::mutex> lock(g_reg_mu);
    const auto it = g_reg.find(w);
    if (it != g_reg.end()) {
        if (it->second.n_in == n_in && it->second.n_out == n_out) return RMI_OK;   // packed already
        return fail(RMI_ERR_STATE, "native_q6_k_pack: these weights are packed with another shape");
    }
    // as the reference's copy (synchronous, the caller's weights complete): every stream of the device drains first
    if (hipDeviceSynchronize() != hipSuccess) return fail(RMI_ERR_LAUNCH, "native_q6_k_pack: device synchronize failed");
    void* packed = nullptr;
    if (hipMalloc(&packed, rmi_q6_k_packed_bytes(n_in, n_out)) != hipSuccess) {
        (void) hipGetLastError();
        return fail(RMI_ERR_LAUNCH, "native_q6_k_pack: out of device memory for the packed copy");
    }
    hipStream_t s = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) {
        (void) hipFree(packed);
        return fail(RMI_ERR_LAUNCH, "native_q6_k_pack: cannot create a stream");
    }
    int rc = pack(w, packed, n_in, n_out, 0, s);
    if (rc == RMI_OK && hipStreamSynchronize(s) != hipSuccess) rc = fail(RMI_ERR_LAUNCH, "native_q6_k_pack: pack failed");
    (void) hipStreamDestroy(s);
    if (rc != RMI_OK) {
        (void) hipFree(packed);
        return rc;
    }
    g_reg.emplace(w, PackedCopy{packed, n_in, n_out});
    g_reg_size.store(static_cast<int>(g_reg.size()), std::memory_order_relaxed);
    return RMI_OK;
}

extern "C" int rmi_native_q6_k_unpack(const void* w) {
    std::lock_guard<std::mutex> lock(g_reg_mu);
    const auto it = g_reg.find(w);
    if (it == g_reg.end()) return RMI_OK;
    // the copy may still be read by launches in flight on any stream
    if (hipDeviceSynchronize() != hipSuccess) return fail(RMI_ERR_LAUNCH, "native_q6_k_unpack: device synchronize failed");
    (void) hipFree(it->second.packed);
    g_reg.erase(it);
    g_reg_size.store(static_cast<int>(g_reg.size()), std::memory_order_relaxed);
    return RMI_OK;
}

extern "C" int rmi_native_q6_k_packed_copies(void) {
    return g_reg_size.load(std::memory_order_relaxed);
}
