// mmvq_kquant.hip - Q4_K / Q5_K x Q8_1 GEMV for gfx950 at ncols 1..16, plain and with the residual + sum-of-squares
// epilogue (reference src/native_mmvq.cu: native_q4_k_mmvq 562-640, native_q5_k_mmvq 185-300, native_q4_k_mmvq_res /
// native_q5_k_mmvq_res 3202-3324).  The matrices of Q5_K_M files (qw:1284-1309).
//
// One wave64 per output row, four rows per workgroup.  Lane l owns the sub-block pair p = l % 4 of blocks l / 4,
// l / 4 + 16, ... of its row (elements 64 p .. 64 p + 63: qs bytes [32 p, 32 p + 32), low nibbles sub-block 2 p,
// high nibbles 2 p + 1, Q5_K's fifth bit from qh bit 2 p / 2 p + 1), so one step of the wave reads 16 whole
// consecutive blocks.  The activation row is staged once per workgroup in LDS with each Q8_1 block's code sum.  Per
// block the lane forms the reference's vec_dot expression for its two sub-blocks (vec_dot_q4_K/q5_K_q8_1_impl_vmmq:
// exact int32 dots and code sums, sumf_d = sum d8 (dot sc), sumf_m = sum d8 (sum(u) m)) and adds d sumf_d - dmin
// sumf_m.  A fixed 64-lane butterfly ends the row, so every column of an ncols >= 2 call is bitwise the ncols = 1
// result and the residual variant is bitwise plain + res.
#include "rmi_common.h"

#include <algorithm>

namespace rmi {
namespace {

constexpr int kStageMax = 64 * 1024;   // LDS per workgroup: codes (32 B) + record (8 B) per Q8_1 block and column

__device__ __forceinline__ int byte_of(uint32_t s0, uint32_t s1, uint32_t s2, int i) {
    const uint32_t w = i < 4 ? s0 : i < 8 ? s1 : s2;
    return static_cast<int>((w >> (8 * (i & 3))) & 0xffu);
}

// 6-bit scale and min of sub-block j from the 12 packed bytes (ggml get_scale_min_k4)
__device__ __forceinline__ void scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j, int& sc, int& m) {
    if (j < 4) {
        sc = byte_of(s0, s1, s2, j) & 63;
        m = byte_of(s0, s1, s2, j + 4) & 63;
    } else {
        sc = (byte_of(s0, s1, s2, j + 4) & 15) | ((byte_of(s0, s1, s2, j - 4) >> 6) << 4);
        m = (byte_of(s0, s1, s2, j + 4) >> 4) | ((byte_of(s0, s1, s2, j) >> 6) << 4);
    }
}

// A lane's weight loads for one block (scales, its 32 quant bytes, Q5_K's 32 high-bit bytes)
template <int TYPE>
struct KBlock {
    uint32_t dm, s0, s1, s2;
    uint4 qa, qb, ha, hb;
};

template <int TYPE>
__device__ __forceinline__ void kblock_load(KBlock<TYPE>& k, const uint8_t* blk, int p) {
    constexpr int kQs = TYPE == 13 ? 48 : 16;
    k.dm = *reinterpret_cast<const uint32_t*>(blk);
    k.s0 = *reinterpret_cast<const uint32_t*>(blk + 4);
    k.s1 = *reinterpret_cast<const uint32_t*>(blk + 8);
    k.s2 = *reinterpret_cast<const uint32_t*>(blk + 12);
    k.qa = *reinterpret_cast<const uint4*>(blk + kQs + 32 * p);
    k.qb = *reinterpret_cast<const uint4*>(blk + kQs + 32 * p + 16);
    if constexpr (TYPE == 13) {
        k.ha = *reinterpret_cast<const uint4*>(blk + 16);
        k.hb = *reinterpret_cast<const uint4*>(blk + 32);
    }
}

// one Q8_1 block (its 9 dwords) into the stage: codes and {sum of codes, d8}
__device__ __forceinline__ void kstage_one(const uint32_t (&wq)[9], int J, uint4* lq, uint2* lr) {
    int su = 0;
#pragma unroll
    for (int i = 1; i <= 8; ++i) su = sdot4(static_cast<int>(wq[i]), 0x01010101, su);
    lq[2 * J] = make_uint4(wq[1], wq[2], wq[3], wq[4]);
    lq[2 * J + 1] = make_uint4(wq[5], wq[6], wq[7], wq[8]);
    lr[J] = make_uint2(static_cast<uint32_t>(su), __float_as_uint(half_bits_to_float(wq[0])));
}

// Issue order (a wave's loads return in issue order): the lane's first kSB activation blocks, then its weight blocks
// of the first NI steps (NI = 1..3, sized by the launch to the row: every step of rows up to 12288 wide), then the
// stage is written;
// every load is unconditional from a clamped address (rows past the last and blocks past the row's end re-read the
// last ones and are not used), so no wait covers loads it does not need.  The arithmetic, block by block in ascending
// order per lane, is unchanged: the same bits as one step at a time.
template <int TYPE, int NCOLS, bool RES, int NI>
__global__ __launch_bounds__(256) void kquant_gemv_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ x,
                                                          float* y, const float* res, float* partials, int n_in,
                                                          int n_out) {
    constexpr int kBytes = TYPE == 13 ? 176 : 144;
    constexpr int kNI = NI;
    // staged blocks per lane held in registers: NCOLS x 8 x 16 NI blocks over 256 lanes, at most 4
    constexpr int kSB = (NCOLS * NI + 1) / 2 < 4 ? (NCOLS * NI + 1) / 2 : 4;
    extern __shared__ uint4 smem[];
    __shared__ float vout[NCOLS][4];
    const int nbq = n_in / 32, nb = n_in / 256;
    uint4* lq = smem;                                             // codes: [col][block][2]
    uint2* lr = reinterpret_cast<uint2*>(smem + 2 * NCOLS * nbq);   // records: [col][block] {sum of codes, d8}
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int row = blockIdx.x * 4 + wv;
    const int p = lane & 3;
    const int nstage = NCOLS * nbq;

    uint32_t sv[kSB][9];
#pragma unroll
    for (int m = 0; m < kSB; ++m) {
        const uint32_t* q = reinterpret_cast<const uint32_t*>(
            x + static_cast<size_t>(min(static_cast<int>(threadIdx.x) + 256 * m, nstage - 1)) * kQ8_1Bytes);
#pragma unroll
        for (int i = 0; i < 9; ++i) sv[m][i] = q[i];
    }
    const uint8_t* wrow = w + static_cast<size_t>(min(row, n_out - 1)) * nb * kBytes;
    KBlock<TYPE> kb[kNI];
#pragma unroll
    for (int i = 0; i < kNI; ++i) kblock_load<TYPE>(kb[i], wrow + static_cast<size_t>(min((lane >> 2) + 16 * i, nb - 1)) * kBytes, p);
#pragma unroll
    for (int m = 0; m < kSB; ++m) kstage_one(sv[m], min(static_cast<int>(threadIdx.x) + 256 * m, nstage - 1), lq, lr);
    for (int J = threadIdx.x + 256 * kSB; J < nstage; J += 256) {
        const uint32_t* q = reinterpret_cast<const uint32_t*>(x + static_cast<size_t>(J) * kQ8_1Bytes);
        uint32_t wq[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) wq[i] = q[i];
        kstage_one(wq, J, lq, lr);
    }
    __syncthreads();

    float acc[NCOLS];
#pragma unroll
    for (int c = 0; c < NCOLS; ++c) acc[c] = 0.0f;
    // block b of the lane: sub-blocks 2 p and 2 p + 1 against every column
    auto block_dot = [&](const KBlock<TYPE>& k, int b) {
        uint32_t Q[8] = {k.qa.x, k.qa.y, k.qa.z, k.qa.w, k.qb.x, k.qb.y, k.qb.z, k.qb.w};
        uint32_t H[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if constexpr (TYPE == 13) {
            H[0] = k.ha.x; H[1] = k.ha.y; H[2] = k.ha.z; H[3] = k.ha.w;
            H[4] = k.hb.x; H[5] = k.hb.y; H[6] = k.hb.z; H[7] = k.hb.w;
        }
        int sc0, m0, sc1, m1;
        scale_min(k.s0, k.s1, k.s2, 2 * p, sc0, m0);
        scale_min(k.s0, k.s1, k.s2, 2 * p + 1, sc1, m1);
        const float d = half_bits_to_float(k.dm & 0xffffu), dmin = half_bits_to_float(k.dm >> 16);
        int v0[8], v1[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v0[i] = static_cast<int>(Q[i] & 0x0f0f0f0fu);
            v1[i] = static_cast<int>((Q[i] >> 4) & 0x0f0f0f0fu);
            if constexpr (TYPE == 13) {
                v0[i] |= static_cast<int>(((H[i] >> (2 * p)) & 0x01010101u) << 4);
                v1[i] |= static_cast<int>(((H[i] >> (2 * p + 1)) & 0x01010101u) << 4);
            }
        }
        const int j = 8 * b + 2 * p;   // Q8_1 block of sub-block 2 p
#pragma unroll
        for (int c = 0; c < NCOLS; ++c) {
            const uint4* cq = lq + 2 * (c * nbq + j);
            const uint4 u0a = cq[0], u0b = cq[1], u1a = cq[2], u1b = cq[3];
            const int u0[8] = {static_cast<int>(u0a.x), static_cast<int>(u0a.y), static_cast<int>(u0a.z),
                               static_cast<int>(u0a.w), static_cast<int>(u0b.x), static_cast<int>(u0b.y),
                               static_cast<int>(u0b.z), static_cast<int>(u0b.w)};
            const int u1[8] = {static_cast<int>(u1a.x), static_cast<int>(u1a.y), static_cast<int>(u1a.z),
                               static_cast<int>(u1a.w), static_cast<int>(u1b.x), static_cast<int>(u1b.y),
                               static_cast<int>(u1b.z), static_cast<int>(u1b.w)};
            int dot0 = 0, dot1 = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                dot0 = sdot4(v0[i], u0[i], dot0);
                dot1 = sdot4(v1[i], u1[i], dot1);
            }
            const uint2 r0 = lr[c * nbq + j], r1 = lr[c * nbq + j + 1];
            const float d80 = __uint_as_float(r0.y), d81 = __uint_as_float(r1.y);
            float sumf_d = d80 * static_cast<float>(dot0 * sc0);
            sumf_d = __builtin_fmaf(d81, static_cast<float>(dot1 * sc1), sumf_d);
            float sumf_m = d80 * static_cast<float>(static_cast<int>(r0.x) * m0);
            sumf_m = __builtin_fmaf(d81, static_cast<float>(static_cast<int>(r1.x) * m1), sumf_m);
            acc[c] += __builtin_fmaf(d, sumf_d, -(dmin * sumf_m));
        }
    };
    if (row < n_out) {
#pragma unroll
        for (int i = 0; i < kNI; ++i)
            if ((lane >> 2) + 16 * i < nb) block_dot(kb[i], (lane >> 2) + 16 * i);
        for (int b = (lane >> 2) + 16 * kNI; b < nb; b += 16) {   // rows wider than 16 kNI blocks
            KBlock<TYPE> k;
            kblock_load<TYPE>(k, wrow + static_cast<size_t>(b) * kBytes, p);
            block_dot(k, b);
        }
    }
#pragma unroll
    for (int c = 0; c < NCOLS; ++c) {
        float s = group_sum<64>(acc[c]);
        if (row < n_out) {
            if constexpr (RES) s += res[static_cast<size_t>(c) * n_out + row];
            if (lane == 0) {
                y[static_cast<size_t>(c) * n_out + row] = s;
                vout[c][wv] = s;
            }
        }
    }
    if constexpr (RES) {
        __syncthreads();
        if (threadIdx.x < NCOLS) {
            const int c = threadIdx.x;
            float pp = 0.0f;
            for (int i = 0; i < 4; ++i)
                if (blockIdx.x * 4 + i < n_out) pp = __builtin_fmaf(vout[c][i], vout[c][i], pp);
            partials[static_cast<size_t>(c) * ((n_out + 3) / 4) + blockIdx.x] = pp;
        }
    }
}

template <int TYPE, int NCOLS, bool RES>
void launch_cols(const uint8_t* w, const uint8_t* x, float* y, const float* res, float* partials, int n_in, int n_out,
                 hipStream_t s) {
    const size_t lds = static_cast<size_t>(NCOLS) * (n_in / 32) * 40;
    const int nb = n_in / 256;
    const dim3 grid((n_out + 3) / 4);
    if (nb <= 16)
        hipLaunchKernelGGL((kquant_gemv_kernel<TYPE, NCOLS, RES, 1>), grid, dim3(256), lds, s, w, x, y, res, partials,
                           n_in, n_out);
    else if (nb <= 32)
        hipLaunchKernelGGL((kquant_gemv_kernel<TYPE, NCOLS, RES, 2>), grid, dim3(256), lds, s, w, x, y, res, partials,
                           n_in, n_out);
    else
        hipLaunchKernelGGL((kquant_gemv_kernel<TYPE, NCOLS, RES, 3>), grid, dim3(256), lds, s, w, x, y, res, partials,
                           n_in, n_out);
}

template <int TYPE, bool RES>
int launch(const void* wv, const void* xv, float* y, const float* res, float* partials, int n_in, int n_out, int ncols,
           hipStream_t s) {
    const auto* w = static_cast<const uint8_t*>(wv);
    const auto* x = static_cast<const uint8_t*>(xv);
    const int per = std::max(1, std::min(4, kStageMax / ((n_in / 32) * 40)));
    const size_t xcol = static_cast<size_t>(n_in / 32) * kQ8_1Bytes;
    const size_t pcol = static_cast<size_t>((n_out + 3) / 4);
    for (int j = 0; j < ncols; j += per) {
        const int nj = std::min(per, ncols - j);
        const uint8_t* xj = x + j * xcol;
        float* yj = y + static_cast<size_t>(j) * n_out;
        const float* rj = RES ? res + static_cast<size_t>(j) * n_out : nullptr;
        float* pj = RES ? partials + j * pcol : nullptr;
        switch (nj) {
            case 1: launch_cols<TYPE, 1, RES>(w, xj, yj, rj, pj, n_in, n_out, s); break;
            case 2: launch_cols<TYPE, 2, RES>(w, xj, yj, rj, pj, n_in, n_out, s); break;
            case 3: launch_cols<TYPE, 3, RES>(w, xj, yj, rj, pj, n_in, n_out, s); break;
            default: launch_cols<TYPE, 4, RES>(w, xj, yj, rj, pj, n_in, n_out, s); break;
        }
        if (const int rc = launch_status(TYPE == 13 ? "native_q5_k_mmvq" : "native_q4_k_mmvq")) return rc;
    }
    return RMI_OK;
}

int validate(const void* w, const void* x, const float* y, int n_in, int n_out, int ncols, void* stream) {
    if (n_in <= 0 || n_in % 256 != 0 || (n_in / 32) * 40 > kStageMax)
        return fail(RMI_ERR_SHAPE, "native MMVQ requires n_in > 0 and divisible by its block element count");
    if (ncols < 1 || ncols > kMaxCols) return fail(RMI_ERR_SHAPE, "native MMVQ requires 1 <= ncols <= 16");
    if (n_out <= 0) return fail(RMI_ERR_SHAPE, "native MMVQ requires n_out > 0");
    if (!aligned16(w) || !aligned4(x) || !aligned4(y))
        return fail(RMI_ERR_POINTER, "K-quant MMVQ requires a 16-byte aligned matrix and 4-byte aligned x, y");
    if (!stream) return fail(RMI_ERR_STREAM, "native MMVQ requires an explicit non-null CUDA stream");
    return RMI_OK;
}

}  // namespace
}  // namespace rmi

using namespace rmi;

extern "C" int rmi_native_q4_k_mmvq(const void* w, const void* x_q8_1, float* y, int n_in, int n_out, int ncols,
                                    void* stream) {
    if (int rc = validate(w, x_q8_1, y, n_in, n_out, ncols, stream)) return rc;
    return launch<12, false>(w, x_q8_1, y, nullptr, nullptr, n_in, n_out, ncols, static_cast<hipStream_t>(stream));
}

extern "C" int rmi_native_q5_k_mmvq(const void* w, const void* x_q8_1, float* y, int n_in, int n_out, int ncols,
                                    void* stream) {
    if (int rc = validate(w, x_q8_1, y, n_in, n_out, ncols, stream)) return rc;
    return launch<13, false>(w, x_q8_1, y, nullptr, nullptr, n_in, n_out, ncols, static_cast<hipStream_t>(stream));
}

extern "C" int rmi_native_q4_k_mmvq_res_n(const void* w, const void* x_q8_1, float* y, const float* res,
                                          float* partials, int n_in, int n_out, int ncols, void* stream) {
    if (int rc = validate(w, x_q8_1, y, n_in, n_out, ncols, stream)) return rc;
    if (!aligned4(res) || !aligned4(partials))
        return fail(RMI_ERR_POINTER, "native MMVQ requires non-null 4-byte aligned device pointers");
    return launch<12, true>(w, x_q8_1, y, res, partials, n_in, n_out, ncols, static_cast<hipStream_t>(stream));
}

extern "C" int rmi_native_q5_k_mmvq_res_n(const void* w, const void* x_q8_1, float* y, const float* res,
                                          float* partials, int n_in, int n_out, int ncols, void* stream) {
    if (int rc = validate(w, x_q8_1, y, n_in, n_out, ncols, stream)) return rc;
    if (!aligned4(res) || !aligned4(partials))
        return fail(RMI_ERR_POINTER, "native MMVQ requires non-null 4-byte aligned device pointers");
    return launch<13, true>(w, x_q8_1, y, res, partials, n_in, n_out, ncols, static_cast<hipStream_t>(stream));
}

extern "C" int rmi_native_q4_k_mmvq_res(const void* w, const void* x_q8_1, float* y, const float* res,
                                        float* partials, int n_in, int n_out, void* stream) {
    return rmi_native_q4_k_mmvq_res_n(w, x_q8_1, y, res, partials, n_in, n_out, 1, stream);
}

extern "C" int rmi_native_q5_k_mmvq_res(const void* w, const void* x_q8_1, float* y, const float* res,
                                        float* partials, int n_in, int n_out, void* stream) {
    return rmi_native_q5_k_mmvq_res_n(w, x_q8_1, y, res, partials, n_in, n_out, 1, stream);
}
