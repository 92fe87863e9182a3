// epilogue_dev.h - device pieces shared by the epilogue kernels (epilogue.hip) and the engine's fused round-tail
// kernels (engine.hip), so that both give the same bits: the norm's partial-sum tree, the normed fp32 output and the
// argmax keys (reference src/qwythos.cpp:602-715, 70-94).
#pragma once

#include "rmi_common.h"

namespace rmi {
namespace {

// sum of a vector's 4-row partials, by the tree of rmi_common.h (norm_load / norm_wave_sum / norm_inv)
__device__ float block_sum_partials(const float* __restrict__ p, int np) {
    __shared__ float red[4];
    NormLoads pv;
    norm_load(pv, p, np, static_cast<int>(threadIdx.x));
    const float s = norm_wave_sum(pv, p, np, static_cast<int>(threadIdx.x));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    const float tot = ((red[0] + red[1]) + red[2]) + red[3];
    __syncthreads();
    return tot;
}

// fp32 out = (x * w) * inv (reference rms_norm_out_kernel, qw:658-672) for column c, elements 256 xb + lane, optionally
// with the output's own partials; one 256-lane workgroup
__device__ __forceinline__ void rms_norm_out_block(const float* __restrict__ x, const float* __restrict__ w,
                                                   const float* __restrict__ partials, float* __restrict__ out,
                                                   float* __restrict__ out_partials, int cols, float eps,
                                                   int out_stride, int c, int xb) {
    x += static_cast<size_t>(c) * cols;
    partials += static_cast<size_t>(c) * (cols / 4);
    out += static_cast<size_t>(c) * out_stride;
    const int i = xb * 256 + threadIdx.x;
    const float xv = x[min(i, cols - 1)], wv = w[min(i, cols - 1)];   // in flight with the partials
    const float ss = block_sum_partials(partials, cols / 4);
    const float inv = rsqrtf(ss / static_cast<float>(cols) + eps);
    float v = 0.0f;
    if (i < cols) {
        v = (xv * wv) * inv;
        out[i] = v;
    }
    if (out_partials) {
        // the 4 rows of a partial slot are 4 consecutive lanes: gather them in row order on the first lane
        const float v0 = quad_lane<0>(v), v1 = quad_lane<1>(v), v2 = quad_lane<2>(v), v3 = quad_lane<3>(v);
        if ((threadIdx.x & 3) == 0 && i < cols) {
            float p = 0.0f;
            p = __builtin_fmaf(v0, v0, p);
            if (i + 1 < cols) p = __builtin_fmaf(v1, v1, p);
            if (i + 2 < cols) p = __builtin_fmaf(v2, v2, p);
            if (i + 3 < cols) p = __builtin_fmaf(v3, v3, p);
            out_partials[static_cast<size_t>(c) * ((cols + 3) / 4) + i / 4] = p;
        }
    }
}

// ---- argmax: lowest index wins ties (qw:70-94: monotonic float bits, n-1-idx packing) -------------------------------
__device__ __forceinline__ uint64_t argmax_key(float v, int idx) {
    uint32_t b = __float_as_uint(v);
    b ^= (b >> 31) ? 0xffffffffu : 0x80000000u;
    return (static_cast<uint64_t>(b) << 32) | static_cast<uint32_t>(0x7fffffff - idx);
}

__device__ __forceinline__ uint64_t key_max64(uint64_t k) {
    auto step = [&](uint32_t lo, uint32_t hi) {
        const uint64_t o = (static_cast<uint64_t>(hi) << 32) | lo;
        k = o > k ? o : k;
    };
    step(xor_lane<32>(static_cast<uint32_t>(k)), xor_lane<32>(static_cast<uint32_t>(k >> 32)));
    step(xor_lane<16>(static_cast<uint32_t>(k)), xor_lane<16>(static_cast<uint32_t>(k >> 32)));
    step(xor_lane<8>(static_cast<uint32_t>(k)), xor_lane<8>(static_cast<uint32_t>(k >> 32)));
    step(xor_lane<4>(static_cast<uint32_t>(k)), xor_lane<4>(static_cast<uint32_t>(k >> 32)));
    step(xor_lane<2>(static_cast<uint32_t>(k)), xor_lane<2>(static_cast<uint32_t>(k >> 32)));
    step(xor_lane<1>(static_cast<uint32_t>(k)), xor_lane<1>(static_cast<uint32_t>(k >> 32)));
    return k;
}

constexpr int kArgmaxBlocks = 256;

// the greedy token of column c from its kArgmaxBlocks partial keys, by one 256-lane workgroup; every lane returns it
__device__ __forceinline__ int argmax_final_block(const uint64_t* __restrict__ part, int c) {
    __shared__ uint64_t red[4];
    __shared__ int res;
    uint64_t best = part[static_cast<size_t>(c) * kArgmaxBlocks + threadIdx.x];
    best = key_max64(best);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t m = red[0];
        for (int i = 1; i < 4; ++i) m = red[i] > m ? red[i] : m;
        res = 0x7fffffff - static_cast<int>(static_cast<uint32_t>(m));
    }
    __syncthreads();
    const int r = res;
    __syncthreads();   // red and res are free for the next call
    return r;
}

}  // namespace

// argmax_partial_kernel over ncols columns into part (kArgmaxBlocks keys per column), on stream s (epilogue.hip)
void argmax_partial_launch(const float* logits, int n, int ncols, int col_stride, uint64_t* part, hipStream_t s);

}  // namespace rmi
