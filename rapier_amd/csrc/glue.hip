// glue.hip - the reference engine's small strata::kernels calls around the attention block, for gfx950:
//   rms_norm_weighted  per-row RMSNorm in place (qw:971-975: the q/k per-head norms, rows = heads, cols = head_dim)
//   native_rope_apply  NEOX RoPE (YaRN ramp) on the first n_rot dims of each head at the head's device position
//                      (qw:1165-1166, 1357-1358, 1542-1544, 2380-2407)
//   add_inplace / scale_inplace / silu_inplace  elementwise (the reference's --split and old-GDN paths, qw:1002,
//                      1053-1068, 1178)
// The engine itself runs these fused (rmi_attn_prep); the standalone forms use the same arithmetic: the norm's
// 64-lane butterfly and fixed wave order, and rope.h's rotation, so norm + rope here gives attn_prep's q bits.
#include "rmi_common.h"
#include "rope.h"

namespace rmi {
namespace {

constexpr int kNormThreads = 256;
constexpr int kMaxNormCols = 8192;

// one workgroup per row: each lane sums its elements t, t + 256, ... in order, a 64-lane butterfly per wave, the four
// wave sums in wave order; inv = rsqrt(ss / cols + eps); x = x * inv * w[c]
__global__ __launch_bounds__(kNormThreads) void rms_norm_weighted_kernel(float* __restrict__ x,
                                                                         const float* __restrict__ w, int cols,
                                                                         float eps) {
    __shared__ float red[kNormThreads / 64];
    constexpr int kPer = kMaxNormCols / kNormThreads;
    float* row = x + static_cast<size_t>(blockIdx.x) * cols;
    const int t = static_cast<int>(threadIdx.x);
    float v[kPer];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int c = t + k * kNormThreads;
        v[k] = c < cols ? row[c] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) ss = k == 0 ? v[0] * v[0] : fmaf(v[k], v[k], ss);
    ss = group_sum<64>(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    const float tot = ((red[0] + red[1]) + red[2]) + red[3];
    const float inv = rsqrtf(tot / static_cast<float>(cols) + eps);
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int c = t + k * kNormThreads;
        if (c < cols) row[c] = v[k] * inv * w[c];
    }
}

// one workgroup per head, one lane per dim; x may alias y (every lane reads its pair before the barrier)
__global__ void rope_apply_kernel(const float* x, float* y, int head_dim, int n_rot, const int* __restrict__ pos,
                                  float theta, Yarn yarn) {
    const int h = blockIdx.x;
    const int d = static_cast<int>(threadIdx.x);
    const size_t base = static_cast<size_t>(h) * head_dim;
    const int half = n_rot / 2;
    const int p = pos[h];
    float a = 0.0f, b = 0.0f;
    if (d < half) {
        a = x[base + d];
        b = x[base + d + half];
    }
    const float own = d < head_dim ? x[base + d] : 0.0f;
    __syncthreads();
    if (d < half) {
        float c, s;
        rope_cos_sin(p, d, n_rot, theta, yarn, &c, &s);
        y[base + d] = rope_lo(a, b, c, s);
        y[base + d + half] = rope_hi(a, b, c, s);
    } else if (d >= n_rot && d < head_dim) {
        y[base + d] = own;
    }
}

enum class Elementwise { Add, Scale, Silu };

template <Elementwise K>
__global__ void elementwise_kernel(float* __restrict__ x, const float* __restrict__ other, float s, size_t n) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if constexpr (K == Elementwise::Add) x[i] = x[i] + other[i];
    else if constexpr (K == Elementwise::Scale) x[i] = x[i] * s;
    else x[i] = silu(x[i]);
}

template <Elementwise K>
int launch_elementwise(float* x, const float* other, float s, int n, void* stream, const char* what) {
    if (n < 0) return fail(RMI_ERR_SHAPE, what);
    if (!aligned4(x) || (K == Elementwise::Add && !aligned4(other))) return fail(RMI_ERR_POINTER, what);
    if (n == 0) return RMI_OK;
    hipLaunchKernelGGL(elementwise_kernel<K>, dim3((n + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream),
                       x, other, s, static_cast<size_t>(n));
    return launch_status(what);
}

}  // namespace
}  // namespace rmi

using namespace rmi;

extern "C" int rmi_rms_norm_weighted(float* x, const float* w, int rows, int cols, float eps, void* stream) {
    if (rows < 0 || cols <= 0 || cols > kMaxNormCols) return fail(RMI_ERR_SHAPE, "rms_norm_weighted: invalid shape");
    if (!aligned4(x) || !aligned4(w)) return fail(RMI_ERR_POINTER, "rms_norm_weighted: invalid pointer");
    if (rows == 0) return RMI_OK;
    hipLaunchKernelGGL(rms_norm_weighted_kernel, dim3(rows), dim3(kNormThreads), 0, static_cast<hipStream_t>(stream),
                       x, w, cols, eps);
    return launch_status("rms_norm_weighted");
}

extern "C" int rmi_native_rope_apply(const float* x, float* y, int heads, int head_dim, int n_rot,
                                     const rmi_rope_params* rope, const int* pos, void* stream) {
    if (heads < 0 || head_dim <= 0 || head_dim > 1024 || n_rot < 0 || n_rot > head_dim || n_rot % 2 || !rope ||
        !(rope->freq_base > 1.0f))
        return fail(RMI_ERR_SHAPE, "native_rope_apply: invalid arguments");
    if (!aligned4(x) || !aligned4(y) || !aligned4(pos)) return fail(RMI_ERR_POINTER, "native_rope_apply: invalid pointer");
    Yarn yarn{};
    if (!yarn_setup(*rope, n_rot, &yarn)) return fail(RMI_ERR_SHAPE, "native_rope_apply: invalid YaRN parameters");
    if (heads == 0) return RMI_OK;
    const int threads = (head_dim + 63) / 64 * 64;
    hipLaunchKernelGGL(rope_apply_kernel, dim3(heads), dim3(threads), 0, static_cast<hipStream_t>(stream), x, y,
                       head_dim, n_rot, pos, rope->freq_base, yarn);
    return launch_status("native_rope_apply");
}

extern "C" int rmi_add_inplace(float* x, const float* y, int n, void* stream) {
    return launch_elementwise<Elementwise::Add>(x, y, 0.0f, n, stream, "add_inplace");
}

extern "C" int rmi_scale_inplace(float* x, int n, float s, void* stream) {
    return launch_elementwise<Elementwise::Scale>(x, nullptr, s, n, stream, "scale_inplace");
}

extern "C" int rmi_silu_inplace(float* x, int n, void* stream) {
    return launch_elementwise<Elementwise::Silu>(x, nullptr, 0.0f, n, stream, "silu_inplace");
}
