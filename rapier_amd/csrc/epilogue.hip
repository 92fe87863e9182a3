// epilogue.hip - the small per-token kernels between GEMVs (reference src/qwythos.cpp:602-715, 70-94, 109-115).
//
// Every kernel takes `ncols` columns (blockIdx.y) so both verify columns ride one launch; a column's arithmetic is
// the same as a single-column call, bit for bit.  Row-norm partials follow the GEMV epilogue contract: one slot per
// 4 rows, partial[g] = fma chain of the 4 rows' squares in row order.
//
// Norm reduction (rms_quant_apply / rms_norm_out): 256 lanes; lane t adds partials t, t+256, t+512, ... in order,
// then a 64-lane xor butterfly, then the 4 wave sums in order.  Every workgroup derives the same bits.
#include "epilogue_dev.h"

namespace rmi {
namespace {

__device__ __forceinline__ float sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }

// Q8_1 of (x * w) * inv of one column, one lane per element (reference rms_quant_apply_kernel, qw:627-655); y is the
// column's first Q8_1 block
__device__ __forceinline__ void rms_quant_column(const float* __restrict__ x, const float* __restrict__ w,
                                                 const float* __restrict__ partials, uint8_t* __restrict__ y, int cols,
                                                 float eps) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    // x and w do not depend on the reduction: in flight together with the partials (clamped, unconditional)
    const float xv = x[min(i, cols - 1)], wv = w[min(i, cols - 1)];
    const float ss = block_sum_partials(partials, cols / 4);
    const float inv = rsqrtf(ss / static_cast<float>(cols) + eps);
    if (i >= cols) return;   // cols % 32 == 0: whole 32-lane groups leave together
    q8_1_store_lane((xv * wv) * inv, y + static_cast<size_t>(i / 32) * kQ8_1Bytes);
}

__global__ __launch_bounds__(256) void rms_quant_apply_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                              const float* __restrict__ partials,
                                                              uint8_t* __restrict__ y, int cols, float eps) {
    const int c = blockIdx.y;
    rms_quant_column(x + static_cast<size_t>(c) * cols, w, partials + static_cast<size_t>(c) * (cols / 4),
                     y + static_cast<size_t>(c) * (cols / 32) * kQ8_1Bytes, cols, eps);
}

// rms_quant_apply_kernel with the partials formed from x in the workgroup (slot g = the fma chain of rows 4g..4g+3
// in row order, as row_sum_partials writes it), then the same tree: the bits of row_sum_partials + rms_quant_apply
// without the partials launch.  x 16-byte aligned, cols a multiple of 32.
__device__ __forceinline__ float block_sum_self(const float* __restrict__ x, int cols) {
    __shared__ float red[4];
    const int np = cols / 4, t = static_cast<int>(threadIdx.x);
    float4 v[kNormLoads];
#pragma unroll
    for (int k = 0; k < kNormLoads; ++k) v[k] = reinterpret_cast<const float4*>(x)[min(t + 256 * k, np - 1)];
    auto slot = [](const float4 q) {
        float p = __builtin_fmaf(q.x, q.x, 0.0f);
        p = __builtin_fmaf(q.y, q.y, p);
        p = __builtin_fmaf(q.z, q.z, p);
        return __builtin_fmaf(q.w, q.w, p);
    };
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < kNormLoads; ++k)
        if (t + 256 * k < np) s += slot(v[k]);
    for (int i = t + 256 * kNormLoads; i < np; i += 256) s += slot(reinterpret_cast<const float4*>(x)[i]);
    s = group_sum<64>(s);
    if ((t & 63) == 0) red[t >> 6] = s;
    __syncthreads();
    const float tot = ((red[0] + red[1]) + red[2]) + red[3];
    __syncthreads();
    return tot;
}

__global__ __launch_bounds__(256) void rms_quant_self_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                             uint8_t* __restrict__ y, int cols, float eps) {
    const int c = blockIdx.y;
    x += static_cast<size_t>(c) * cols;
    y += static_cast<size_t>(c) * (cols / 32) * kQ8_1Bytes;
    const int i = blockIdx.x * 256 + threadIdx.x;
    const float xv = x[min(i, cols - 1)], wv = w[min(i, cols - 1)];
    const float ss = block_sum_self(x, cols);
    const float inv = rsqrtf(ss / static_cast<float>(cols) + eps);
    if (i >= cols) return;   // cols % 32 == 0: whole 32-lane groups leave together
    q8_1_store_lane((xv * wv) * inv, y + static_cast<size_t>(i / 32) * kQ8_1Bytes);
}

// two normed vectors of a column into the two halves of one Q8_1 row of 2 cols (blockIdx.z = half)
struct NormInput {
    const float* x;
    const float* w;
    const float* partials;
};

__global__ __launch_bounds__(256) void rms_quant_pair_kernel(NormInput a, NormInput b, uint8_t* __restrict__ y,
                                                             int cols, float eps) {
    const int c = blockIdx.y;
    const NormInput& in = blockIdx.z ? b : a;
    rms_quant_column(in.x + static_cast<size_t>(c) * cols, in.w, in.partials + static_cast<size_t>(c) * (cols / 4),
                     y + (static_cast<size_t>(c) * 2 + blockIdx.z) * (cols / 32) * kQ8_1Bytes, cols, eps);
}

// fp32 out = (x * w) * inv (reference rms_norm_out_kernel, qw:658-672), optionally with the output's own partials
__global__ __launch_bounds__(256) void rms_norm_out_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                           const float* __restrict__ partials, float* __restrict__ out,
                                                           float* __restrict__ out_partials, int cols, float eps,
                                                           int out_stride) {
    rms_norm_out_block(x, w, partials, out, out_partials, cols, eps, out_stride, blockIdx.y, blockIdx.x);
}

// partials[g] = sum of squares of rows 4g..4g+3 (reference row_sum_partials_kernel, qw:616-623); optionally x += o
// first (add_partials_1024_kernel, qw:602-614)
__global__ __launch_bounds__(256) void add_partials_kernel(float* __restrict__ x, const float* __restrict__ o,
                                                           float* __restrict__ partials, int n) {
    const int c = blockIdx.y;
    const int g = blockIdx.x * 256 + threadIdx.x;
    const int np = (n + 3) / 4;
    if (g >= np) return;
    x += static_cast<size_t>(c) * n;
    float p = 0.0f;
    for (int r = 4 * g; r < 4 * g + 4 && r < n; ++r) {
        float v = x[r];
        if (o) {
            v += o[static_cast<size_t>(c) * n + r];
            x[r] = v;
        }
        p = __builtin_fmaf(v, v, p);
    }
    partials[static_cast<size_t>(c) * np + g] = p;
}

// Q8_1 of silu(gate) * up (reference swiglu_quant_kernel, qw:676-689)
__global__ __launch_bounds__(256) void swiglu_quant_kernel(const float* __restrict__ up, const float* __restrict__ gate,
                                                           uint8_t* __restrict__ y, int n, int col_stride) {
    const int c = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    // loads from a clamped index ahead of the range check, held there by the asm: with the check first, the pointer
    // arguments are fetched only after it, one more round trip before the data loads
    const size_t off = static_cast<size_t>(c) * col_stride + min(i, n - 1);
    float g = gate[off], u = up[off];
    asm volatile("" : "+v"(g), "+v"(u));
    if (i >= n) return;   // n % 32 == 0: whole 32-lane groups leave together
    q8_1_store_lane(silu(g) * u, y + (static_cast<size_t>(c) * (n / 32) + i / 32) * kQ8_1Bytes);
}

// the same over an up||gate output in the SwiGLU row order (64-row groups [gate 32 | up 32]): output i reads gate at
// 64 (i / 32) + i % 32 and up 32 rows later
__global__ __launch_bounds__(256) void swiglu_quant_interleaved_kernel(const float* __restrict__ ug,
                                                                       uint8_t* __restrict__ y, int n, int col_stride) {
    const int c = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int ic = min(i, n - 1);
    const size_t off = static_cast<size_t>(c) * col_stride + 64 * (ic / 32) + ic % 32;
    float g = ug[off], u = ug[off + 32];
    asm volatile("" : "+v"(g), "+v"(u));   // loads ahead of the range check (see swiglu_quant_kernel)
    if (i >= n) return;
    q8_1_store_lane(silu(g) * u, y + (static_cast<size_t>(c) * (n / 32) + i / 32) * kQ8_1Bytes);
}

// Q8_1 of o * sigmoid(g) (reference sig_mul_quant_kernel, qw:692-704)
__global__ __launch_bounds__(256) void sig_mul_quant_kernel(const float* __restrict__ o, const float* __restrict__ g,
                                                            uint8_t* __restrict__ y, int n, int o_stride,
                                                            int g_stride) {
    const int c = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float v = o[static_cast<size_t>(c) * o_stride + i] * sigmoid(g[static_cast<size_t>(c) * g_stride + i]);
    q8_1_store_lane(v, y + (static_cast<size_t>(c) * (n / 32) + i / 32) * kQ8_1Bytes);
}

// beta = sigmoid(beta) in place; gate = softplus(alpha + dt) * ssm_a, softplus linear above 20 (qw:707-715).
// Layout per column: [beta n | alpha n] at ab + c * ab_stride.
__global__ __launch_bounds__(64) void beta_gate_kernel(float* __restrict__ ab, const float* __restrict__ dt,
                                                       const float* __restrict__ ssm_a, float* __restrict__ ggate,
                                                       int n, int ab_stride) {
    const int c = blockIdx.y;
    const int i = blockIdx.x * 64 + threadIdx.x;
    if (i >= n) return;
    float* beta = ab + static_cast<size_t>(c) * ab_stride;
    const float* alpha = beta + n;
    beta[i] = sigmoid(beta[i]);
    const float v = alpha[i] + dt[i];
    ggate[static_cast<size_t>(c) * n + i] = (v > 20.0f ? v : log1pf(expf(v))) * ssm_a[i];
}

// ---- argmax: lowest index wins ties (qw:70-94: monotonic float bits, n-1-idx packing; keys in epilogue_dev.h) -----
__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* __restrict__ l, int n, int col_stride,
                                                             uint64_t* __restrict__ part) {
    __shared__ uint64_t red[4];
    const int c = blockIdx.y;
    l += static_cast<size_t>(c) * col_stride;
    // four logits per lane per pass, loaded before the first compare (the max does not depend on the order)
    constexpr int kPer = 4, kStride = kArgmaxBlocks * 256;
    uint64_t best = 0;
    for (int i0 = blockIdx.x * 256 + threadIdx.x; i0 < n; i0 += kPer * kStride) {
        float v[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) v[k] = i0 + k * kStride < n ? l[i0 + k * kStride] : 0.0f;
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            if (i0 + k * kStride < n) {
                const uint64_t key = argmax_key(v[k], i0 + k * kStride);
                best = key > best ? key : best;
            }
        }
    }
    best = key_max64(best);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t m = red[0];
        for (int i = 1; i < 4; ++i) m = red[i] > m ? red[i] : m;
        part[static_cast<size_t>(c) * kArgmaxBlocks + blockIdx.x] = m;
    }
}

__global__ __launch_bounds__(256) void argmax_final_kernel(const uint64_t* __restrict__ part, int* __restrict__ out) {
    const int r = argmax_final_block(part, blockIdx.x);
    if (threadIdx.x == 0) out[blockIdx.x] = r;
}

// ---- token embedding: device dequant of one row per token ---------------------------------------------------------
// GGUF types 14 (Q6_K, ggml dequantize_row_q6_K order), 13 (Q5_K) and 12 (Q4_K) (ggml dequantize_row_q5_K / q4_K):
// every weight is d * sc * q (- dmin * m), whose products are exact in fp32, so one rounding at most.  One lane per
// element of a 256-block; partials of 4 consecutive elements in order.
__device__ __forceinline__ void k4_scale_min(const uint8_t* s, int j, int& sc, int& m) {
    if (j < 4) {
        sc = s[j] & 63;
        m = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

template <int TYPE>
__device__ __forceinline__ float embed_value(const uint8_t* b, int e) {
    if constexpr (TYPE == 14) {
        const int n = e >> 7, k = (e & 127) >> 5, l = e & 31;
        const uint8_t lo = b[64 * n + 32 * (k & 1) + l];
        const int nib = (k >> 1) ? (lo >> 4) : (lo & 15);
        const int hi = (b[128 + 32 * n + l] >> (2 * k)) & 3;
        const int sc = static_cast<int8_t>(b[192 + 8 * n + l / 16 + 2 * k]);
        const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(b + 208));
        return (d * static_cast<float>(sc)) * static_cast<float>((nib | (hi << 4)) - 32);
    } else {
        const int j = e >> 5, c = j >> 1, h = j & 1, l = e & 31;
        const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(b));
        const float dmin = half_bits_to_float(*reinterpret_cast<const uint16_t*>(b + 2));
        int sc, m;
        k4_scale_min(b + 4, j, sc, m);
        int q;
        if constexpr (TYPE == 13) q = ((b[48 + 32 * c + l] >> (4 * h)) & 15) | (((b[16 + l] >> j) & 1) << 4);
        else q = (b[16 + 32 * c + l] >> (4 * h)) & 15;
        return (d * static_cast<float>(sc)) * static_cast<float>(q) - dmin * static_cast<float>(m);
    }
}

template <int TYPE>
__global__ __launch_bounds__(256) void embed_kernel(const uint8_t* __restrict__ emb, const int* __restrict__ tok,
                                                    float* __restrict__ x, float* __restrict__ partials, int n_embd,
                                                    int n_vocab) {
    constexpr int kBytes = TYPE == 14 ? kQ6KBytes : TYPE == 13 ? 176 : 144;
    const int c = blockIdx.y;
    int t = tok[c];
    t = t < 0 ? 0 : (t >= n_vocab ? n_vocab - 1 : t);   // an out-of-range id never reads outside the table
    const int nb = n_embd / 256;
    const uint8_t* b = emb + (static_cast<size_t>(t) * nb + blockIdx.x) * kBytes;
    const int e = threadIdx.x;
    const float v = embed_value<TYPE>(b, e);
    const int idx = blockIdx.x * 256 + e;
    x[static_cast<size_t>(c) * n_embd + idx] = v;
    const float v0 = quad_lane<0>(v), v1 = quad_lane<1>(v), v2 = quad_lane<2>(v), v3 = quad_lane<3>(v);
    if ((e & 3) == 0) {
        float p = 0.0f;
        p = __builtin_fmaf(v0, v0, p);
        p = __builtin_fmaf(v1, v1, p);
        p = __builtin_fmaf(v2, v2, p);
        p = __builtin_fmaf(v3, v3, p);
        partials[static_cast<size_t>(c) * (n_embd / 4) + idx / 4] = p;
    }
}

bool bad_cols(int ncols) { return ncols < 1 || ncols > kMaxCols; }

}  // namespace
}  // namespace rmi

using namespace rmi;

extern "C" int rmi_rms_quant_apply(const float* x, const float* w, const float* partials, void* y_q8_1, int cols,
                                   float eps, int ncols, void* stream) {
    if (cols <= 0 || cols % 32 != 0 || bad_cols(ncols)) return fail(RMI_ERR_SHAPE, "rms_quant_apply: bad shape");
    if (!aligned4(x) || !aligned4(w) || !aligned4(partials) || !aligned4(y_q8_1))
        return fail(RMI_ERR_POINTER, "rms_quant_apply: null or misaligned pointer");
    hipLaunchKernelGGL(rms_quant_apply_kernel, dim3((cols + 255) / 256, ncols), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, w, partials, static_cast<uint8_t*>(y_q8_1), cols, eps);
    return launch_status("rms_quant_apply");
}

extern "C" int rmi_rms_quant_apply_self(const float* x, const float* w, void* y_q8_1, int cols, float eps, int ncols,
                                        void* stream) {
    if (cols <= 0 || cols % 32 != 0 || bad_cols(ncols)) return fail(RMI_ERR_SHAPE, "rms_quant_apply_self: bad shape");
    if (!aligned16(x) || !aligned4(w) || !aligned4(y_q8_1))
        return fail(RMI_ERR_POINTER, "rms_quant_apply_self: null or misaligned pointer");
    hipLaunchKernelGGL(rms_quant_self_kernel, dim3((cols + 255) / 256, ncols), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, w, static_cast<uint8_t*>(y_q8_1), cols, eps);
    return launch_status("rms_quant_apply_self");
}

extern "C" int rmi_rms_quant_apply_pair(const float* x0, const float* w0, const float* partials0, const float* x1,
                                        const float* w1, const float* partials1, void* y_q8_1, int cols, float eps,
                                        int ncols, void* stream) {
    if (cols <= 0 || cols % 32 != 0 || bad_cols(ncols)) return fail(RMI_ERR_SHAPE, "rms_quant_apply_pair: bad shape");
    if (!aligned4(x0) || !aligned4(w0) || !aligned4(partials0) || !aligned4(x1) || !aligned4(w1) ||
        !aligned4(partials1) || !aligned4(y_q8_1))
        return fail(RMI_ERR_POINTER, "rms_quant_apply_pair: null or misaligned pointer");
    hipLaunchKernelGGL(rms_quant_pair_kernel, dim3((cols + 255) / 256, ncols, 2), dim3(256), 0,
                       static_cast<hipStream_t>(stream), NormInput{x0, w0, partials0}, NormInput{x1, w1, partials1},
                       static_cast<uint8_t*>(y_q8_1), cols, eps);
    return launch_status("rms_quant_apply_pair");
}

extern "C" int rmi_rms_norm_out_strided(const float* x, const float* w, const float* partials, float* out,
                                        int out_stride, float* out_partials, int cols, float eps, int ncols,
                                        void* stream) {
    if (cols <= 0 || cols % 4 != 0 || bad_cols(ncols) || out_stride < cols)
        return fail(RMI_ERR_SHAPE, "rms_norm_out: bad shape");
    if (!aligned4(x) || !aligned4(w) || !aligned4(partials) || !aligned4(out))
        return fail(RMI_ERR_POINTER, "rms_norm_out: null or misaligned pointer");
    hipLaunchKernelGGL(rms_norm_out_kernel, dim3((cols + 255) / 256, ncols), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, w, partials, out, out_partials, cols, eps, out_stride);
    return launch_status("rms_norm_out");
}

extern "C" int rmi_rms_norm_out(const float* x, const float* w, const float* partials, float* out, float* out_partials,
                                int cols, float eps, int ncols, void* stream) {
    return rmi_rms_norm_out_strided(x, w, partials, out, cols, out_partials, cols, eps, ncols, stream);
}

extern "C" int rmi_row_sum_partials(const float* x, float* partials, int n, int ncols, void* stream) {
    if (n <= 0 || bad_cols(ncols)) return fail(RMI_ERR_SHAPE, "row_sum_partials: bad shape");
    if (!aligned4(x) || !aligned4(partials)) return fail(RMI_ERR_POINTER, "row_sum_partials: null pointer");
    const int np = (n + 3) / 4;
    hipLaunchKernelGGL(add_partials_kernel, dim3((np + 255) / 256, ncols), dim3(256), 0,
                       static_cast<hipStream_t>(stream), const_cast<float*>(x), nullptr, partials, n);
    return launch_status("row_sum_partials");
}

extern "C" int rmi_add_partials(float* x, const float* o, float* partials, int n, int ncols, void* stream) {
    if (n <= 0 || bad_cols(ncols)) return fail(RMI_ERR_SHAPE, "add_partials: bad shape");
    if (!aligned4(x) || !aligned4(o) || !aligned4(partials)) return fail(RMI_ERR_POINTER, "add_partials: null pointer");
    const int np = (n + 3) / 4;
    hipLaunchKernelGGL(add_partials_kernel, dim3((np + 255) / 256, ncols), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, o, partials, n);
    return launch_status("add_partials");
}

extern "C" int rmi_swiglu_quant_interleaved(const float* up_gate, void* y_q8_1, int n, int ncols, int col_stride,
                                            void* stream) {
    if (n <= 0 || n % 32 != 0 || bad_cols(ncols) || col_stride < 2 * n)
        return fail(RMI_ERR_SHAPE, "swiglu_quant_interleaved: bad shape");
    if (!aligned4(up_gate) || !aligned4(y_q8_1)) return fail(RMI_ERR_POINTER, "swiglu_quant_interleaved: bad pointer");
    hipLaunchKernelGGL(swiglu_quant_interleaved_kernel, dim3((n + 255) / 256, ncols), dim3(256), 0,
                       static_cast<hipStream_t>(stream), up_gate, static_cast<uint8_t*>(y_q8_1), n, col_stride);
    return launch_status("swiglu_quant_interleaved");
}

extern "C" int rmi_swiglu_quant(const float* up, const float* gate, void* y_q8_1, int n, int ncols, int col_stride,
                                void* stream) {
    if (n <= 0 || n % 32 != 0 || bad_cols(ncols) || col_stride < n) return fail(RMI_ERR_SHAPE, "swiglu_quant: bad shape");
    if (!aligned4(up) || !aligned4(gate) || !aligned4(y_q8_1)) return fail(RMI_ERR_POINTER, "swiglu_quant: null pointer");
    hipLaunchKernelGGL(swiglu_quant_kernel, dim3((n + 255) / 256, ncols), dim3(256), 0,
                       static_cast<hipStream_t>(stream), up, gate, static_cast<uint8_t*>(y_q8_1), n, col_stride);
    return launch_status("swiglu_quant");
}

extern "C" int rmi_sig_mul_quant(const float* o, const float* g, void* y_q8_1, int n, int ncols, int o_stride,
                                 int g_stride, void* stream) {
    if (n <= 0 || n % 32 != 0 || bad_cols(ncols)) return fail(RMI_ERR_SHAPE, "sig_mul_quant: bad shape");
    if (!aligned4(o) || !aligned4(g) || !aligned4(y_q8_1)) return fail(RMI_ERR_POINTER, "sig_mul_quant: null pointer");
    hipLaunchKernelGGL(sig_mul_quant_kernel, dim3((n + 255) / 256, ncols), dim3(256), 0,
                       static_cast<hipStream_t>(stream), o, g, static_cast<uint8_t*>(y_q8_1), n, o_stride, g_stride);
    return launch_status("sig_mul_quant");
}

extern "C" int rmi_beta_gate(float* beta_alpha, const float* dt, const float* ssm_a, float* ggate, int n, int ncols,
                             int ab_stride, void* stream) {
    if (n <= 0 || bad_cols(ncols) || ab_stride < 2 * n) return fail(RMI_ERR_SHAPE, "beta_gate: bad shape");
    if (!aligned4(beta_alpha) || !aligned4(dt) || !aligned4(ssm_a) || !aligned4(ggate))
        return fail(RMI_ERR_POINTER, "beta_gate: null pointer");
    hipLaunchKernelGGL(beta_gate_kernel, dim3((n + 63) / 64, ncols), dim3(64), 0, static_cast<hipStream_t>(stream),
                       beta_alpha, dt, ssm_a, ggate, n, ab_stride);
    return launch_status("beta_gate");
}

namespace rmi {
void argmax_partial_launch(const float* logits, int n, int ncols, int col_stride, uint64_t* part, hipStream_t s) {
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(kArgmaxBlocks, ncols), dim3(256), 0, s, logits, n, col_stride, part);
}
}  // namespace rmi

extern "C" size_t rmi_argmax_workspace_bytes(int ncols) {
    return static_cast<size_t>(ncols > 0 ? ncols : 1) * kArgmaxBlocks * sizeof(uint64_t);
}

extern "C" int rmi_argmax(const float* logits, int n, int ncols, int col_stride, int* out_idx, void* workspace,
                          void* stream) {
    if (n <= 0 || bad_cols(ncols) || col_stride < n) return fail(RMI_ERR_SHAPE, "argmax: bad shape");
    if (!aligned4(logits) || !aligned4(out_idx) || !workspace || (reinterpret_cast<uintptr_t>(workspace) & 7u))
        return fail(RMI_ERR_POINTER, "argmax: null or misaligned pointer");
    auto* part = static_cast<uint64_t*>(workspace);
    argmax_partial_launch(logits, n, ncols, col_stride, part, static_cast<hipStream_t>(stream));
    hipLaunchKernelGGL(argmax_final_kernel, dim3(ncols), dim3(256), 0, static_cast<hipStream_t>(stream), part, out_idx);
    return launch_status("argmax");
}

// The draft input in one launch: blockIdx.z = 0 norms the embedding row of token tok[c] (dequantized here; each lane
// forms the partial slots the norm tree gives it, 4 elements each, as embed_kernel writes them), z = 1 the hidden
// vector b (its partials given) - the bits of rmi_embed followed by rmi_rms_quant_apply_pair.
template <int TYPE>
__global__ __launch_bounds__(256) void embed_quant_pair_kernel(const uint8_t* __restrict__ emb,
                                                               const int* __restrict__ tok, const float* __restrict__ w0,
                                                               NormInput b, uint8_t* __restrict__ y, int cols,
                                                               int n_vocab, float eps) {
    constexpr int kBytes = TYPE == 14 ? kQ6KBytes : TYPE == 13 ? 176 : 144;
    const int c = blockIdx.y;
    uint8_t* yc = y + (static_cast<size_t>(c) * 2 + blockIdx.z) * (cols / 32) * kQ8_1Bytes;
    if (blockIdx.z == 1) {
        rms_quant_column(b.x + static_cast<size_t>(c) * cols, b.w, b.partials + static_cast<size_t>(c) * (cols / 4), yc,
                         cols, eps);
        return;
    }
    __shared__ float red[4];
    int t = tok[c];
    t = t < 0 ? 0 : (t >= n_vocab ? n_vocab - 1 : t);   // as embed_kernel: never outside the table
    const uint8_t* row = emb + static_cast<size_t>(t) * (cols / 256) * kBytes;
    const int lane = static_cast<int>(threadIdx.x), i = blockIdx.x * 256 + lane;
    const float wv = w0[min(i, cols - 1)];
    const float v = embed_value<TYPE>(row + static_cast<size_t>(i / 256) * kBytes, i & 255);
    // the norm tree over the row's partial slots g = lane + 256 k (elements 4g .. 4g + 3)
    const int np = cols / 4;
    float s = 0.0f;
    for (int g = lane; g < np; g += 256) {
        float p = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int e = 4 * g + r;
            const float u = embed_value<TYPE>(row + static_cast<size_t>(e / 256) * kBytes, e & 255);
            p = __builtin_fmaf(u, u, p);
        }
        s += p;
    }
    s = group_sum<64>(s);
    if ((lane & 63) == 0) red[lane >> 6] = s;
    __syncthreads();
    const float inv = rsqrtf((((red[0] + red[1]) + red[2]) + red[3]) / static_cast<float>(cols) + eps);
    if (i >= cols) return;   // cols % 256 == 0 here: whole workgroups
    q8_1_store_lane((v * wv) * inv, yc + static_cast<size_t>(i / 32) * kQ8_1Bytes);
}

extern "C" int rmi_embed_quant_apply_pair(int type, const void* emb, const int* tokens, const float* w0,
                                          const float* x1, const float* w1, const float* partials1, void* y_q8_1,
                                          int cols, int n_vocab, float eps, int ncols, void* stream) {
    if (cols <= 0 || cols % 256 != 0 || n_vocab <= 0 || bad_cols(ncols))
        return fail(RMI_ERR_SHAPE, "embed_quant_apply_pair: bad shape");
    if (type != 14 && type != 13 && type != 12) return fail(RMI_ERR_UNSUPPORTED, "embed_quant_apply_pair: type");
    if (!emb || !aligned4(tokens) || !aligned4(w0) || !aligned4(x1) || !aligned4(w1) || !aligned4(partials1) ||
        !aligned4(y_q8_1))
        return fail(RMI_ERR_POINTER, "embed_quant_apply_pair: null or misaligned pointer");
    const auto* e = static_cast<const uint8_t*>(emb);
    auto* y = static_cast<uint8_t*>(y_q8_1);
    const dim3 grid(cols / 256, ncols, 2), block(256);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const NormInput b{x1, w1, partials1};
    if (type == 14) hipLaunchKernelGGL(embed_quant_pair_kernel<14>, grid, block, 0, s, e, tokens, w0, b, y, cols, n_vocab, eps);
    else if (type == 13) hipLaunchKernelGGL(embed_quant_pair_kernel<13>, grid, block, 0, s, e, tokens, w0, b, y, cols, n_vocab, eps);
    else hipLaunchKernelGGL(embed_quant_pair_kernel<12>, grid, block, 0, s, e, tokens, w0, b, y, cols, n_vocab, eps);
    return launch_status("embed_quant_apply_pair");
}

extern "C" int rmi_embed(int type, const void* emb, const int* tokens, float* x, float* partials, int n_embd,
                         int n_vocab, int ncols, void* stream) {
    if (n_embd <= 0 || n_embd % 256 != 0 || n_vocab <= 0 || bad_cols(ncols))
        return fail(RMI_ERR_SHAPE, "embed: bad shape");
    if (type != 14 && type != 13 && type != 12) return fail(RMI_ERR_UNSUPPORTED, "embed: token_embd type must be Q6_K, Q5_K or Q4_K");
    if (!emb || !aligned4(tokens) || !aligned4(x) || !aligned4(partials))
        return fail(RMI_ERR_POINTER, "embed: null or misaligned pointer");
    const auto s = static_cast<hipStream_t>(stream);
    const dim3 grid(n_embd / 256, ncols), block(256);
    const auto* e = static_cast<const uint8_t*>(emb);
    if (type == 14) hipLaunchKernelGGL(embed_kernel<14>, grid, block, 0, s, e, tokens, x, partials, n_embd, n_vocab);
    else if (type == 13) hipLaunchKernelGGL(embed_kernel<13>, grid, block, 0, s, e, tokens, x, partials, n_embd, n_vocab);
    else hipLaunchKernelGGL(embed_kernel<12>, grid, block, 0, s, e, tokens, x, partials, n_embd, n_vocab);
    return launch_status("embed");
}

extern "C" int rmi_embed_q6_k(const void* emb, const int* tokens, float* x, float* partials, int n_embd, int n_vocab,
                              int ncols, void* stream) {
    return rmi_embed(14, emb, tokens, x, partials, n_embd, n_vocab, ncols, stream);
}
