// mmvq_q8_0.hip - Q8_0 x Q8_1 GEMV (reference src/native_mmvq.cu: small_q8_dot 835-847, native_small_mmvq_kernel
// 865-900, residual variant 3142-3185) and the GGML-type dispatcher native_mmvq (3787-3818).
//
// One wave64 per output row, four rows per workgroup; lane l owns Q8_0 blocks l, l + 64, ...  Per block:
// sumi = sum of 8 v_dot4 over the 32 int8 pairs (exact), then acc = fma(d_w * d_x, float(sumi), acc) - the
// reference's d0 * d1 * float(sumi).  Rows are reduced by a fixed 64-lane butterfly, so every column of an
// ncols >= 2 call is bitwise the ncols = 1 result and the residual variant is bitwise plain + res.
#include "rmi_common.h"

namespace rmi {
namespace {

__device__ __forceinline__ uint32_t ldg_u32_b2(const uint8_t* p) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
    return static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16);
}

template <int NCOLS, bool RES>
__global__ __launch_bounds__(256) void q8_0_gemv_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ x,
                                                        float* y, const float* res, float* partials, int n_in,
                                                        int n_out) {
    __shared__ float vout[NCOLS][4];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int row = blockIdx.x * 4 + wv;
    const int nb = n_in / 32;
    float acc[NCOLS];
#pragma unroll
    for (int c = 0; c < NCOLS; ++c) acc[c] = 0.0f;
    if (row < n_out) {
        for (int j = lane; j < nb; j += 64) {
            const uint8_t* blk = w + (static_cast<size_t>(row) * nb + j) * kQ8_0Bytes;
            const float dw = half_bits_to_float(*reinterpret_cast<const uint16_t*>(blk));
            int v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = static_cast<int>(ldg_u32_b2(blk + 2 + 4 * i));
#pragma unroll
            for (int c = 0; c < NCOLS; ++c) {
                const uint32_t* xb = reinterpret_cast<const uint32_t*>(x + (static_cast<size_t>(c) * nb + j) * kQ8_1Bytes);
                int sumi = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) sumi = sdot4(v[i], static_cast<int>(xb[1 + i]), sumi);
                acc[c] = __builtin_fmaf(dw * half_bits_to_float(xb[0]), static_cast<float>(sumi), acc[c]);
            }
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
            float p = 0.0f;
            for (int i = 0; i < 4; ++i)
                if (blockIdx.x * 4 + i < n_out) p = __builtin_fmaf(vout[c][i], vout[c][i], p);
            partials[static_cast<size_t>(c) * ((n_out + 3) / 4) + blockIdx.x] = p;
        }
    }
}

template <bool RES>
int launch(const void* wv, const void* xv, float* y, const float* res, float* partials, int n_in, int n_out,
           int ncols, hipStream_t s) {
    const auto* w = static_cast<const uint8_t*>(wv);
    const auto* x = static_cast<const uint8_t*>(xv);
    const dim3 grid((n_out + 3) / 4), block(256);
    if (ncols > 4) {
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
    switch (ncols) {
        case 1: hipLaunchKernelGGL((q8_0_gemv_kernel<1, RES>), grid, block, 0, s, w, x, y, res, partials, n_in, n_out); break;
        case 2: hipLaunchKernelGGL((q8_0_gemv_kernel<2, RES>), grid, block, 0, s, w, x, y, res, partials, n_in, n_out); break;
        case 3: hipLaunchKernelGGL((q8_0_gemv_kernel<3, RES>), grid, block, 0, s, w, x, y, res, partials, n_in, n_out); break;
        default: hipLaunchKernelGGL((q8_0_gemv_kernel<4, RES>), grid, block, 0, s, w, x, y, res, partials, n_in, n_out); break;
    }
    return launch_status("native_q8_0_mmvq");
}

int validate(const void* w, const void* x, const float* y, int n_in, int n_out, int ncols, void* stream) {
    if (n_in <= 0 || n_in % 32 != 0)
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

extern "C" int rmi_native_q8_0_mmvq(const void* w, const void* x_q8_1, float* y, int n_in, int n_out, int ncols,
                                    void* stream) {
    if (int rc = validate(w, x_q8_1, y, n_in, n_out, ncols, stream)) return rc;
    return launch<false>(w, x_q8_1, y, nullptr, nullptr, n_in, n_out, ncols, static_cast<hipStream_t>(stream));
}

extern "C" int rmi_native_q8_0_mmvq_res_n(const void* w, const void* x_q8_1, float* y, const float* res,
                                          float* partials, int n_in, int n_out, int ncols, void* stream) {
    if (int rc = validate(w, x_q8_1, y, n_in, n_out, ncols, stream)) return rc;
    if (!aligned4(res) || !aligned4(partials))
        return fail(RMI_ERR_POINTER, "native MMVQ requires non-null 4-byte aligned device pointers");
    return launch<true>(w, x_q8_1, y, res, partials, n_in, n_out, ncols, static_cast<hipStream_t>(stream));
}

extern "C" int rmi_native_q8_0_mmvq_res(const void* w, const void* x_q8_1, float* y, const float* res,
                                        float* partials, int n_in, int n_out, void* stream) {
    return rmi_native_q8_0_mmvq_res_n(w, x_q8_1, y, res, partials, n_in, n_out, 1, stream);
}

extern "C" int rmi_native_mmvq_supported(int ggml_type) {
    return ggml_type == 14 || ggml_type == 13 || ggml_type == 12 || ggml_type == 8;
}

extern "C" size_t rmi_native_mmvq_weight_bytes(int ggml_type, int n_in, int n_out) {
    int elems, bytes;
    if (ggml_type == 14) { elems = 256; bytes = kQ6KBytes; }
    else if (ggml_type == 13) { elems = 256; bytes = 176; }
    else if (ggml_type == 12) { elems = 256; bytes = 144; }
    else if (ggml_type == 8) { elems = 32; bytes = kQ8_0Bytes; }
    else { set_error("unsupported native MMVQ GGML type"); return 0; }
    if (n_in <= 0 || n_in % elems != 0 || n_out <= 0) {
        set_error("native MMVQ requires n_in > 0 and divisible by its block element count");
        return 0;
    }
    return static_cast<size_t>(n_in / elems) * bytes * static_cast<size_t>(n_out);
}

extern "C" int rmi_native_q6_k_mmvq(const void*, const void*, float*, int, int, int, void*);
extern "C" int rmi_native_q5_k_mmvq(const void*, const void*, float*, int, int, int, void*);
extern "C" int rmi_native_q4_k_mmvq(const void*, const void*, float*, int, int, int, void*);

extern "C" int rmi_native_mmvq(int ggml_type, const void* w, const void* x_q8_1, float* y, int n_in, int n_out,
                               int ncols, void* stream) {
    // more than 16 columns: passes of 16 over the same weights (each column unchanged), as the reference does
    if (ncols > kMaxCols) {
        const size_t xcol = static_cast<size_t>(n_in / 32) * kQ8_1Bytes;
        for (int j = 0; j < ncols; j += kMaxCols) {
            const int nj = ncols - j < kMaxCols ? ncols - j : kMaxCols;
            const int rc = rmi_native_mmvq(ggml_type, w, static_cast<const uint8_t*>(x_q8_1) + j * xcol,
                                           y + static_cast<size_t>(j) * n_out, n_in, n_out, nj, stream);
            if (rc != RMI_OK) return rc;
        }
        return RMI_OK;
    }
    if (ggml_type == 14) return rmi_native_q6_k_mmvq(w, x_q8_1, y, n_in, n_out, ncols, stream);
    if (ggml_type == 13) return rmi_native_q5_k_mmvq(w, x_q8_1, y, n_in, n_out, ncols, stream);
    if (ggml_type == 12) return rmi_native_q4_k_mmvq(w, x_q8_1, y, n_in, n_out, ncols, stream);
    if (ggml_type == 8) return rmi_native_q8_0_mmvq(w, x_q8_1, y, n_in, n_out, ncols, stream);
    return fail(RMI_ERR_UNSUPPORTED, "unsupported native MMVQ GGML type");
}
