// q8_1.hip - fp32 -> Q8_1 activation quantizer (reference src/native_mmvq.cu:158-173, launcher 3054-3071).
// One lane per element; each 32-lane half of a wave64 owns one 36-byte block.
#include "rmi_common.h"

namespace rmi {
namespace {

__global__ __launch_bounds__(256) void quantize_q8_1_kernel(const float* __restrict__ x, uint8_t* __restrict__ y,
                                                            int n_total) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n_total) return;   // n_total % 32 == 0: whole 32-lane groups leave together
    q8_1_store_lane(x[i], y + static_cast<size_t>(i / 32) * kQ8_1Bytes);
}

}  // namespace
}  // namespace rmi

using namespace rmi;

extern "C" size_t rmi_native_q8_1_bytes(int n_in, int ncols) {
    if (n_in <= 0 || n_in % 32 != 0 || ncols < 1 || ncols > kMaxCols) {
        set_error("native MMVQ requires n_in > 0 and divisible by its block element count");
        return 0;
    }
    return static_cast<size_t>(ncols) * static_cast<size_t>(n_in / 32) * kQ8_1Bytes;
}

extern "C" int rmi_native_quantize_q8_1(const float* x, void* x_q8_1, int n_in, int ncols, void* stream) {
    if (n_in <= 0 || n_in % 32 != 0)
        return fail(RMI_ERR_SHAPE, "native MMVQ requires n_in > 0 and divisible by its block element count");
    if (ncols < 1 || ncols > kMaxCols) return fail(RMI_ERR_SHAPE, "native MMVQ requires 1 <= ncols <= 16");
    if (!aligned4(x) || !aligned4(x_q8_1))
        return fail(RMI_ERR_POINTER, "native MMVQ requires non-null 4-byte aligned device pointers");
    if (!stream) return fail(RMI_ERR_STREAM, "native MMVQ requires an explicit non-null CUDA stream");
    // columns are contiguous and n_in % 32 == 0, so ncols columns quantize as one vector of ncols * n_in
    const int n_total = n_in * ncols;
    hipLaunchKernelGGL(quantize_q8_1_kernel, dim3((n_total + 255) / 256), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, static_cast<uint8_t*>(x_q8_1), n_total);
    return launch_status("native_quantize_q8_1");
}
