// rapier_mi_q8_1.hpp - the device-side Q8_1 block helpers the reference engine's own kernels call
// (strata/kernels/q8_1_finite.hpp, qw:10-13, used at qw:650-653, 684-688, 699-703), with the Q8_1 policy of
// librapier_mi's quantizer, so blocks written by an engine kernel and by rmi_native_quantize_q8_1 are the same bytes:
//   d = amax / 127 in fp32 (q8_1_finite keeps it as computed), q = round-half-away(v / d) (0 when amax is 0),
//   ds = (fp16 d, fp16 sum), each rounded to nearest even and saturated to +-65504 so a block stays finite.
// HIP device code: include from a file compiled with hipcc.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

namespace strata::kernels {

__host__ __device__ inline float q8_1_finite(float d) { return d; }

__host__ __device__ inline int8_t q8_1_quant(float v, float d, float amax) {
    return amax == 0.0f ? int8_t(0) : static_cast<int8_t>(static_cast<int>(roundf(v / d)));
}

__host__ __device__ inline __half q8_1_half_sat(float v) {
    return __float2half_rn(fminf(fmaxf(v, -65504.0f), 65504.0f));
}

__host__ __device__ inline __half2 q8_1_ds(float d, float sum) {
    return __halves2half2(q8_1_half_sat(d), q8_1_half_sat(sum));
}

}  // namespace strata::kernels
