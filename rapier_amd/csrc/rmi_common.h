// rmi_common.h - shared definitions for the MI355X (gfx950) kernels behind the rapier_mi C ABI.
//
// Block formats are GGUF's (reference src/native_mmvq.cu:98-140): Q6_K 210 B per 256 weights, Q8_0 34 B per 32,
// Q8_1 activations 36 B per 32 (fp16 d, fp16 sum, 32 int8 codes).  Everything here is wave64 CDNA4 code.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/rapier_mi.h"

namespace rmi {

constexpr int kQ6KBytes = 210;
constexpr int kQ8_0Bytes = 34;
constexpr int kQ8_1Bytes = 36;
constexpr int kMaxCols = 16;   // the reference's validate_shape limit (mmvq:2312-2318)

// ---- error reporting: the C ABI returns codes, the message of the last failure is kept per thread ----
void set_error(const char* msg);
int fail(int code, const char* msg);
int launch_status(const char* what);   // hipGetLastError after a launch -> RMI_ERR_LAUNCH with the HIP message

// return the status of a call that failed
#define RMI_TRY(expr)                  \
    do {                               \
        const int rc_ = (expr);        \
        if (rc_ != RMI_OK) return rc_; \
    } while (0)

inline bool aligned4(const void* p) { return p && (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }
inline bool aligned16(const void* p) { return p && (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---- device helpers ----
__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits & 0xffffu)));
}

// fp16 store with the Q8_1 finite policy: round to nearest even, saturated to +-65504
__device__ __forceinline__ uint32_t float_to_half_sat(float v) {
    v = fminf(fmaxf(v, -65504.0f), 65504.0f);
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(v)));
}

// The value of lane l ^ K (K = 1, 2, 4, 8, 16, 32) on the VALU, the partner __shfl_xor would fetch through the LDS
// unit: DPP within a row of 16 lanes (quad permutes; row shifts by 4 picked by lane bit 2, since a row shift reads
// lane l + 4 / l - 4; a row rotation by 8), and gfx950's lane swaps across rows (v_permlane16_swap pairs rows 0-1 and
// 2-3, v_permlane32_swap the two halves; each returns both rows side by side).  The partner lane must be active.
template <int K>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
    const int x = static_cast<int>(v);
    if constexpr (K == 1) {
        return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, x, 0xb1, 0xf, 0xf, false));   // quad_perm 1,0,3,2
    } else if constexpr (K == 2) {
        return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, x, 0x4e, 0xf, 0xf, false));   // quad_perm 2,3,0,1
    } else if constexpr (K == 4) {
        const int up = __builtin_amdgcn_update_dpp(0, x, 0x104, 0xf, 0xf, false);   // row_shl:4 - lane l + 4
        const int dn = __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);   // row_shr:4 - lane l - 4
        return static_cast<uint32_t>((__lane_id() & 4) ? dn : up);
    } else if constexpr (K == 8) {
        return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, x, 0x128, 0xf, 0xf, false));  // row_ror:8
    } else if constexpr (K == 16) {
        const auto a = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (__lane_id() & 16) ? a[0] : a[1];
    } else {
        static_assert(K == 32, "xor_lane: K must be 1, 2, 4, 8, 16 or 32");
        const auto a = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (__lane_id() & 32) ? a[0] : a[1];
    }
}
template <int K>
__device__ __forceinline__ float xor_lane(float v) {
    return __uint_as_float(xor_lane<K>(__float_as_uint(v)));
}

// member K of the lane's quad (lanes 4 (l / 4) + K), by a DPP quad broadcast
template <int K>
__device__ __forceinline__ float quad_lane(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), K * 0x55, 0xf, 0xf, false));
}

// xor butterfly over groups of W lanes (offsets W / 2 .. 1); every lane of a group ends with the same value
template <int W>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (W >= 64) v += xor_lane<32>(v);
    if constexpr (W >= 32) v += xor_lane<16>(v);
    if constexpr (W >= 16) v += xor_lane<8>(v);
    if constexpr (W >= 8) v += xor_lane<4>(v);
    if constexpr (W >= 4) v += xor_lane<2>(v);
    if constexpr (W >= 2) v += xor_lane<1>(v);
    return v;
}
template <int W>
__device__ __forceinline__ float group_max(float v) {
    if constexpr (W >= 64) v = fmaxf(v, xor_lane<32>(v));
    if constexpr (W >= 32) v = fmaxf(v, xor_lane<16>(v));
    if constexpr (W >= 16) v = fmaxf(v, xor_lane<8>(v));
    if constexpr (W >= 8) v = fmaxf(v, xor_lane<4>(v));
    if constexpr (W >= 4) v = fmaxf(v, xor_lane<2>(v));
    if constexpr (W >= 2) v = fmaxf(v, xor_lane<1>(v));
    return v;
}

// Quantizes one value per lane into the Q8_1 block its 32-lane group owns (lane & 31 = element).
// d = amax / 127 in fp32, q = roundf(v / d) (0 for an all-zero block), ds = (fp16 d, fp16 sum) saturated.
// amax and sum use the 32-lane xor butterfly, so every finite block has one defined bit pattern.
__device__ __forceinline__ void q8_1_store_lane(float v, uint8_t* block) {
    const float amax = group_max<32>(fabsf(v));
    const float sum = group_sum<32>(v);
    const float d = amax / 127.0f;
    const int q = amax == 0.0f ? 0 : static_cast<int>(roundf(v / d));
    const int lane = threadIdx.x & 31;
    block[4 + lane] = static_cast<uint8_t>(static_cast<int8_t>(q));
    if (lane == 0) {
        *reinterpret_cast<uint32_t*>(block) = float_to_half_sat(d) | (float_to_half_sat(sum) << 16);
    }
}

// roundf(v / d) of the Q8_1 quantizer (d = amax / 127 with |v| <= amax) with a multiply in place of the divide:
// y = v * inv_d, inv_d = 1 / d correctly rounded once per block, lies within 2.3e-5 of the correctly rounded quotient,
// so rounding y gives roundf(v / d) unless y is within 2^-14 of a half-integer - and away from the half-integers
// round-half-even (rint, one instruction) and roundf's round-half-away agree.  Returns rint(y) and sets slow when the
// caller must take roundf(v / d) instead (those values, and blocks whose d is not a normal number).  Checked for every
// float v with |v| <= 128 d at a spread of d against roundf(v / d) (tests/cpp/q8_round_check.c).
__device__ __forceinline__ float q8_round_fast(float v, float d, float inv_d, bool& slow) {
    const float y = v * inv_d;
    const float fr = __builtin_amdgcn_fractf(fabsf(y));   // |y| - floor(|y|), exact for |y| >= 0
    slow = !(fabsf(fr - 0.5f) > 0x1p-14f) || !(d >= 0x1p-126f && d <= 0x1p126f);
    return __builtin_rintf(y);
}

// ---- the row-norm reduction over 4-row partials ------------------------------------------------------------------
// One tree for every kernel that derives a norm's inv = rsqrt(sum / cols + eps) from a vector's 4-row partials
// (rms_quant_apply, rms_norm_out, and the GEMVs that quantize a norm in their stage), so they all get the same bits:
// 256 lanes (waves 0..3); lane t adds slots t, t + 256, t + 512, ... in order starting from 0, a 64-lane xor butterfly,
// then the four wave sums in wave order.  A lane's first kNormLoads slots are loaded before the first add (clamped,
// unconditional: a strided loop or a load under a branch waits on each load in turn).
constexpr int kNormLoads = 8;

struct NormLoads {
    float v[kNormLoads];
};

__device__ __forceinline__ void norm_load(NormLoads& pv, const float* __restrict__ p, int np, int t) {
#pragma unroll
    for (int k = 0; k < kNormLoads; ++k) pv.v[k] = p[min(t + 256 * k, np - 1)];
}

// the lane's ordered sum and the wave's butterfly; every lane of the wave ends with the wave sum
__device__ __forceinline__ float norm_wave_sum(const NormLoads& pv, const float* __restrict__ p, int np, int t) {
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < kNormLoads; ++k)
        if (t + 256 * k < np) s += pv.v[k];
    for (int i = t + 256 * kNormLoads; i < np; i += 256) s += p[i];
    return group_sum<64>(s);
}

__device__ __forceinline__ float norm_inv(const float* red, int cols, float eps) {
    const float tot = ((red[0] + red[1]) + red[2]) + red[3];
    return rsqrtf(tot / static_cast<float>(cols) + eps);
}

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }

// The drop-in entry points' packed copy (rmi_native_q6_k_pack_copy): runs the packed GEMV (res null: plain) when w has
// a registered copy of this shape, else returns -1 and launches nothing
int registry_mmvq(const void* w, const void* x_q8_1, float* y, const float* res, float* partials, int n_in, int n_out,
                  int ncols, void* stream);

// GGUF-layout stream GEMV (mmvq_q6k_packed.hip) for the drop-in entry points: returns -1, launching nothing, for shapes
// it does not take (rows other than 4096 / 8192 / 12288 elements, more than four columns, a matrix not 16-byte aligned)
int gguf_stream_gemv(const uint8_t* w, const uint8_t* x, float* y, const float* res, float* partials, int n_in,
                     int n_out, int ncols, hipStream_t s);

}  // namespace rmi
