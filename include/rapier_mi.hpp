// rapier_mi.hpp - header-only C++ shim: the reference's strata::kernels launch surface (same names, signatures and
// error behaviour) implemented over the C ABI of librapier_mi.so (rapier_mi.h).  An engine written against the
// reference's headers (native_mmvq.hpp, fused_gdn.hpp as used by src/qwythos.cpp) compiles against this file instead.
//
// Error behaviour, as in the reference:
//   MMVQ family (mmvq:2312-2331): std::invalid_argument for shape / ncols / pointer / null-stream errors,
//   std::runtime_error for a failed launch.
//   fused_gdn family (fgdn:169-175, 194-204): message on stderr and std::exit(1).
//   RoPE, per-row norm and elementwise calls: as the MMVQ family (their strata definitions are absent from the
//   reference tree).
// The device-side Q8_1 helpers the reference's own kernels call (q8_1_finite / q8_1_quant / q8_1_ds, qw:10-13) are in
// rapier_mi_q8_1.hpp (HIP device code).
#pragma once

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <stdexcept>
#include <string>

#include "rapier_mi.h"

namespace strata::kernels {

namespace rmi_detail {
inline void check_mmvq(int rc) {
    if (rc == RMI_OK) return;
    if (rc == RMI_ERR_LAUNCH || rc == RMI_ERR_STATE) throw std::runtime_error(rmi_last_error());
    throw std::invalid_argument(rmi_last_error());
}
inline void check_exit(int rc) {
    if (rc == RMI_OK) return;
    std::fprintf(stderr, "%s\n", rmi_last_error());
    std::exit(1);
}
}  // namespace rmi_detail

// mmvq:3054-3057
inline std::size_t native_q8_1_bytes(int n_in, int ncols) {
    const std::size_t n = rmi_native_q8_1_bytes(n_in, ncols);
    if (n == 0) throw std::invalid_argument(rmi_last_error());
    return n;
}
// mmvq:3059-3071
inline void native_quantize_q8_1(const float* x, void* x_q8_1, int n_in, int ncols, void* stream) {
    rmi_detail::check_mmvq(rmi_native_quantize_q8_1(x, x_q8_1, n_in, ncols, stream));
}
// mmvq:3627-3660
inline void native_q6_k_mmvq(const void* w, const void* x_q8_1, float* y, int n_in, int n_out, int ncols,
                             void* stream) {
    rmi_detail::check_mmvq(rmi_native_q6_k_mmvq(w, x_q8_1, y, n_in, n_out, ncols, stream));
}
// mmvq:3187-3200 (header patches/0002:9-24)
inline void native_q6_k_mmvq_res(const void* w, const void* x_q8_1, float* y, const float* res, float* partials,
                                 int n_in, int n_out, void* stream) {
    rmi_detail::check_mmvq(rmi_native_q6_k_mmvq_res(w, x_q8_1, y, res, partials, n_in, n_out, stream));
}
// mmvq:2922-2928: the opt-in switch the reference's engine reads before it packs (STRATA_Q6_PACKED=1)
inline bool native_q6_k_packed_enabled() {
    static const bool enabled = [] {
        const char* v = std::getenv("STRATA_Q6_PACKED");
        return v && v[0] == '1' && v[1] == '\0';
    }();
    return enabled;
}
// mmvq:2930-2960: a library-owned packed copy that native_q6_k_mmvq / _res then run on; false where the packed layout
// does not take the shape or the copy could not be made (the GGUF-layout kernels keep running), one stderr line per copy
inline bool native_q6_k_pack(const void* weights, int n_in, int n_out, const char* what) {
    const int before = rmi_native_q6_k_packed_copies();
    if (rmi_native_q6_k_pack_copy(weights, n_in, n_out) != RMI_OK) return false;
    if (rmi_native_q6_k_packed_copies() != before)
        std::fprintf(stderr, "rapier_mi: packed the %s (%d x %d) into a wave-tile copy\n", what ? what : "matrix", n_out,
                     n_in);
    return true;
}
// mmvq:3042-3048
inline void native_q6_k_unpack(const void* weights) { rmi_detail::check_mmvq(rmi_native_q6_k_unpack(weights)); }
// mmvq:3732-3736
inline void native_q8_0_mmvq(const void* w, const void* x_q8_1, float* y, int n_in, int n_out, int ncols,
                             void* stream) {
    rmi_detail::check_mmvq(rmi_native_q8_0_mmvq(w, x_q8_1, y, n_in, n_out, ncols, stream));
}
// mmvq:3326-3339
inline void native_q8_0_mmvq_res(const void* w, const void* x_q8_1, float* y, const float* res, float* partials,
                                 int n_in, int n_out, void* stream) {
    rmi_detail::check_mmvq(rmi_native_q8_0_mmvq_res(w, x_q8_1, y, res, partials, n_in, n_out, stream));
}
// mmvq:3587-3612, 3341-3366 (Q5_K_M matrices)
inline void native_q4_k_mmvq(const void* w, const void* x_q8_1, float* y, int n_in, int n_out, int ncols,
                             void* stream) {
    rmi_detail::check_mmvq(rmi_native_q4_k_mmvq(w, x_q8_1, y, n_in, n_out, ncols, stream));
}
inline void native_q5_k_mmvq(const void* w, const void* x_q8_1, float* y, int n_in, int n_out, int ncols,
                             void* stream) {
    rmi_detail::check_mmvq(rmi_native_q5_k_mmvq(w, x_q8_1, y, n_in, n_out, ncols, stream));
}
// mmvq:3296-3324
inline void native_q4_k_mmvq_res(const void* w, const void* x_q8_1, float* y, const float* res, float* partials,
                                 int n_in, int n_out, void* stream) {
    rmi_detail::check_mmvq(rmi_native_q4_k_mmvq_res(w, x_q8_1, y, res, partials, n_in, n_out, stream));
}
inline void native_q5_k_mmvq_res(const void* w, const void* x_q8_1, float* y, const float* res, float* partials,
                                 int n_in, int n_out, void* stream) {
    rmi_detail::check_mmvq(rmi_native_q5_k_mmvq_res(w, x_q8_1, y, res, partials, n_in, n_out, stream));
}
// mmvq:3787-3818
inline void native_mmvq(int ggml_type, const void* w, const void* x_q8_1, float* y, int n_in, int n_out, int ncols,
                        void* stream) {
    rmi_detail::check_mmvq(rmi_native_mmvq(ggml_type, w, x_q8_1, y, n_in, n_out, ncols, stream));
}
inline bool native_mmvq_supported(int ggml_type) noexcept { return rmi_native_mmvq_supported(ggml_type) != 0; }
inline std::size_t native_mmvq_weight_bytes(int ggml_type, int n_in, int n_out) {
    const std::size_t n = rmi_native_mmvq_weight_bytes(ggml_type, n_in, n_out);
    if (n == 0) throw std::invalid_argument(rmi_last_error());
    return n;
}
// fgdn:167-176
inline void fused_gdn_conv_l2(float* history, const float* qkv, const float* conv_w, float* h, int channels,
                              int qk_heads, float eps, void* stream) {
    rmi_detail::check_exit(rmi_fused_gdn_conv_l2(history, qkv, conv_w, h, channels, qk_heads, eps, stream));
}
// fgdn:221-225 (header patches/0001:9-15)
inline void fused_gdn_step_norm_silu_q8(float* state, const float* q, const float* k, const float* v,
                                        const float* gate, const float* beta, const float* z, const float* gamma,
                                        float eps, float* y, uint8_t* q8, int h_k, int h_v, void* stream) {
    rmi_detail::check_exit(
        rmi_fused_gdn_step_norm_silu_q8(state, q, k, v, gate, beta, z, gamma, eps, y, q8, h_k, h_v, stream));
}

// RoPE configuration as the reference fills it for qwen35 (qw:280, 1991-1999).  strata's own definition is absent
// from the reference tree: these are the members the reference sets; RopeScalingType::None is plain NEOX RoPE.
enum class RopeScalingType { None, YaRN };
struct RopeScaling {
    RopeScalingType type = RopeScalingType::None;
    float freq_base = 10000.0f;
    float factor = 1.0f;
    float orig_ctx = 0.0f;
    float ext_factor = 0.0f;
    float attn_factor = 1.0f;
    float beta_fast = 32.0f;
    float beta_slow = 1.0f;
};
// qw:1165-1166, 1357-1358, 1542-1544, 2380-2407: heads rows of head_dim, head h at position pos[h] (device)
inline void native_rope_apply(const float* x, float* y, int heads, int head_dim, int n_rot, const RopeScaling& rope,
                              const int* pos, void* stream) {
    const bool yarn = rope.type == RopeScalingType::YaRN;
    const rmi_rope_params p{rope.freq_base, yarn ? rope.factor : 1.0f, rope.orig_ctx, rope.ext_factor,
                            rope.attn_factor, rope.beta_fast, rope.beta_slow};
    rmi_detail::check_mmvq(rmi_native_rope_apply(x, y, heads, head_dim, n_rot, &p, pos, stream));
}
// qw:971-975
inline void rms_norm_weighted(float* x, const float* w, int rows, int cols, float eps, void* stream) {
    rmi_detail::check_mmvq(rmi_rms_norm_weighted(x, w, rows, cols, eps, stream));
}
// qw:1002, 1068, 1178 (x += y), 1059 (x *= s), 1053 (x = silu(x))
inline void add_inplace(float* x, const float* y, int n, void* stream) {
    rmi_detail::check_mmvq(rmi_add_inplace(x, y, n, stream));
}
inline void scale_inplace(float* x, int n, float s, void* stream) {
    rmi_detail::check_mmvq(rmi_scale_inplace(x, n, s, stream));
}
inline void silu_inplace(float* x, int n, void* stream) { rmi_detail::check_mmvq(rmi_silu_inplace(x, n, stream)); }

}  // namespace strata::kernels
