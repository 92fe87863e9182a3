/*
 * rapier_mi.h - C ABI of the MI355X-native exact-verify MTP hot path (librapier_mi.so, gfx950).
 *
 * Every entry point replaces one launch-level function of Rapier's engine (reference paths are given as
 * file:line; "mmvq" = src/native_mmvq.cu, "fgdn" = src/fused_gdn.cu, "qw" = src/qwythos.cpp).  Layouts are the
 * reference's: GGUF Q6_K / Q8_0 weight blocks row-major, Q8_1 activation blocks column-major by block (column j at
 * block j * n_in/32), outputs column j at y + j * n_out, one partials slot per 4 output rows.
 *
 * Conventions:
 *   - all pointers are device pointers owned by the caller; no entry point allocates, frees or synchronizes;
 *   - `stream` is a hipStream_t; work is enqueued asynchronously and is stream-capture safe;
 *   - the return value is RMI_OK or an error code; rmi_last_error() returns the message of the calling thread's
 *     last failure.  include/rapier_mi.hpp rethrows these with the reference's exception types.
 */
#ifndef RAPIER_MI_H
#define RAPIER_MI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    RMI_OK = 0,
    RMI_ERR_SHAPE = 1,       /* std::invalid_argument in the reference: bad n_in / n_out / ncols / heads */
    RMI_ERR_POINTER = 2,     /* std::invalid_argument: null or misaligned device pointer */
    RMI_ERR_STREAM = 3,      /* std::invalid_argument: null stream where the reference requires one */
    RMI_ERR_LAUNCH = 4,      /* std::runtime_error: the HIP launch failed */
    RMI_ERR_UNSUPPORTED = 5, /* std::invalid_argument: unsupported GGML type */
    RMI_ERR_STATE = 6        /* engine misuse (context full, bad token, not built) */
};

const char* rmi_last_error(void);
const char* rmi_version(void);

/* ---------------------------------------------------------------------------------------------------------------
 * Q8_1 activations
 * ------------------------------------------------------------------------------------------------------------- */

/* bytes of ncols Q8_1 columns of n_in elements.  Replaces strata::kernels::native_q8_1_bytes (mmvq:3054-3057);
 * returns 0 on a bad shape. */
size_t rmi_native_q8_1_bytes(int n_in, int ncols);

/* fp32 x[ncols][n_in] -> Q8_1.  Replaces native_quantize_q8_1 (mmvq:3059-3071, kernel mmvq:158-173). */
int rmi_native_quantize_q8_1(const float* x, void* x_q8_1, int n_in, int ncols, void* stream);

/* ---------------------------------------------------------------------------------------------------------------
 * Quantized GEMV (MMVQ): y[j][r] = sum_k W[r][k] * x_j[k]
 * ------------------------------------------------------------------------------------------------------------- */

/* Q6_K x Q8_1, 1 <= ncols <= 16.  Replaces native_q6_k_mmvq (mmvq:3627-3660; kernels mmvq:753-789 at ncols = 1
 * and native_mmvq_multi_kernel mmvq:1261-1356 at ncols >= 2).  Every column of an ncols >= 2 call is bitwise
 * the ncols = 1 result on that column. */
int rmi_native_q6_k_mmvq(const void* w, const void* x_q8_1, float* y, int n_in, int n_out, int ncols, void* stream);

/* Residual epilogue, ncols = 1: y[r] = acc + res[r] (y may alias res), partials[r/4] = sum of the 4 rows' y^2.
 * partials has ceil(n_out/4) slots.  Replaces native_q6_k_mmvq_res (mmvq:3187-3200, kernel mmvq:3096-3140). */
int rmi_native_q6_k_mmvq_res(const void* w, const void* x_q8_1, float* y, const float* res, float* partials,
                             int n_in, int n_out, void* stream);

/* Residual epilogue at ncols columns: column j uses res + j*n_out, y + j*n_out, partials + j*ceil(n_out/4).
 * No reference counterpart: the reference's verify pass runs mm_q2 and then add_partials_1024_kernel per column
 * (qw:1489-1494, 1512-1517); this fuses both, and column j equals rmi_native_q6_k_mmvq_res on that column. */
int rmi_native_q6_k_mmvq_res_n(const void* w, const void* x_q8_1, float* y, const float* res, float* partials,
                               int n_in, int n_out, int ncols, void* stream);

/* Q8_0 x Q8_1.  Replaces native_q8_0_mmvq (mmvq:3732-3736; dot mmvq:835-847) and native_q8_0_mmvq_res
 * (mmvq:3326-3339, kernel mmvq:3142-3185). */
int rmi_native_q8_0_mmvq(const void* w, const void* x_q8_1, float* y, int n_in, int n_out, int ncols, void* stream);
int rmi_native_q8_0_mmvq_res(const void* w, const void* x_q8_1, float* y, const float* res, float* partials,
                             int n_in, int n_out, void* stream);
int rmi_native_q8_0_mmvq_res_n(const void* w, const void* x_q8_1, float* y, const float* res, float* partials,
                               int n_in, int n_out, int ncols, void* stream);

/* Type-dispatched GEMV (GGML type 14 = Q6_K, 8 = Q8_0; others RMI_ERR_UNSUPPORTED).  Replaces native_mmvq
 * (mmvq:3787-3818), including its split of more than 16 columns into passes. */
int rmi_native_mmvq(int ggml_type, const void* w, const void* x_q8_1, float* y, int n_in, int n_out, int ncols,
                    void* stream);
int rmi_native_mmvq_supported(int ggml_type);
/* weight bytes of an n_out x n_in matrix (native_mmvq_weight_bytes, mmvq:3758-3785); 0 on a bad shape */
size_t rmi_native_mmvq_weight_bytes(int ggml_type, int n_in, int n_out);

/* Integer block dot products of the Q6_K x Q8_1 core, out[r][j] = sum over Q8_1 block j of sc * (q6 - 32) * q8
 * (exact int32), one column.  Exposes the integer stage of q6_q8_dot_impl (mmvq:642-655) for bit-exact checks;
 * it runs the same device decode as the GEMV. */
int rmi_q6_k_block_dots(const void* w, const void* x_q8_1, int32_t* out, int n_in, int n_out, void* stream);

#ifdef __cplusplus
}
#endif
#endif
