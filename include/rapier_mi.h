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
    RMI_ERR_STATE = 6        /* engine misuse (context full, bad token, not built), or a GDN exchange wait that timed out */
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

/* Packed Q6_K: a caller-owned copy of an n_out x n_in Q6_K matrix re-laid in (4-row, 8-block) wave tiles so a
 * wave loads each lane's half-block with contiguous 1 KB accesses (layout in mmvq_q6k_packed.hip).  Replaces the
 * reference's registry-owned packed copy (native_q6_k_pack, mmvq:2930-3040; looked up by native_q6_k_mmvq at
 * mmvq:3629).  n_in a multiple of 2048; packed bytes are 6720 per (4 rows x 2048 elements), the last 4-row group
 * zero-padded.  The packed GEMVs give, bit for bit, the results of the 16-row tiled kernel (every column of an
 * ncols >= 2 call equal to the ncols = 1 call; _res_n equal to plain + res with one partial per 4 rows). */
size_t rmi_q6_k_packed_bytes(int n_in, int n_out);
int rmi_q6_k_pack(const void* w, void* w_packed, int n_in, int n_out, void* stream);
/* The reference's registry-owned copy itself (native_q6_k_pack, mmvq:2930-2960; native_q6_k_unpack, mmvq:3042-3048):
 * the library packs the GGUF-layout matrix w into a copy of its own (synchronously: every stream of the device drains
 * first, as the reference's host round trip does), and from then on rmi_native_q6_k_mmvq, _res and _res_n called with
 * w and the same shape run the packed kernels on that copy (the same bits), as native_q6_k_mmvq looks up its registry
 * first (mmvq:3629).  RMI_OK when packed or packed already; RMI_ERR_UNSUPPORTED for shapes the packed layout does not
 * take (n_in not a multiple of 2048: the GGUF-layout kernels keep running); RMI_ERR_STATE when w is packed with
 * another shape.  rmi_native_q6_k_unpack frees the copy (a no-op for weights without one) after draining the device.
 * rmi_native_q6_k_packed_copies counts the copies held. */
int rmi_native_q6_k_pack_copy(const void* w, int n_in, int n_out);
int rmi_native_q6_k_unpack(const void* w);
int rmi_native_q6_k_packed_copies(void);
/* No counterpart in the reference (a fusion of its up/gate GEMVs, mmvq:1261-1356, with swiglu_quant_kernel,
 * qw:676-689).  Packs an up||gate Q6_K matrix (2 n_ff rows: up rows, then gate rows) in the SwiGLU row order:
 * packed rows 64 G .. 64 G + 31 are gate rows 32 G .., rows 64 G + 32 .. 64 G + 63 up rows 32 G ...  n_ff a multiple
 * of 32; the buffer is rmi_q6_k_packed_bytes(n_in, 2 n_ff).  A plain packed GEMV over it returns the rows in that
 * order (rmi_swiglu_quant_interleaved takes them). */
int rmi_q6_k_pack_swiglu(const void* w, void* w_packed, int n_in, int n_ff, void* stream);
/* No counterpart in the reference (see rmi_q6_k_pack_swiglu).  Q8_1 of silu(gate) * up for 1 or 2 columns straight
 * from the SwiGLU-packed up||gate matrix, n_in = 4096: bitwise the packed GEMV followed by rmi_swiglu_quant, in one
 * launch and with no fp32 up / gate rows in memory. */
int rmi_native_q6_k_swiglu_packed(const void* w_packed, const void* x_q8_1, void* y_q8_1, int n_in, int n_ff,
                                  int ncols, void* stream);
/* The reference's norm + GEMV launch pair, rms_quant_apply_kernel (qw:627-655) then native_q6_k_mmvq (mmvq:3627) or
 * the up / gate GEMVs with swiglu_quant_kernel (qw:676-689), as one launch: the GEMV's workgroups quantize
 * (x * w_norm) * inv, inv = rsqrt(sum of x's 4-row partials / n_in + eps) by rms_quant_apply's reduction tree, straight
 * into their activation stage.  Bitwise equal to rmi_rms_quant_apply followed by rmi_native_q6_k_mmvq_packed /
 * rmi_native_q6_k_swiglu_packed on its Q8_1 output.  x: ncols fp32 columns of n_in (column j at x + j n_in), 16-byte
 * aligned, as is w_norm; partials: ncols columns of n_in / 4 slots.  n_in = 4096, ncols 1 or 2 (and n_out <= 32768 for
 * the plain GEMV). */
int rmi_native_q6_k_mmvq_packed_norm(const void* w_packed, const float* x, const float* w_norm, const float* partials,
                                     float eps, float* y, int n_in, int n_out, int ncols, void* stream);
int rmi_native_q6_k_swiglu_packed_norm(const void* w_packed, const float* x, const float* w_norm,
                                       const float* partials, float eps, void* y_q8_1, int n_in, int n_ff, int ncols,
                                       void* stream);
/* 1 where rmi_native_q6_k_mmvq_packed_norm is measured faster than the two launches it replaces (its 8-wave workgroups
 * of 16 row quads cover at least 3/4 of the CUs, or 4-wave workgroups of up to 4 quads per wave can), else 0 (also for
 * shapes it does not take). */
int rmi_q6_k_packed_norm_preferred(int n_in, int n_out, int ncols);
int rmi_native_q6_k_mmvq_packed(const void* w_packed, const void* x_q8_1, float* y, int n_in, int n_out, int ncols,
                                void* stream);
int rmi_native_q6_k_mmvq_packed_res_n(const void* w_packed, const void* x_q8_1, float* y, const float* res,
                                      float* partials, int n_in, int n_out, int ncols, void* stream);

/* Q8_0 x Q8_1.  Replaces native_q8_0_mmvq (mmvq:3732-3736; dot mmvq:835-847) and native_q8_0_mmvq_res
 * (mmvq:3326-3339, kernel mmvq:3142-3185). */
int rmi_native_q8_0_mmvq(const void* w, const void* x_q8_1, float* y, int n_in, int n_out, int ncols, void* stream);
int rmi_native_q8_0_mmvq_res(const void* w, const void* x_q8_1, float* y, const float* res, float* partials,
                             int n_in, int n_out, void* stream);
int rmi_native_q8_0_mmvq_res_n(const void* w, const void* x_q8_1, float* y, const float* res, float* partials,
                               int n_in, int n_out, int ncols, void* stream);

/* Q4_K / Q5_K x Q8_1 GEMV, ncols 1..16, plain and with the residual + partials epilogue (the matrices of Q5_K_M
 * files).  Replace native_q4_k_mmvq / native_q5_k_mmvq (mmvq:562-640, 185-300, 3587-3624, 3341-3379) and
 * native_q4_k_mmvq_res / native_q5_k_mmvq_res (mmvq:3202-3324); the _res_n forms take ncols columns in one call.
 * The matrix is 16-byte aligned (every GGUF row is: 144 and 176 bytes per block); n_in <= 52224. */
int rmi_native_q4_k_mmvq(const void* w, const void* x_q8_1, float* y, int n_in, int n_out, int ncols, void* stream);
int rmi_native_q5_k_mmvq(const void* w, const void* x_q8_1, float* y, int n_in, int n_out, int ncols, void* stream);
int rmi_native_q4_k_mmvq_res(const void* w, const void* x_q8_1, float* y, const float* res, float* partials, int n_in,
                             int n_out, void* stream);
int rmi_native_q5_k_mmvq_res(const void* w, const void* x_q8_1, float* y, const float* res, float* partials, int n_in,
                             int n_out, void* stream);
int rmi_native_q4_k_mmvq_res_n(const void* w, const void* x_q8_1, float* y, const float* res, float* partials,
                               int n_in, int n_out, int ncols, void* stream);
int rmi_native_q5_k_mmvq_res_n(const void* w, const void* x_q8_1, float* y, const float* res, float* partials,
                               int n_in, int n_out, int ncols, void* stream);

/* Type-dispatched GEMV (GGML type 14 = Q6_K, 13 = Q5_K, 12 = Q4_K, 8 = Q8_0; others RMI_ERR_UNSUPPORTED).
 * Replaces native_mmvq (mmvq:3787-3818), including its split of more than 16 columns into passes. */
int rmi_native_mmvq(int ggml_type, const void* w, const void* x_q8_1, float* y, int n_in, int n_out, int ncols,
                    void* stream);
int rmi_native_mmvq_supported(int ggml_type);
/* weight bytes of an n_out x n_in matrix (native_mmvq_weight_bytes, mmvq:3758-3785); 0 on a bad shape */
size_t rmi_native_mmvq_weight_bytes(int ggml_type, int n_in, int n_out);

/* Integer block dot products of the Q6_K x Q8_1 core, out[r][j] = sum over Q8_1 block j of sc * (q6 - 32) * q8
 * (exact int32), one column.  Exposes the integer stage of q6_q8_dot_impl (mmvq:642-655) for bit-exact checks;
 * it runs the same device decode as the GEMV. */
int rmi_q6_k_block_dots(const void* w, const void* x_q8_1, int32_t* out, int n_in, int n_out, void* stream);

/* ---------------------------------------------------------------------------------------------------------------
 * Norm / activation epilogues (qw:602-715).  `ncols` columns per launch; column c of x at x + c * cols, of partials
 * at partials + c * cols / 4, of Q8_1 output at c * cols / 32 blocks.  Partials: one slot per 4 rows.
 * ------------------------------------------------------------------------------------------------------------- */

/* Q8_1 of (x * w) * rsqrt(sum(partials) / cols + eps).  Replaces rms_quant_apply_kernel (qw:627-655). */
int rmi_rms_quant_apply(const float* x, const float* w, const float* partials, void* y_q8_1, int cols, float eps,
                        int ncols, void* stream);
/* No counterpart in the reference: rmi_row_sum_partials(x) followed by rmi_rms_quant_apply, in one launch and with the
 * same bytes - each workgroup forms the 4-row partials from x itself.  For a vector whose partials no GEMV epilogue
 * wrote (x 16-byte aligned). */
int rmi_rms_quant_apply_self(const float* x, const float* w, void* y_q8_1, int cols, float eps, int ncols,
                             void* stream);
/* Two rmi_rms_quant_apply results of cols each into the two halves of one 2 cols Q8_1 row per column (x0 -> blocks
 * [0, cols/32), x1 -> [cols/32, cols/16)).  No counterpart in the reference: it replaces its two rms_norm_out calls
 * and the quantize of their concatenation in the draft's input (qw:1327-1332), with the same bits. */
int rmi_rms_quant_apply_pair(const float* x0, const float* w0, const float* partials0, const float* x1,
                             const float* w1, const float* partials1, void* y_q8_1, int cols, float eps, int ncols,
                             void* stream);
/* fp32 out = (x * w) * rsqrt(...); out_partials (nullable) gets the output's own 4-row partials.
 * Replaces rms_norm_out_kernel (qw:658-672) fused with row_sum_partials_kernel (qw:616-623). */
int rmi_rms_norm_out(const float* x, const float* w, const float* partials, float* out, float* out_partials, int cols,
                     float eps, int ncols, void* stream);
/* the same with column c of out at out + c * out_stride (the draft's [enorm(emb) | hnorm(h)] concat, qw:1327-1332) */
int rmi_rms_norm_out_strided(const float* x, const float* w, const float* partials, float* out, int out_stride,
                             float* out_partials, int cols, float eps, int ncols, void* stream);
/* partials of x.  Replaces row_sum_partials_kernel (qw:616-623). */
int rmi_row_sum_partials(const float* x, float* partials, int n, int ncols, void* stream);
/* x += o, then partials of x.  Replaces add_partials_1024_kernel (qw:602-614). */
int rmi_add_partials(float* x, const float* o, float* partials, int n, int ncols, void* stream);
/* Q8_1 of silu(gate) * up; column c reads up/gate at + c * col_stride.  Replaces swiglu_quant_kernel (qw:676-689). */
int rmi_swiglu_quant(const float* up, const float* gate, void* y_q8_1, int n, int ncols, int col_stride, void* stream);
/* rmi_swiglu_quant over up||gate rows in the SwiGLU order of rmi_q6_k_pack_swiglu (column c at up_gate + c col_stride,
 * col_stride >= 2 n).  No counterpart in the reference (its rows are never interleaved). */
int rmi_swiglu_quant_interleaved(const float* up_gate, void* y_q8_1, int n, int ncols, int col_stride, void* stream);
/* Q8_1 of o * sigmoid(g).  Replaces sig_mul_quant_kernel (qw:692-704). */
int rmi_sig_mul_quant(const float* o, const float* g, void* y_q8_1, int n, int ncols, int o_stride, int g_stride,
                      void* stream);
/* beta = sigmoid(beta) in place, ggate = softplus(alpha + dt) * ssm_a; per column [beta n | alpha n] (the
 * reference's beta|alpha concat order, qw:2085).  Replaces beta_gate_kernel (qw:707-715). */
int rmi_beta_gate(float* beta_alpha, const float* dt, const float* ssm_a, float* ggate, int n, int ncols,
                  int ab_stride, void* stream);
/* greedy argmax per column, lowest index wins ties; workspace of rmi_argmax_workspace_bytes(ncols) bytes.
 * Replaces argmax_kernel / serve_argmax_dev (qw:70-94) and the host scan (qw:3199-3205), without the memset. */
size_t rmi_argmax_workspace_bytes(int ncols);
int rmi_argmax(const float* logits, int n, int ncols, int col_stride, int* out_idx, void* workspace, void* stream);
/* the k largest of n logits (k <= 64, n <= 1048576) with their ids, logit descending, lower id first among equal
 * logits (-0 equals +0): out_idx[k] and out_val[k] on the device; workspace of rmi_topk_workspace_bytes(n) bytes.
 * Replaces topk_out's host scan (qw:2513-2531) and the 1 MB logits copy before it (qw:1800-1803). */
size_t rmi_topk_workspace_bytes(int n);
int rmi_topk(const float* logits, int n, int k, int* out_idx, float* out_val, void* workspace, void* stream);
/* Device-resident token embedding: x[c] = dequant(row tokens[c]) of a GGUF type 14 (Q6_K), 13 (Q5_K) or 12 (Q4_K)
 * table, partials of each row (4 elements per slot).  Replaces the host dequant + H2D copy of emb_dequant_block
 * (qw:109-115, 1418-1430); Q3_K and IQ4_XS tables are RMI_ERR_UNSUPPORTED. */
int rmi_embed(int type, const void* emb, const int* tokens, float* x, float* partials, int n_embd, int n_vocab,
              int ncols, void* stream);
/* rmi_embed of tokens[c] followed by rmi_rms_quant_apply_pair(emb rows, w0, their partials, x1, w1, partials1) in
 * one launch: the same Q8_1 bytes, without the fp32 embedding rows in HBM.  The draft's input (eh_proj over
 * [enorm(emb) | hnorm(h)], qw:1327-1332); cols a multiple of 256. */
int rmi_embed_quant_apply_pair(int type, const void* emb, const int* tokens, const float* w0, const float* x1,
                               const float* w1, const float* partials1, void* y_q8_1, int cols, int n_vocab, float eps,
                               int ncols, void* stream);
/* rmi_embed with type 14 */
int rmi_embed_q6_k(const void* emb, const int* tokens, float* x, float* partials, int n_embd, int n_vocab, int ncols,
                   void* stream);

/* ---------------------------------------------------------------------------------------------------------------
 * Gated DeltaNet (fgdn:40-133)
 * ------------------------------------------------------------------------------------------------------------- */

/* causal width-4 conv + SiLU + L2 of the first qk_heads 128-channel heads; history [c][3] updated in place, h may
 * alias qkv.  Replaces fused_gdn_conv_l2 (fgdn:167-176). */
int rmi_fused_gdn_conv_l2(float* history, const float* qkv, const float* conv_w, float* h, int channels, int qk_heads,
                          float eps, void* stream);
/* one delta-rule step per value head, state [128][h_v][128] in place, y = rmsnorm(o) * gamma * silu(z), q8 (nullable)
 * its Q8_1 blocks.  gate = decay logit (g = exp(gate)), beta after its sigmoid.  Replaces
 * fused_gdn_step_norm_silu_q8 (fgdn:221-225, patches/0001:9-15). */
int rmi_fused_gdn_step_norm_silu_q8(float* state, const float* q, const float* k, const float* v, const float* gate,
                                    const float* beta, const float* z, const float* gamma, float eps, float* y,
                                    uint8_t* q8, int h_k, int h_v, void* stream);
/* The whole GDN chain of one layer for ntok = 1 (decode) or 2 (verify) tokens in one launch: conv + SiLU + L2,
 * beta/decay from the raw beta|alpha GEMV output, the step with the state in registers across both tokens, norm *
 * silu gate, Q8_1.  qkvz and ab are read only.  The conv history is kept per value head, [h_v][q 128 | k 128 | v 128][3]
 * (value head h sees k-head h % h_k), so each of the two value heads of a k-head owns a copy of its q/k history.
 * state_a/state_b and hist_a/hist_b are the two buffers of the selector *sel (live = sel ? b : a).  With ntok = 2
 * the state and history after token 0 go to the non-live buffers, so a rejected draft is rolled back by flipping
 * *sel.  No reference counterpart as one call: replaces beta_gate + fused_gdn_conv_l2 + fused_gdn_step_norm_silu_q8
 * per column and the snapshot copies of launch_token_verify (qw:1448-1478, 3225-3233). */
int rmi_gdn_layer_tokens(float* state_a, float* state_b, float* hist_a, float* hist_b, const int* sel, float* qkvz,
                         int qkvz_stride, const float* ab, int ab_stride, const float* conv_w, const float* dt,
                         const float* ssm_a, const float* gamma, float eps, float* y, int y_stride, uint8_t* q8,
                         int q8_stride, int h_k, int h_v, int ntok, void* stream);
/* rmi_gdn_layer_tokens with the decode / verify launches (ntok 1 or 2) split over four workgroups per value head, 32
 * state columns each (bitwise the same results).  The output norm's partial sums cross the head's workgroups through
 * xch: a caller-owned device buffer of rmi_gdn_exchange_bytes(h_v) bytes, zeroed once before its first use and used
 * by one stream at a time (launches that overlap on one buffer race).  No reference counterpart. */
size_t rmi_gdn_exchange_bytes(int h_v);
int rmi_gdn_layer_tokens_x(float* state_a, float* state_b, float* hist_a, float* hist_b, const int* sel, float* qkvz,
                           int qkvz_stride, const float* ab, int ab_stride, const float* conv_w, const float* dt,
                           const float* ssm_a, const float* gamma, float eps, float* y, int y_stride, uint8_t* q8,
                           int q8_stride, int h_k, int h_v, int ntok, void* xch, void* stream);
/* Waits of the split kernel for the other workgroups of a value head that ran out of their bound, since the library
 * was loaded (0 in every correct run; a nonzero count means a launch's outputs are not to be trusted). */
unsigned int rmi_gdn_exchange_timeouts(void);
/* Test hook (no reference counterpart): set the wait's bound to spin_limit polls (0 = the default, 2^20) and, with
 * force_miss, make every wait run to that bound and count as timed out, so the error path of the engine calls can be
 * exercised with every kernel ending normally.  Outputs of launches made meanwhile are not valid.  Synchronous. */
int rmi_gdn_exchange_test(unsigned int spin_limit, int force_miss);

/* ---------------------------------------------------------------------------------------------------------------
 * GQA attention over an fp16 KV cache [pos][n_kv][head_dim]
 * ------------------------------------------------------------------------------------------------------------- */

/* per token t (position pos[0] + t): split q|gate, per-head RMSNorm (qn, kn), NEOX RoPE on n_rot dims, fp32 q to
 * qout[t][head][d], fp16 K/V into the caches.  Replaces split_qg_kernel (qw:320-327), rms_norm_weighted,
 * native_rope_apply and store_kv2_kernel (qw:340-345) as launched at qw:1532-1548. */
int rmi_attn_prep(const float* q3, int q3_stride, const float* qn, const float* kn, uint16_t* kcache, uint16_t* vcache,
                  const int* pos, float* qout, int n_head, int n_kv, int head_dim, int n_rot, float theta, float eps,
                  int ntok, int max_ctx, void* stream);
/* RoPE parameters as the reference sets them for qwen35 (qw:1991-1999): YaRN with freq_base, factor (the GGUF's
 * rope.scaling.factor; <= 1 is plain NEOX RoPE) and orig_ctx (rope.scaling.original_context_length), ext_factor 1,
 * attn_factor 1, beta_fast 32, beta_slow 1. */
typedef struct rmi_rope_params {
    float freq_base, factor, orig_ctx, ext_factor, attn_factor, beta_fast, beta_slow;
} rmi_rope_params;
/* rmi_attn_prep with YaRN scaling (native_rope_apply with RopeScalingType::YaRN, qw:1991-1999, 1540-1546) */
int rmi_attn_prep_rope(const float* q3, int q3_stride, const float* qn, const float* kn, uint16_t* kcache,
                       uint16_t* vcache, const int* pos, float* qout, int n_head, int n_kv, int head_dim, int n_rot,
                       const rmi_rope_params* rope, float eps, int ntok, int max_ctx, void* stream);
/* Per-row RMSNorm in place: x[r][c] = x[r][c] * rsqrt(mean_c(x[r][:]^2) + eps) * w[c], rows x cols, cols <= 8192.
 * Replaces strata::kernels::rms_norm_weighted (qw:971-975; the q / k per-head norms, rows = heads, cols = 256).  At
 * cols = 256 the bits equal rmi_attn_prep's fused norm. */
int rmi_rms_norm_weighted(float* x, const float* w, int rows, int cols, float eps, void* stream);
/* NEOX RoPE (YaRN ramp when rope->factor > 1) on the first n_rot dims of each of `heads` rows of head_dim floats,
 * head h at position pos[h] (device), dims >= n_rot copied; x may equal y.  Replaces strata::kernels::native_rope_apply
 * (qw:1165-1166, 1357-1358, 1542-1544, 2380-2407; parameters qw:1991-1999).  Norm + rope equals rmi_attn_prep's q. */
int rmi_native_rope_apply(const float* x, float* y, int heads, int head_dim, int n_rot, const rmi_rope_params* rope,
                          const int* pos, void* stream);
/* x += y; x *= s; x = silu(x) over n floats.  Replace strata::kernels::add_inplace / scale_inplace / silu_inplace
 * (qw:1002, 1053, 1059, 1068, 1178: the reference's --split and old-GDN paths). */
int rmi_add_inplace(float* x, const float* y, int n, void* stream);
int rmi_scale_inplace(float* x, int n, float s, void* stream);
int rmi_silu_inplace(float* x, int n, void* stream);
/* split-K flash decode for ntok query tokens at positions pos[0] + t, sigmoid gate from gate_src (the wq output,
 * gate of head h at + h * 2 * head_dim + head_dim), fp32 y (nullable) and Q8_1 (nullable).  workspace holds
 * rmi_gqa_workspace_bytes(max_ctx, n_kv, nsub) bytes; chunks are 64 * nsub positions.  ntok * (n_head / n_kv)
 * <= 64 (an ingest chunk of 16 tokens at 4 query heads per KV head); q, kcache, vcache and workspace 16-byte
 * aligned.  Each query's result is bitwise the single-token result at its position.  Replaces gqa_head_kernel
 * (qw:384-442) + sig_mul_quant_kernel (qw:692-704) per column, and the chunk's shared-K score pass
 * (gqa_score_chunk_kernel + gqa_from_scores_kernel, qw:444-559). */
size_t rmi_gqa_workspace_bytes(int max_ctx, int n_kv, int nsub);
int rmi_gqa_flash_decode(const float* q, const uint16_t* kcache, const uint16_t* vcache, const int* pos,
                         const float* gate_src, int gate_stride, float* y, int y_stride, uint8_t* q8, int q8_stride,
                         void* workspace, int n_head, int n_kv, int head_dim, int ntok, int max_ctx, int nsub,
                         float scale, void* stream);
/* attn_prep (the per-head RMSNorm, RoPE and fp16 K / V store of the new rows; split_qg_kernel, rms, native_rope_apply
 * and store_kv2_kernel, qw:320-345, 971-975, 1535-1548) folded into rmi_gqa_flash_decode for decode and verify (ntok x
 * n_head / n_kv <= 8, an even n_head / n_kv, n_rot = 64): q3 is attn_prep's input (per token [n_head x (q | gate) |
 * k | v], stride q3_stride), which also supplies the gate.  Bitwise rmi_attn_prep_rope followed by
 * rmi_gqa_flash_decode, in two launches instead of three. */
int rmi_gqa_flash_decode_prep(const float* q3, int q3_stride, const float* qn, const float* kn, uint16_t* kcache,
                              uint16_t* vcache, const int* pos, float* y, int y_stride, uint8_t* q8, int q8_stride,
                              void* workspace, int n_head, int n_kv, int head_dim, int n_rot,
                              const rmi_rope_params* rope, float eps, int ntok, int max_ctx, int nsub, float scale,
                              void* stream);
/* rmi_gqa_flash_decode_prep with a table of the rotation's (cos, sin), for the attention layers of one forward pass,
 * which all rotate at the same positions.  No counterpart in the reference (the engine's form of the call above).
 * rope_table holds rmi_gqa_rope_table_bytes(n_rot) bytes, 8-byte aligned: [2 tokens][n_rot / 2 pairs] (cos, sin) at
 * positions pos[0] + t.  table_mode 0: the launch computes its rotation (rmi_gqa_flash_decode_prep); 1: it also
 * stores the table; 2: it loads the table instead of computing it (the pass's later layers, with the same pos and
 * ntok as the mode-1 launch before them on the stream).  Every mode gives the bits of rmi_gqa_flash_decode_prep. */
size_t rmi_gqa_rope_table_bytes(int n_rot);
int rmi_gqa_flash_decode_prep_rt(const float* q3, int q3_stride, const float* qn, const float* kn, uint16_t* kcache,
                                 uint16_t* vcache, const int* pos, float* y, int y_stride, uint8_t* q8, int q8_stride,
                                 void* workspace, int n_head, int n_kv, int head_dim, int n_rot,
                                 const rmi_rope_params* rope, float eps, int ntok, int max_ctx, int nsub, float scale,
                                 float* rope_table, int table_mode, void* stream);

/* rmi_gqa_flash_decode without the workspace argument, for callers that cannot allocate (code under HIP graph
 * capture, serving loops that forbid hipMalloc).  No counterpart in the reference.  The split-K records go to the
 * library's own scratch array on the stream's GPU (rmi_gqa_noalloc_scratch_max() = 16 MiB, held until the process
 * ends); the call allocates and frees nothing.  Needs rmi_gqa_noalloc_scratch_bytes(max_ctx, n_kv, nsub,
 * ntok * n_head / n_kv) <= that maximum (decode at ctx 65536 with nsub >= 4 fits), else RMI_ERR_SHAPE.  Every call on
 * one GPU shares the array: calls that overlap on one GPU (two streams) race.  Results equal rmi_gqa_flash_decode's
 * bit for bit. */
size_t rmi_gqa_noalloc_scratch_bytes(int max_ctx, int n_kv, int nsub, int slots);
size_t rmi_gqa_noalloc_scratch_max(void);
int rmi_gqa_flash_decode_noalloc(const float* q, const uint16_t* kcache, const uint16_t* vcache, const int* pos,
                                 const float* gate_src, int gate_stride, float* y, int y_stride, uint8_t* q8,
                                 int q8_stride, int n_head, int n_kv, int head_dim, int ntok, int max_ctx, int nsub,
                                 float scale, void* stream);

/* ---------------------------------------------------------------------------------------------------------------
 * Seeded synthetic tensors in HBM (stand-in for a GGUF file: random-init weights; no reference counterpart)
 * ------------------------------------------------------------------------------------------------------------- */
int rmi_gen_q6_k(void* w, size_t nblocks, uint64_t seed, float d_std, void* stream);
int rmi_gen_q8_0(void* w, size_t nblocks, uint64_t seed, float d_std, void* stream);
int rmi_gen_normal(float* out, size_t n, uint64_t seed, float mean, float std, void* stream);
int rmi_gen_normal_f16(uint16_t* out, size_t n, uint64_t seed, float mean, float std, void* stream);
/* Reads `bytes` (a multiple of 16, 16-byte aligned) with grid x 256 lanes of streaming 16-byte loads and discards
 * them: the single-launch read-bandwidth reference the GEMV legs are set against (no reference counterpart; `out` is
 * one device word, written only in the unlikely case that the data fold to a sentinel). */
int rmi_stream_read(const void* p, size_t bytes, int grid, unsigned* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif
