/*
 * oracle.h - CPU restatement of Rapier's exact-verify MTP hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the HIP path is compared against (and, in bench.py,
 * the timed CPU baseline).  Nothing in the product library (rapier_amd/, include/) links or calls it.
 *
 * Every function names the reference file:line whose behaviour it restates ("mmvq" = src/native_mmvq.cu,
 * "fgdn" = src/fused_gdn.cu, "qw" = src/qwythos.cpp).  Two flavours exist where it matters:
 *   - exact integer arithmetic for the Q6_K / Q8_0 x Q8_1 block dot products (bit-exact by construction);
 *   - fp64 references for every floating-point output (compared under the tolerances the tests state).
 * Parity status per function is listed in the oracle section of DESIGN.md and repeated in oracle.c.
 */
#ifndef RAPIER_ORACLE_H
#define RAPIER_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- block formats (mmvq:98-103 Q8_1, 113-116 Q8_0, 121-140 Q6_K) ---- */
enum { ORC_Q6K_BYTES = 210, ORC_Q6K_ELEMS = 256, ORC_Q8_0_BYTES = 34, ORC_Q8_1_BYTES = 36, ORC_QK8 = 32 };
enum { ORC_Q4K_BYTES = 144, ORC_Q5K_BYTES = 176 };   /* token_embd of Q5_K_M files (qw:109-115) */

/* ---- seeded counter-based generators (same stream on every platform: splitmix64 + Box-Muller in fp64) ---- */
uint64_t orc_rand_u64(uint64_t seed, uint64_t index);
double orc_rand_unit(uint64_t seed, uint64_t index);                      /* [0,1) with 53 bits */
double orc_rand_normal(uint64_t seed, uint64_t index);                    /* N(0,1) */
void orc_fill_normal(float* out, size_t n, uint64_t seed, double mean, double std);
void orc_gen_q6k(uint8_t* w, size_t nblocks, uint64_t seed, double d_std);  /* codes U{0..63}, sc U[-32,31], d=|N(0,d_std)| */
void orc_gen_q8_0(uint8_t* w, size_t nblocks, uint64_t seed, double d_std);

/* ---- fp16 ---- */
uint16_t orc_f32_to_f16(float x);   /* IEEE round-to-nearest-even, overflow -> inf */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f16_sat(float x);      /* the Q8_1 finite policy: RNE, saturated to +-65504 */

/* ---- Q8_1 quantizer (mmvq:158-173) ---- */
void orc_quantize_q8_1(const float* x, uint8_t* y, int n_in, int ncols);
void orc_dequantize_q8_1(const uint8_t* y, float* x, int n);

/* ---- Q6_K helpers ---- */
int orc_q6k_code(const uint8_t* block, int e);                       /* 6-bit code of element e, 0..63 */
void orc_q6k_dequant_row(const uint8_t* w, float* y, int n);          /* ggml dequantize_row_q6_K order */
void orc_q4k_dequant_row(const uint8_t* w, float* y, int n);          /* ggml dequantize_row_q4_K */
void orc_q5k_dequant_row(const uint8_t* w, float* y, int n);          /* ggml dequantize_row_q5_K */

/* ---- integer block dots (mmvq:642-655, 733-748 restated in closed form) ---- */
/* out[r * (n_in/32) + j] = sum over the 32 elements of Q8_1 block j of sc(e) * (q6(e) - 32) * q8(e), exact int32 */
void orc_q6k_block_dots(const uint8_t* w, const uint8_t* xq, int32_t* out, int n_in, int n_out);
/* lane-mapped form of the reference (per lane iqs, two dp4a, mmvq:733-748) for the brute-force cross-check */
void orc_q6k_block_dots_lanes(const uint8_t* w, const uint8_t* xq, int32_t* out, int n_in, int n_out);
void orc_q8_0_block_dots(const uint8_t* w, const uint8_t* xq, int32_t* out, int n_in, int n_out);

/* ---- fp64 GEMVs (mmvq:753-789, 1261-1356, 3096-3140, 835-847) ---- */
/* y[j*n_out + r] = sum_b d_b * sum_j8 d8 * I  (+ res[j*n_out + r]); partials[j*ceil(n_out/4) + g] = sum y^2 */
void orc_q6k_gemv(const uint8_t* w, const uint8_t* xq, const float* res, double* y, double* partials, int n_in,
                  int n_out, int ncols);
void orc_q8_0_gemv(const uint8_t* w, const uint8_t* xq, const float* res, double* y, double* partials, int n_in,
                   int n_out, int ncols);
/* Q4_K / Q5_K x Q8_1 GEMV (mmvq:185-300, 562-640, residual 3202-3294): exact integer sub-block dots and code sums,
 * d*sc*d8*dot - dmin*m*d8*sum(u) in fp64 */
void orc_q4k_gemv(const uint8_t* w, const uint8_t* xq, const float* res, double* y, double* partials, int n_in,
                  int n_out, int ncols);
void orc_q5k_gemv(const uint8_t* w, const uint8_t* xq, const float* res, double* y, double* partials, int n_in,
                  int n_out, int ncols);
/* same math in fp32, threaded (OpenMP), for the CPU timing baseline */
void orc_q6k_gemv_f32_omp(const uint8_t* w, const uint8_t* xq, const float* res, float* y, float* partials,
                          int n_in, int n_out, int ncols, int threads);

/* ---- norm / activation epilogues (qw:602-715) ---- */
void orc_row_sum_partials(const float* x, double* partials, int n);
double orc_rms_inv(const double* partials, int nparts, int cols, double eps);
void orc_rms_norm_out(const float* x, const float* w, double inv, double* out, int n);
void orc_swiglu(const float* up, const float* gate, double* out, int n);
void orc_sig_mul(const float* o, const float* g, double* out, int n);
void orc_beta_gate(const float* beta_in, const float* alpha, const float* dt, const float* ssm_a, double* beta_out,
                   double* gate_out, int n);

/* ---- Gated DeltaNet (fgdn:40-133) ---- */
void orc_gdn_conv_l2(float* hist, const float* x, const float* w, double* h, int channels, int qk_heads, double eps);
void orc_gdn_step_norm(double* state, const double* q, const double* k, const double* v, const double* gate,
                       const double* beta, const float* z, const float* gamma, double eps, double* y, int h_k,
                       int h_v);

/* ---- attention (qw:384-442), fp64 over fp16 K/V ---- */
void orc_gqa_decode(const float* q, const uint16_t* kc, const uint16_t* vc, double* o, int n_head, int n_kv, int hd,
                    int n_tok, double scale);
void orc_rms_norm_heads(const float* x, const float* w, double* out, int rows, int cols, double eps);
void orc_rope_neox(const double* x, double* out, int heads, int hd, int n_rot, int pos, double theta);
/* YaRN (qw:1991-1999 parameters; ggml's rope_yarn restated) */
void orc_rope_yarn(const double* x, double* out, int heads, int hd, int n_rot, int pos, double base, double factor,
                   double orig_ctx, double ext_factor, double attn_factor, double beta_fast, double beta_slow);

/* ---- argmax, lowest index wins ties (qw:70-94) ---- */
int orc_argmax(const float* l, int n);

/* ---- top-k list of the serve protocol (topk_out, qw:2513-2531): returns the entries written (min(n, k)) ---- */
int orc_topk(const float* l, int n, int k, int* ids, float* vals);

#ifdef __cplusplus
}
#endif
#endif
