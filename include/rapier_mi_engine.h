/*
 * rapier_mi_engine.h - the decode engine around the kernels of rapier_mi.h: a qwen35 hybrid (Gated-DeltaNet layers,
 * GQA every 4th layer, one nextn draft block) held in HBM, the single-token greedy forward and the exact-verify MTP
 * round, each captured as one hipGraph.
 *
 * Reference: src/qwythos.cpp - Engine / alloc_primary / load_model (152-281, 1838-2134), forward_token (1773-1824),
 * draft_predict (1316-1406), launch_token_verify (1412-1618), the MTP accept / rollback loop (3182-3241, serve
 * 2761-2808) and capture_graph (1757-1771).  Weights are either seeded random-init Q6_K of the qwen35 shapes
 * (rmi_engine_create, the benchmark configs) or a qwen35 GGUF file (rmi_engine_create_gguf, load_model's tensor names
 * and metadata keys); everything else follows the reference's engine.
 *
 * Unlike the kernel entry points, the engine owns its memory: rmi_engine_create allocates the model, the caches and
 * the round buffers once; generation allocates nothing on the device.
 */
#ifndef RAPIER_MI_ENGINE_H
#define RAPIER_MI_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#include "rapier_mi.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct rmi_model_config {
    int n_embd;        /* 4096 (kEmb, qw:34) */
    int n_ff;          /* 12288 (kFF) */
    int n_vocab;       /* 248320 (kVocab) */
    int n_layer;       /* 32 trunk layers; layer il is attention when (il + 1) % 4 == 0 (qw:2016) */
    int ssm_h_k;       /* 16 GDN key heads (kHk) */
    int ssm_h_v;       /* 32 GDN value heads (kHv); state size 128 (kS) */
    int n_head;        /* 16 attention heads (kHeads) */
    int n_kv;          /* 4 KV heads (kKv) */
    int head_dim;      /* 256 (kHd) */
    int n_rot;         /* 64 rotary dims (kRot) */
    float rope_theta;  /* 1e7 */
    float eps;         /* 1e-6 */
    float rope_factor; /* qwen35.rope.scaling.factor: YaRN when > 1, plain RoPE otherwise (qw:1991-1999) */
    float rope_orig_ctx; /* qwen35.rope.scaling.original_context_length (262144) */
} rmi_model_config;

typedef struct rmi_engine rmi_engine;

typedef struct rmi_engine_info_t {
    size_t trunk_weight_bytes;   /* all trunk matrices */
    size_t lm_head_bytes;
    size_t draft_block_bytes;    /* eh_proj + the draft attention / FFN block */
    size_t round_weight_bytes;   /* one verify round: trunk + lm_head + draft block + lm_head */
    size_t token_weight_bytes;   /* one greedy token: trunk + lm_head */
    size_t kv_bytes_per_pos;     /* fp16 K+V of the trunk attention layers per position */
    int gdn_layers, attn_layers, max_ctx, attn_chunk;
} rmi_engine_info_t;

enum { RMI_GEN_GREEDY = 0, RMI_GEN_MTP = 1, RMI_GEN_MTP_FORCED = 2 };

typedef struct rmi_gen_request {
    int mode;                 /* RMI_GEN_* */
    int n_gen;                /* tokens to generate after the current token */
    int use_graph;            /* 1: one hipGraph launch per token / round */
    const int* ref_tokens;    /* forced mode: the reference stream, ref_tokens[i] at position ref_base + i */
    int ref_base, ref_len;
    const uint8_t* pattern;   /* forced mode: round r accepts iff pattern[r % pattern_len] */
    int pattern_len;
} rmi_gen_request;

typedef struct rmi_gen_stats {
    int tokens, emitted, rounds, accepted;
    float gpu_ms;             /* device time of the whole generation (events on the engine stream) */
} rmi_gen_stats;

rmi_model_config rmi_qwen35_9b_config(void);
int rmi_engine_create(const rmi_model_config* cfg, uint64_t seed, int max_ctx, void* stream, rmi_engine** out);
int rmi_engine_destroy(rmi_engine* e);
int rmi_engine_info(const rmi_engine* e, rmi_engine_info_t* info);
/* prompt of n host tokens from position 0; *first_out = the greedy token after it (the current token).  Ingests in
 * chunks of 16 tokens (rmi_engine_prefill_batch with batch 16). */
int rmi_engine_prefill(rmi_engine* e, const int* tokens, int n, int* first_out);
/* batch 1: token by token (forward_token per prompt token, qw:1773-1824, plus the draft KV row); batch 2..16: chunks
 * of `batch` tokens, one weight pass per chunk (serve_ingest_kernels, qw:2192-2502, the batch loop qw:2658-2722; the
 * reference takes 2..8 or 16).  Every batch leaves the same state, bit for bit: GDN state and history, trunk and
 * draft KV, hidden, position and first token. */
int rmi_engine_prefill_batch(rmi_engine* e, const int* tokens, int n, int batch, int* first_out);
/* seeded synthetic state for positions [0, n_ctx - 1), then one forward of last_token at n_ctx - 1 */
int rmi_engine_synth_context(rmi_engine* e, int n_ctx, uint64_t seed, int last_token, int* first_out);
int rmi_engine_save_state(rmi_engine* e);
int rmi_engine_restore_state(rmi_engine* e, int pos, int cur_token);
int rmi_engine_state(rmi_engine* e, int* pos, int* cur_token);
/* rmi_engine_generate, rmi_engine_ingest (and so the prefills) and rmi_engine_gen_step return RMI_ERR_STATE when a
 * bounded wait of the GDN layer kernel ran out during the call (rmi_gdn_exchange_timeouts grew): the tokens and the
 * state it produced are not valid. */
int rmi_engine_generate(rmi_engine* e, const rmi_gen_request* req, int* out_tokens, rmi_gen_stats* stats);

/* ---- serving: the context continues across calls (serve_loop, qw:2593-2813) ---- */
/* empty context at position 0 (the serve reset, qw:2533-2549) */
int rmi_engine_reset(rmi_engine* e);
/* feed n tokens at the current position (batch as in rmi_engine_prefill_batch; the same state bit for bit);
 * *first_out = the greedy token after them (the current token).  rmi_engine_prefill_batch = reset + ingest. */
int rmi_engine_ingest(rmi_engine* e, const int* tokens, int n, int batch, int* first_out);
/* token-at-a-time generation from the current token: gen_begin(RMI_GEN_GREEDY or RMI_GEN_MTP), then each gen_step
 * runs one greedy forward (out[0] = the next token; the current one is fed) or one verify round (out[0] = c0, and
 * out[1] = c1 when the draft was accepted; *n_out = 1 or 2).  Any call that replaces the context ends the stream. */
int rmi_engine_gen_begin(rmi_engine* e, int mode);
int rmi_engine_gen_step(rmi_engine* e, int* out_tokens, int* n_out);
/* the k (1..64) largest logits of column col (0 or 1) of the last head pass, with their ids (rmi_topk order).  Column 0
 * after an ingest or a greedy step: the logits that chose the current token (topk_out, qw:2513-2531). */
int rmi_engine_topk(rmi_engine* e, int col, int k, int* ids, float* logits);

/* The --serve JSON-lines protocol (qw:2139-2148, serve_loop qw:2593-2813): reads requests from in_fd until end of input,
 * writes one response line each to out_fd.  Requests: {"op":"reset"}, {"op":"run","tokens":[..],"gen":N,"mtp":B}
 * (optional "topk":K, 0..64).  Responses: {"ok":true,"op":"reset"}; per generated token {"id":I,"top":[[id,logit],..]}
 * (%.5f logits; with mtp only the first token carries its list); {"done":true,"pos":P}; {"error":"..."}.
 * Returns RMI_OK at end of input, or the code of a device failure after its error line. */
typedef struct rmi_serve_options {
    int eos;     /* generation stops after this id: 248046, the qwen35 end-of-turn id the reference compares */
    int batch;   /* ingest chunk, 1..16 (16) */
    int topk;    /* list length when a request names none (40) */
} rmi_serve_options;
/* the engine behind the protocol, as function pointers (a test can drive the loop with its own backend) */
typedef struct rmi_serve_backend {
    void* user;
    int max_ctx;
    int (*reset)(void* user);
    int (*ingest)(void* user, const int* tokens, int n, int batch, int* first);
    int (*topk)(void* user, int k, int* ids, float* logits);
    int (*gen_begin)(void* user, int mode);
    int (*gen_step)(void* user, int* out_tokens, int* n_out);
    int (*position)(void* user, int* pos);
    const char* (*error)(void* user);   /* message of the last failure (may be NULL) */
} rmi_serve_backend;
rmi_serve_options rmi_serve_default_options(void);
int rmi_serve_fd(const rmi_serve_backend* b, const rmi_serve_options* o, int in_fd, int out_fd);
int rmi_serve_engine(rmi_engine* e, const rmi_serve_options* o, int in_fd, int out_fd);

/* ---- GGUF (v2 / v3) files: the reader the engine loads through (the role of strata::GgufFile, qw:945-957,
 * 1978-2134).  Tensors are memory-mapped; dims[0] is the innermost dimension (n_in of a matrix). ---- */
typedef struct rmi_gguf rmi_gguf;
int rmi_gguf_open(const char* path, rmi_gguf** out);
void rmi_gguf_close(rmi_gguf* g);
int64_t rmi_gguf_tensor_count(const rmi_gguf* g);
int64_t rmi_gguf_find(const rmi_gguf* g, const char* name);      /* tensor index or -1 */
/* GGML type, rank, dims[4] (unused dims 1), data bytes (0 for a type the reader does not size) and data pointer */
int rmi_gguf_tensor_info(const rmi_gguf* g, int64_t i, const char** name, int* type, int* n_dims, int64_t* dims,
                         size_t* bytes, const void** data);
int rmi_gguf_get_num(const rmi_gguf* g, const char* key, double* out);       /* any numeric scalar */
int rmi_gguf_get_str(const rmi_gguf* g, const char* key, const char** out);
int64_t rmi_gguf_array_len(const rmi_gguf* g, const char* key);             /* -1 if not an array */
int rmi_gguf_array_str(const rmi_gguf* g, const char* key, int64_t i, const char** out);
int rmi_gguf_array_num(const rmi_gguf* g, const char* key, int64_t i, double* out);

/* Create the engine from a qwen35 GGUF (load_model, qw:1978-2134): general.architecture "qwen35", trunk layers =
 * block_count - nextn_predict_layers, layer il attention when blk.il.attn_q.weight exists, the draft block at
 * blk.<n_layer> with its nextn tensors; shapes from the tensors, eps / RoPE / YaRN from the metadata.  Matrices are
 * Q6_K (concatenated as the reference's try_cat groups: attn_qkv | attn_gate | ssm_beta | ssm_alpha, attn_q | attn_k |
 * attn_v, ffn_up | ffn_gate), token_embd Q6_K / Q5_K / Q4_K, norms and GDN vectors F32.  Other matrix types are
 * RMI_ERR_UNSUPPORTED. */
int rmi_engine_create_gguf(const char* path, int max_ctx, void* stream, rmi_engine** out);
/* the model configuration the engine runs (from the file for a GGUF engine) */
int rmi_engine_config(const rmi_engine* e, rmi_model_config* out);

/* engine buffers readable with rmi_engine_read (the reference's QWYTHOS_IDUMP probes read the same state) */
enum {
    RMI_BUF_GDN_STATE = 0,   /* live GDN state of a GDN layer, fp32 [128][h_v][128] */
    RMI_BUF_GDN_HIST = 1,    /* live conv history of a GDN layer, fp32 [h_v][3 * 128][3] */
    RMI_BUF_K_CACHE = 2,     /* K cache of an attention layer (layer n_layer: the draft block), fp16 [pos][n_kv][256] */
    RMI_BUF_V_CACHE = 3,
    RMI_BUF_HIDDEN = 4,      /* final-normed hidden of the last forward, fp32 [n_embd] (the first draft's input) */
    RMI_BUF_LOGITS = 5,      /* logits of the last head pass, fp32 [2][n_vocab] (column 0: the last forward) */
    RMI_BUF_ROUND = 6        /* the round's token slots, int32 [8] (layer ignored): position of the current token,
                                current token, draft candidate for the next verify, verify argmax of columns 0 / 1,
                                draft argmax of columns 0 / 1, accept flag of the last verify */
};
/* copy bytes [offset, offset + bytes) of an engine buffer to host memory; synchronizes the engine stream */
int rmi_engine_read(rmi_engine* e, int which, int layer, size_t offset, void* dst, size_t bytes);

#ifdef __cplusplus
}
#endif
#endif
