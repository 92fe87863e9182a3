// engine.hip - the qwen35 hybrid decode engine around the kernels: a seeded random-init model in HBM, the
// single-token forward (non-MTP greedy) and the exact-verify MTP round, each captured as one hipGraph.
//
// Reference: src/qwythos.cpp - Engine (152-281), load_model's concatenations (2082-2087, 2125-2128), forward_gdn /
// forward_attn / ffn (1011-1226), launch_token_gpu (1228-1238), draft_predict (1316-1406), launch_token_verify
// (1412-1618), the accept / rollback loop (3182-3241) and capture_graph (1757-1771).
//
// What differs from the reference, by design:
//   * every per-round decision lives on the device: token ids, positions, the accept flag, the GDN rollback
//     selector, the emitted-token ring.  One verify round is one hipGraph launch with no host round trip.
//   * the verify pass uses the fused residual epilogue at ncols = 2 (the reference runs mm_q2 then add_partials);
//     each column of every kernel is bitwise the single-column result, so the MTP stream equals the greedy stream.
//   * GDN rollback flips a selector instead of copying 24 x (2 MiB + 96 KiB) snapshots.
//   * the draft always runs two columns after a verify: column 0 = (c0, hidden of verify column 0) at pos + 1 and
//     column 1 = (c1, hidden of column 1) at pos + 2.  On reject column 0 is the reference's corrected draft step; on
//     accept column 0 is its KV-fill step and column 1 its next-candidate step.  Both weight passes become one.
//   * the KV cache is fp16; the token embedding is dequantized on the device.
#include "epilogue_dev.h"
#include "rmi_common.h"

#include <cstdlib>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "../../include/rapier_mi_engine.h"

namespace rmi {
namespace {

constexpr int kS = 128;          // GDN state size
constexpr int kRingCap = 1 << 16;
constexpr int kChunk = kMaxCols;  // ingest chunk: prompt tokens per weight pass
constexpr int kAttnSlots = 64;    // query vectors per KV head one rmi_gqa_flash_decode launch takes

int hip_check(hipError_t e, const char* what) {
    if (e == hipSuccess) return RMI_OK;
    char buf[512];
    std::snprintf(buf, sizeof buf, "%s: %s", what, hipGetErrorString(e));
    return fail(RMI_ERR_LAUNCH, buf);
}
#define HIP_TRY(expr) RMI_TRY(hip_check((expr), #expr))

size_t q6_bytes(int n_out, int n_in) { return static_cast<size_t>(n_out) * (n_in / 256) * kQ6KBytes; }
size_t q81_bytes(int n) { return static_cast<size_t>(n / 32) * kQ8_1Bytes; }
// conv history of one GDN layer, per value head: [h_v][q 128 | k 128 | v 128][3]
size_t hist_floats(const rmi_model_config& c) { return static_cast<size_t>(c.ssm_h_v) * 3 * kS * 3; }

// A matrix of GGML type 14 (Q6_K: the packed wave-tiled copy when n_in is a multiple of 2048, every 9B matrix, else
// GGUF blocks), 13 (Q5_K), 12 (Q4_K) or 8 (Q8_0), in GGUF blocks.  A group whose parts differ in type (a Q5_K_M file's
// qkv | z | beta | alpha, say) keeps its parts: the GEMV then runs per part and per column into the group's rows, the
// reference's mm_q2_group fallback (qw:1284-1309).
struct Mat {
    uint8_t* w = nullptr;
    int n_in = 0, n_out = 0;
    int type = 14;
    bool packed = false;
    int swiglu_ff = 0;           // > 0: an up||gate matrix packed in the SwiGLU row order (ff rows each)
    size_t bytes = 0;            // GGUF bytes of the matrix (the weight pass it costs)
    std::vector<Mat> parts;      // non-empty: a mixed-type group
};

struct Layer {
    bool gdn = true;
    float* attn_norm = nullptr;
    float* post_norm = nullptr;
    Mat in_proj;     // GDN: qkv|z|beta|alpha ; attention: wq|wk|wv
    Mat out_proj;    // GDN: ssm_out ; attention: wo
    Mat upgate, down;
    // GDN
    float *conv_w = nullptr, *dt = nullptr, *ssm_a = nullptr, *ssm_norm = nullptr;
    float* state[2] = {nullptr, nullptr};
    float* hist[2] = {nullptr, nullptr};
    // attention
    float *qn = nullptr, *kn = nullptr;
    uint16_t *kc = nullptr, *vc = nullptr;
};

// device-side round state: one int block
enum Slot {
    kPos = 0,      // position of column 0 (the current token)
    kTok0, kTok1,  // verify / forward tokens: current token, draft candidate
    kV0, kV1,      // argmax of the verify (or forward) columns
    kD0, kD1,      // draft input tokens
    kDPos,         // draft position of column 0
    kC0, kC1,      // argmax of the draft columns
    kSel,          // GDN rollback selector
    kAccept,       // accept flag of the last verify
    kNOut,         // tokens emitted into the ring
    kRound,        // rounds run
    kNAcc,         // accepted drafts
    kMode,         // 0 natural draft, 1 forced by pattern
    kPatLen,
    kVocab,
    kMaxPos,       // last usable position
    kNumSlots
};

struct Engine {
    rmi_model_config cfg{};
    int max_ctx = 0, nsub = 1;
    // the next norm forms its vector's partials itself (rmi_rms_quant_apply_self): the draft's eh_proj output, whose
    // partials no GEMV epilogue writes
    bool norm_self = false;
    // a norm and the packed GEMV that reads it run as one launch where the GEMV takes the norm in its stage
    // (RMI_FUSE_NORM=0: two launches, for measurement; the same bits either way)
    bool fuse_norm = true;
    hipStream_t s = nullptr;
    bool own_stream = false;
    std::vector<void*> allocs;
    uint8_t* gen_tmp = nullptr;   // GGUF staging for the packed matrices, only while the model is created
    size_t gen_tmp_bytes = 0;

    Mat lm_head;
    uint8_t* tok_embd = nullptr;
    int emb_type = 14;              // GGML type of the token embedding table (Q6_K, Q5_K or Q4_K)
    rmi_rope_params rope{};
    float* out_norm = nullptr;
    std::vector<Layer> layers;
    Layer draft;
    Mat eh_proj;
    float *enorm = nullptr, *hnorm = nullptr, *shnorm = nullptr;

    // sizes
    int qkvz_rows = 0, q3_rows = 0, gdn_v = 0, attn_q = 0, max_in = 0;

    int* ints = nullptr;            // kNumSlots
    int* cints = nullptr;           // ingest chunk: trunk tokens [0, 16), positions [16, 32)
    int* prompt = nullptr;          // ingest: the prompt's token ids, indexed by position
    int* ring = nullptr;            // emitted tokens
    int* ref_tok = nullptr;         // forced-acceptance reference stream, indexed by position
    uint8_t* pattern = nullptr;     // forced-acceptance pattern, indexed by round

    // activations (kChunk columns; decode uses the first two).  hsave / hpart hold kChunk + 1 columns: an ingest chunk
    // writes its hidden to columns 1..nc, so that column c - 1 is the draft input of column c
    float *x = nullptr, *part = nullptr, *proj = nullptr, *ug = nullptr, *y = nullptr, *logits = nullptr;
    float *hsave = nullptr, *hpart = nullptr, *hzero = nullptr, *pzero = nullptr, *qbuf = nullptr;
    float *dx = nullptr, *dpart = nullptr;
    uint8_t *q8a = nullptr, *q8f = nullptr, *q8y = nullptr;
    void *attn_ws = nullptr, *argmax_ws = nullptr, *topk_ws = nullptr;
    float* rope_cs = nullptr;   // the trunk pass's RoPE (cos, sin) table: written by its first attention layer
    unsigned long long* gdn_xch = nullptr;   // the split GDN step's exchange words (rmi_gdn_exchange_bytes), zeroed once
    int* topk_out = nullptr;        // top-k ids [0, 64) and logits (as float) [64, 128)
    int stream_mode = -1;           // rmi_engine_gen_begin's mode, -1 before it
    // saved GDN state and draft hidden for restore
    std::vector<float*> saved_state, saved_hist;
    float *saved_h = nullptr, *saved_hp = nullptr;

    hipGraphExec_t g_single = nullptr, g_round = nullptr, g_draft1 = nullptr, g_chunk = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;

    ~Engine() {
        if (g_single) (void) hipGraphExecDestroy(g_single);
        if (g_round) (void) hipGraphExecDestroy(g_round);
        if (g_draft1) (void) hipGraphExecDestroy(g_draft1);
        if (g_chunk) (void) hipGraphExecDestroy(g_chunk);
        if (ev0) (void) hipEventDestroy(ev0);
        if (ev1) (void) hipEventDestroy(ev1);
        for (void* p : allocs) (void) hipFree(p);
        if (gen_tmp) (void) hipFree(gen_tmp);
        if (own_stream && s) (void) hipStreamDestroy(s);
    }

    template <typename T>
    int alloc(T** p, size_t count) {
        void* v = nullptr;
        const size_t bytes = std::max<size_t>(count * sizeof(T), 256);
        HIP_TRY(hipMalloc(&v, bytes));
        allocs.push_back(v);
        *p = static_cast<T*>(v);
        return RMI_OK;
    }
};

// ---- small device kernels of the round ----------------------------------------------------------------------------
__global__ void fill_f32_kernel(float* p, size_t n, float v) {
    const size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) p[i] = v;
}
__global__ void fill_i32_kernel(int* p, size_t n, int v) {
    const size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) p[i] = v;
}

// after a single-token forward: emit the argmax, feed it back, advance one position (one thread)
__device__ void advance_single(int* st, int* ring) {
    const int id = st[kV0];
    const int n = st[kNOut];
    if (n < kRingCap) ring[n] = id;
    st[kNOut] = n + 1;
    st[kTok0] = id;
    st[kPos] = min(st[kPos] + 1, st[kMaxPos]);
}

// after the verify: accept c0 == candidate, roll back the GDN state on reject, emit, set up the draft columns (one
// thread)
__device__ void accept_tokens(int* st, int* ring) {
    const int c0 = st[kV0], c1 = st[kV1];
    const int accept = c0 == st[kTok1];
    int n = st[kNOut];
    if (n < kRingCap) ring[n] = c0;
    ++n;
    if (accept) {
        if (n < kRingCap) ring[n] = c1;
        ++n;
        st[kNAcc] += 1;
    } else {
        st[kSel] ^= 1;   // the state after column 0 becomes the live one
    }
    st[kNOut] = n;
    st[kAccept] = accept;
    st[kD0] = c0;
    st[kD1] = c1;
    st[kDPos] = st[kPos] + 1;
}

// dst[i] = src[i], i < n, by one workgroup (dst and src do not overlap): every load of a lane's pass is issued before
// its first store, where a strided loop would wait on each load in turn
__device__ void wg_copy(float* __restrict__ dst, const float* __restrict__ src, int n) {
    constexpr int kPer = 16;
    const int nt = static_cast<int>(blockDim.x);
    for (int b = static_cast<int>(threadIdx.x); b < n; b += kPer * nt) {
        float v[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) v[k] = b + k * nt < n ? src[b + k * nt] : 0.0f;
#pragma unroll
        for (int k = 0; k < kPer; ++k)
            if (b + k * nt < n) dst[b + k * nt] = v[k];
    }
}

// after the draft: pick the candidate, advance (1 or 2 positions), apply the forced-acceptance override.  On accept the
// last fed token is column 1, whose hidden moves to column 0, so that column 0 always holds the hidden of the token
// before the current one (the input of a later first draft or ingest chunk).  One workgroup.
__device__ void finalize_round(int* st, const int* ref_tok, const uint8_t* pattern, float* hsave, float* hpart, int n,
                               int np) {
    const int accept = st[kAccept];
    if (accept) {
        wg_copy(hsave, hsave + n, n);
        wg_copy(hpart, hpart + np, np);
    }
    if (threadIdx.x != 0) return;
    const int pos = min(st[kPos] + (accept ? 2 : 1), st[kMaxPos]);
    const int cur = accept ? st[kV1] : st[kV0];
    int cand = accept ? st[kC1] : st[kC0];
    const int round = st[kRound];
    if (st[kMode] == 1 && st[kPatLen] > 0) {
        // the candidate for position pos + 1: the reference stream's token (accepted) or another one (rejected)
        const int truth = ref_tok[min(pos + 1, st[kMaxPos])];
        cand = pattern[(round + 1) % st[kPatLen]] ? truth : (truth + 1) % st[kVocab];   // for the next round
    }
    st[kPos] = pos;
    st[kTok0] = cur;
    st[kTok1] = cand;
    st[kRound] = round + 1;
}

// initial draft candidate (1-column draft with head): cand = draft argmax, or the forced one (one thread)
__device__ void first_candidate(int* st, const int* ref_tok, const uint8_t* pattern) {
    int cand = st[kC0];
    if (st[kMode] == 1 && st[kPatLen] > 0) {
        const int truth = ref_tok[min(st[kPos] + 1, st[kMaxPos])];
        cand = pattern[0] ? truth : (truth + 1) % st[kVocab];
    }
    st[kTok1] = cand;
}

// The decode tails: the greedy tokens of the lm_head columns (argmax_final_block over argmax_partial_launch's keys)
// and the integer bookkeeping that reads them run in one launch; after the trunk's lm_head the same launch also takes
// the final norm of the hidden (rms_norm_out_block) on workgroups 1.., which neither reads nor writes what workgroup 0
// does.  Same bits as the separate launches (argmax, rms_norm_out, accept / advance / finalize / first candidate).
struct NormOut {
    const float* x;
    const float* w;
    const float* part;
    float* out;
    float* out_part;
    int cols;
    float eps;
};

__device__ void norm_out_workgroup(const NormOut& no, int b) {
    const int nb = (no.cols + 255) / 256;
    rms_norm_out_block(no.x, no.w, no.part, no.out, no.out_part, no.cols, no.eps, no.cols, b / nb, b % nb);
}

// after the verify's lm_head (2 columns): c0, c1, then the acceptance
__global__ __launch_bounds__(256) void verify_tail_kernel(int* st, int* ring, const uint64_t* keys, NormOut no) {
    if (blockIdx.x == 0) {
        const int c0 = argmax_final_block(keys, 0), c1 = argmax_final_block(keys, 1);
        if (threadIdx.x == 0) {
            st[kV0] = c0;
            st[kV1] = c1;
            accept_tokens(st, ring);
        }
        return;
    }
    norm_out_workgroup(no, static_cast<int>(blockIdx.x) - 1);
}

// after a single-token forward's lm_head: the token, then the advance
__global__ __launch_bounds__(256) void single_tail_kernel(int* st, int* ring, const uint64_t* keys, NormOut no) {
    if (blockIdx.x == 0) {
        const int v0 = argmax_final_block(keys, 0);
        if (threadIdx.x == 0) {
            st[kV0] = v0;
            advance_single(st, ring);
        }
        return;
    }
    norm_out_workgroup(no, static_cast<int>(blockIdx.x) - 1);
}

// after the round's 2-column draft head: both candidates, then finalize_round (one workgroup)
__global__ __launch_bounds__(256) void draft_tail_kernel(int* st, const uint64_t* keys, const int* ref_tok,
                                                         const uint8_t* pattern, float* hsave, float* hpart, int n,
                                                         int np) {
    const int c0 = argmax_final_block(keys, 0), c1 = argmax_final_block(keys, 1);
    if (threadIdx.x == 0) {
        st[kC0] = c0;
        st[kC1] = c1;
    }
    __syncthreads();
    finalize_round(st, ref_tok, pattern, hsave, hpart, n, np);
}

// after the first draft's head (1 column): the candidate
__global__ __launch_bounds__(256) void first_tail_kernel(int* st, const uint64_t* keys, const int* ref_tok,
                                                         const uint8_t* pattern) {
    const int c0 = argmax_final_block(keys, 0);
    if (threadIdx.x == 0) {
        st[kC0] = c0;
        first_candidate(st, ref_tok, pattern);
    }
}

// ingest chunk set-up: nc prompt tokens from position st[kPos]; column c is token prompt[pos + c] at pos + c
__global__ void chunk_setup_kernel(const int* st, const int* prompt, int* cints, int nc) {
    const int c = threadIdx.x;
    const int p = st[kPos] + c;
    if (c < nc) {
        cints[c] = prompt[p];
        cints[kChunk + c] = p;
    }
}

// after an ingest chunk: advance the position; column nc's hidden becomes column 0 (the next chunk's draft input, and
// the hidden of the last token for the first draft of generation); with the head, the greedy token is current
__global__ void chunk_finish_kernel(int* st, float* hsave, float* hpart, int n, int np, int nc, int head) {
    wg_copy(hsave, hsave + static_cast<size_t>(nc) * n, n);
    wg_copy(hpart, hpart + static_cast<size_t>(nc) * np, np);
    if (threadIdx.x == 0) {
        st[kPos] = st[kPos] + nc;
        if (head) st[kTok0] = st[kV0];
    }
}

unsigned grid1(size_t n) { return static_cast<unsigned>((n + 255) / 256); }

// ---- model construction ------------------------------------------------------------------------------------------
uint64_t mix_seed(uint64_t seed, int layer, int what) {
    uint64_t z = seed ^ (0x9E3779B97F4A7C15ULL * static_cast<uint64_t>(layer + 7)) ^
                 (0xC2B2AE3D27D4EB4FULL * static_cast<uint64_t>(what + 1));
    z = (z ^ (z >> 31)) * 0xBF58476D1CE4E5B9ULL;
    return z ^ (z >> 29);
}

// an up||gate matrix ([up | gate], swiglu) of 4096-wide rows is packed in the SwiGLU row order, for the fused
// up||gate + SwiGLU kernel
bool swiglu_packing(const Mat& m, bool swiglu) { return swiglu && m.packed && m.n_in == 4096 && (m.n_out / 2) % 32 == 0; }

int pack_mat(Engine& e, Mat& m, bool swiglu) {
    if (swiglu_packing(m, swiglu)) {
        m.swiglu_ff = m.n_out / 2;
        return rmi_q6_k_pack_swiglu(e.gen_tmp, m.w, m.n_in, m.swiglu_ff, e.s);
    }
    return rmi_q6_k_pack(e.gen_tmp, m.w, m.n_in, m.n_out, e.s);
}

int make_mat(Engine& e, Mat& m, int n_out, int n_in, uint64_t seed, bool swiglu = false) {
    m.n_in = n_in;
    m.n_out = n_out;
    static const bool use_packed = [] {
        const char* v = std::getenv("RMI_ENGINE_PACKED");
        return !(v && v[0] == '0');
    }();
    m.packed = use_packed && n_in % 2048 == 0;
    m.type = 14;
    m.bytes = q6_bytes(n_out, n_in);
    if (!m.packed) {
        RMI_TRY(e.alloc(&m.w, q6_bytes(n_out, n_in)));
        return rmi_gen_q6_k(m.w, static_cast<size_t>(n_out) * (n_in / 256), seed, 1e-3f, e.s);
    }
    // the seeded GGUF blocks go through the engine's staging buffer into the packed copy
    const size_t gguf = q6_bytes(n_out, n_in);
    if (gguf > e.gen_tmp_bytes) return fail(RMI_ERR_STATE, "engine: generation buffer too small");
    RMI_TRY(e.alloc(&m.w, rmi_q6_k_packed_bytes(n_in, n_out)));
    RMI_TRY(rmi_gen_q6_k(e.gen_tmp, static_cast<size_t>(n_out) * (n_in / 256), seed, 1e-3f, e.s));
    return pack_mat(e, m, swiglu);
}

int gemv(Engine& e, const Mat& m, const uint8_t* xq, float* y, int nc) {
    if (!m.parts.empty()) {   // mixed-type group: each part, each column, into its rows (qw:1296-1308)
        const size_t xcol = q81_bytes(m.n_in);
        for (int c = 0; c < nc; ++c) {
            int off = 0;
            for (const Mat& p : m.parts) {
                RMI_TRY(gemv(e, p, xq + c * xcol, y + static_cast<size_t>(c) * m.n_out + off, 1));
                off += p.n_out;
            }
        }
        return RMI_OK;
    }
    if (m.packed) return rmi_native_q6_k_mmvq_packed(m.w, xq, y, m.n_in, m.n_out, nc, e.s);
    return rmi_native_mmvq(m.type, m.w, xq, y, m.n_in, m.n_out, nc, e.s);
}

int gemv_res(Engine& e, const Mat& m, const uint8_t* xq, float* x, float* part, int nc) {
    if (m.packed) return rmi_native_q6_k_mmvq_packed_res_n(m.w, xq, x, x, part, m.n_in, m.n_out, nc, e.s);
    switch (m.type) {
        case 14: return rmi_native_q6_k_mmvq_res_n(m.w, xq, x, x, part, m.n_in, m.n_out, nc, e.s);
        case 13: return rmi_native_q5_k_mmvq_res_n(m.w, xq, x, x, part, m.n_in, m.n_out, nc, e.s);
        case 12: return rmi_native_q4_k_mmvq_res_n(m.w, xq, x, x, part, m.n_in, m.n_out, nc, e.s);
        case 8: return rmi_native_q8_0_mmvq_res_n(m.w, xq, x, x, part, m.n_in, m.n_out, nc, e.s);
        default: return fail(RMI_ERR_UNSUPPORTED, "engine: residual GEMV of an unsupported type");
    }
}

int make_vec(Engine& e, float** p, size_t n, uint64_t seed, float mean, float std) {
    RMI_TRY(e.alloc(p, n));
    if (std == 0.0f) {
        hipLaunchKernelGGL(fill_f32_kernel, dim3(grid1(n)), dim3(256), 0, e.s, *p, n, mean);
        return launch_status("fill");
    }
    return rmi_gen_normal(*p, n, seed, mean, std, e.s);
}

int zero_f32(Engine& e, float* p, size_t n) {
    hipLaunchKernelGGL(fill_f32_kernel, dim3(grid1(n)), dim3(256), 0, e.s, p, n, 0.0f);
    return launch_status("fill");
}

// fp16 K/V caches of an attention layer, zeroed
int alloc_attn_state(Engine& e, Layer& L) {
    const auto& c = e.cfg;
    const size_t kv = static_cast<size_t>(e.max_ctx) * c.n_kv * c.head_dim;
    RMI_TRY(e.alloc(&L.kc, kv));
    RMI_TRY(e.alloc(&L.vc, kv));
    HIP_TRY(hipMemsetAsync(L.kc, 0, kv * 2, e.s));
    HIP_TRY(hipMemsetAsync(L.vc, 0, kv * 2, e.s));
    return RMI_OK;
}

// the two GDN state and history buffers of a layer, zeroed
int alloc_gdn_state(Engine& e, Layer& L) {
    const auto& c = e.cfg;
    const size_t st = static_cast<size_t>(kS) * c.ssm_h_v * kS;
    for (int b = 0; b < 2; ++b) {
        RMI_TRY(e.alloc(&L.state[b], st));
        RMI_TRY(e.alloc(&L.hist[b], hist_floats(c)));
        RMI_TRY(zero_f32(e, L.state[b], st));
        RMI_TRY(zero_f32(e, L.hist[b], hist_floats(c)));
    }
    return RMI_OK;
}

int make_attn(Engine& e, Layer& L, int li, uint64_t seed) {
    const auto& c = e.cfg;
    L.gdn = false;
    RMI_TRY(make_vec(e, &L.attn_norm, c.n_embd, mix_seed(seed, li, 1), 1.0f, 0.1f));
    RMI_TRY(make_vec(e, &L.post_norm, c.n_embd, mix_seed(seed, li, 2), 1.0f, 0.1f));
    RMI_TRY(make_mat(e, L.in_proj, e.q3_rows, c.n_embd, mix_seed(seed, li, 3)));
    RMI_TRY(make_mat(e, L.out_proj, c.n_embd, e.attn_q, mix_seed(seed, li, 4)));
    RMI_TRY(make_mat(e, L.upgate, 2 * c.n_ff, c.n_embd, mix_seed(seed, li, 5), true));
    RMI_TRY(make_mat(e, L.down, c.n_embd, c.n_ff, mix_seed(seed, li, 6)));
    RMI_TRY(make_vec(e, &L.qn, c.head_dim, mix_seed(seed, li, 7), 1.0f, 0.1f));
    RMI_TRY(make_vec(e, &L.kn, c.head_dim, mix_seed(seed, li, 8), 1.0f, 0.1f));
    return alloc_attn_state(e, L);
}

int make_gdn(Engine& e, Layer& L, int li, uint64_t seed) {
    const auto& c = e.cfg;
    L.gdn = true;
    RMI_TRY(make_vec(e, &L.attn_norm, c.n_embd, mix_seed(seed, li, 1), 1.0f, 0.1f));
    RMI_TRY(make_vec(e, &L.post_norm, c.n_embd, mix_seed(seed, li, 2), 1.0f, 0.1f));
    RMI_TRY(make_mat(e, L.in_proj, e.qkvz_rows, c.n_embd, mix_seed(seed, li, 3)));
    RMI_TRY(make_mat(e, L.out_proj, c.n_embd, e.gdn_v, mix_seed(seed, li, 4)));
    RMI_TRY(make_mat(e, L.upgate, 2 * c.n_ff, c.n_embd, mix_seed(seed, li, 5), true));
    RMI_TRY(make_mat(e, L.down, c.n_embd, c.n_ff, mix_seed(seed, li, 6)));
    const int ch = 2 * c.ssm_h_k * kS + c.ssm_h_v * kS;
    RMI_TRY(make_vec(e, &L.conv_w, static_cast<size_t>(4) * ch, mix_seed(seed, li, 7), 0.0f, 0.5f));
    RMI_TRY(make_vec(e, &L.dt, c.ssm_h_v, 0, 0.0f, 0.0f));
    RMI_TRY(make_vec(e, &L.ssm_a, c.ssm_h_v, mix_seed(seed, li, 8), 0.0f, 0.5f));
    RMI_TRY(make_vec(e, &L.ssm_norm, kS, mix_seed(seed, li, 9), 1.0f, 0.1f));
    return alloc_gdn_state(e, L);
}

// per-value-head copy of a [channels][3] conv history: head h takes k-head h % h_k's q and k channels and its v
__global__ void hist_expand_kernel(const float* __restrict__ std_hist, float* __restrict__ per_head, int h_k, int h_v) {
    const int i = blockIdx.x * 256 + threadIdx.x;   // (head, kind, j)
    if (i >= h_v * 3 * kS) return;
    const int head = i / (3 * kS), kind = (i / kS) % 3, j = i % kS;
    const int qh = head % h_k;
    const int c = kind == 0 ? qh * kS + j : kind == 1 ? (h_k + qh) * kS + j : (2 * h_k + head) * kS + j;
    for (int t = 0; t < 3; ++t) per_head[3 * i + t] = std_hist[3 * c + t];
}

__global__ void neg_exp_kernel(float* p, int n) {   // ssm_a = -exp(N(0, 0.5^2))
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = -expf(p[i]);
}

// ---- the forward building blocks (ncols = 1 or 2; every kernel is column-invariant) --------------------------------
// A norm feeds its GEMV through q8a = Q8_1((x * w) * inv) (rms_quant_apply, qw:627-655) of columns
// col0 .. col0 + nc - 1.
int norm_input(Engine& e, const float* x, const float* part, const float* w, int col0, int nc, const uint8_t** xq) {
    const auto& c = e.cfg;
    const size_t xs = static_cast<size_t>(col0) * c.n_embd, ps = static_cast<size_t>(col0) * (c.n_embd / 4);
    *xq = e.q8a;
    if (e.norm_self) {
        e.norm_self = false;
        return rmi_rms_quant_apply_self(x + xs, w, e.q8a, c.n_embd, c.eps, nc, e.s);
    }
    return rmi_rms_quant_apply(x + xs, w, part + ps, e.q8a, c.n_embd, c.eps, nc, e.s);
}

// A norm and the GEMV behind it in one launch (rms_quant_apply quantized into the GEMV's own stage, the same bits):
// a packed single-type matrix of 4096-wide rows at one or two columns, whose norm has its partials at hand
bool norm_fusable(const Engine& e, const Mat& m, int nc) {
    return e.fuse_norm && !e.norm_self && m.packed && m.parts.empty() && m.n_in == 4096 && nc <= 2;
}

// norm(x) -> GEMV into y (columns 0 .. nc - 1); one launch where the shape favours it
int norm_gemv(Engine& e, const Mat& m, const float* x, const float* part, const float* w, float* y, int nc) {
    if (norm_fusable(e, m, nc) && rmi_q6_k_packed_norm_preferred(m.n_in, m.n_out, nc))
        return rmi_native_q6_k_mmvq_packed_norm(m.w, x, w, part, e.cfg.eps, y, m.n_in, m.n_out, nc, e.s);
    const uint8_t* xq = nullptr;
    RMI_TRY(norm_input(e, x, part, w, 0, nc, &xq));
    return gemv(e, m, xq, y, nc);
}

// post-attention norm, up||gate + SwiGLU, down with the residual
int ffn(Engine& e, Layer& L, float* x, float* part, int nc) {
    const auto& c = e.cfg;
    if (L.upgate.swiglu_ff && nc <= 2 && norm_fusable(e, L.upgate, nc)) {   // norm, up||gate, SwiGLU, Q8_1: one launch
        RMI_TRY(rmi_native_q6_k_swiglu_packed_norm(L.upgate.w, x, L.post_norm, part, c.eps, e.q8f, c.n_embd, c.n_ff, nc,
                                                   e.s));
        return gemv_res(e, L.down, e.q8f, x, part, nc);
    }
    const uint8_t* xq = nullptr;
    RMI_TRY(norm_input(e, x, part, L.post_norm, 0, nc, &xq));
    if (L.upgate.swiglu_ff && nc <= 2) {   // up||gate GEMV + SwiGLU + Q8_1 in one launch
        RMI_TRY(rmi_native_q6_k_swiglu_packed(L.upgate.w, xq, e.q8f, c.n_embd, c.n_ff, nc, e.s));
    } else {
        RMI_TRY(gemv(e, L.upgate, xq, e.ug, nc));
        if (L.upgate.swiglu_ff)
            RMI_TRY(rmi_swiglu_quant_interleaved(e.ug, e.q8f, c.n_ff, nc, 2 * c.n_ff, e.s));
        else
            RMI_TRY(rmi_swiglu_quant(e.ug, e.ug + c.n_ff, e.q8f, c.n_ff, nc, 2 * c.n_ff, e.s));
    }
    return gemv_res(e, L.down, e.q8f, x, part, nc);
}

// pos[0] is the position of column 0; with more columns than one attention launch takes (64 query vectors per KV
// head: 16 tokens at 4 query heads per KV head) pos is an array, pos[c] = pos[0] + c, and the launch for columns
// c0.. reads pos + c0.  Every KV row of the nc columns is stored before any of them attends, and query c sees
// positions <= pos[0] + c only, as in the per-token path.  rope_mode (decode / verify): 0 the launch computes its
// rotation, 1 it also writes the trunk pass's table e.rope_cs, 2 it reads the table (the same bits).
int attn_block(Engine& e, Layer& L, float* x, float* part, const int* pos, int nc, int rope_mode = 0) {
    const auto& c = e.cfg;
    RMI_TRY(norm_gemv(e, L.in_proj, x, part, L.attn_norm, e.proj, nc));
    const size_t q8y_col = q81_bytes(e.attn_q);
    if (nc * (c.n_head / c.n_kv) <= 8 && c.n_rot == 64 && (c.n_head / c.n_kv) % 2 == 0) {
        // decode / verify: the per-head norm, RoPE and K / V store in the attention's partial launch
        RMI_TRY(rmi_gqa_flash_decode_prep_rt(e.proj, e.q3_rows, L.qn, L.kn, L.kc, L.vc, pos, nullptr, 0, e.q8y,
                                             static_cast<int>(q8y_col), e.attn_ws, c.n_head, c.n_kv, c.head_dim,
                                             c.n_rot, &e.rope, c.eps, nc, e.max_ctx, e.nsub,
                                             1.0f / sqrtf(static_cast<float>(c.head_dim)), e.rope_cs, rope_mode, e.s));
        RMI_TRY(gemv_res(e, L.out_proj, e.q8y, x, part, nc));
        return ffn(e, L, x, part, nc);
    }
    RMI_TRY(rmi_attn_prep_rope(e.proj, e.q3_rows, L.qn, L.kn, L.kc, L.vc, pos, e.qbuf, c.n_head, c.n_kv, c.head_dim,
                               c.n_rot, &e.rope, c.eps, nc, e.max_ctx, e.s));
    const int per = std::max(1, kAttnSlots / (c.n_head / c.n_kv));   // tokens per attention launch
    for (int c0 = 0; c0 < nc; c0 += per) {
        RMI_TRY(rmi_gqa_flash_decode(e.qbuf + static_cast<size_t>(c0) * e.attn_q, L.kc, L.vc, pos + c0,
                                     e.proj + static_cast<size_t>(c0) * e.q3_rows, e.q3_rows, nullptr, 0,
                                     e.q8y + c0 * q8y_col, static_cast<int>(q8y_col), e.attn_ws, c.n_head, c.n_kv,
                                     c.head_dim, std::min(per, nc - c0), e.max_ctx, e.nsub,
                                     1.0f / sqrtf(static_cast<float>(c.head_dim)), e.s));
    }
    RMI_TRY(gemv_res(e, L.out_proj, e.q8y, x, part, nc));
    return ffn(e, L, x, part, nc);
}

int gdn_block(Engine& e, Layer& L, int nc) {
    const auto& c = e.cfg;
    RMI_TRY(norm_gemv(e, L.in_proj, e.x, e.part, L.attn_norm, e.proj, nc));
    const int qkvz = 2 * c.ssm_h_k * kS + 2 * c.ssm_h_v * kS;
    RMI_TRY(rmi_gdn_layer_tokens_x(L.state[0], L.state[1], L.hist[0], L.hist[1], e.ints + kSel, e.proj, e.qkvz_rows,
                                   e.proj + qkvz, e.qkvz_rows, L.conv_w, L.dt, L.ssm_a, L.ssm_norm, c.eps, e.y, e.gdn_v,
                                   e.q8y, static_cast<int>(q81_bytes(e.gdn_v)), c.ssm_h_k, c.ssm_h_v, nc, e.gdn_xch,
                                   e.s));
    RMI_TRY(gemv_res(e, L.out_proj, e.q8y, e.x, e.part, nc));
    return ffn(e, L, e.x, e.part, nc);
}

enum Head { kHeadAll, kHeadLast, kHeadNone };

// trunk for nc columns: tokens tok[c] at positions pos[0] + c (pos: see attn_block).  The head (output norm, lm_head,
// argmax to ints[kV0 + c]) runs on every column, on the last one only (as ints[kV0]; an ingest chunk, qw:2700-2722),
// or not at all.  The final-normed hidden goes to h / hp (the draft's input, qw:1235-1237).
// what follows the lm_head of a decode forward in the same launch as the final norm (see verify_tail_kernel)
enum Tail { kTailNone, kTailVerify, kTailSingle };

int trunk_cols(Engine& e, int nc, const int* tok, const int* pos, float* h, float* hp, Head head,
               Tail tail = kTailNone) {
    const auto& c = e.cfg;
    RMI_TRY(rmi_embed(e.emb_type, e.tok_embd, tok, e.x, e.part, c.n_embd, c.n_vocab, nc, e.s));
    const int nl = static_cast<int>(e.layers.size());
    int rope_mode = 1;   // every attention layer of the pass rotates at pos: the first writes the table, the rest read
    for (int il = 0; il < nl; ++il) {
        Layer& L = e.layers[il];
        if (L.gdn) {
            RMI_TRY(gdn_block(e, L, nc));
        } else {
            RMI_TRY(attn_block(e, L, e.x, e.part, pos, nc, rope_mode));
            rope_mode = 2;
        }
    }
    if (head != kHeadNone) {
        const int first = head == kHeadAll ? 0 : nc - 1;
        const int ncol = nc - first;
        const uint8_t* xq = nullptr;
        RMI_TRY(norm_input(e, e.x, e.part, e.out_norm, first, ncol, &xq));
        RMI_TRY(gemv(e, e.lm_head, xq, e.logits, ncol));
        if (tail != kTailNone) {   // head on every column (nc 1 or 2): tokens, bookkeeping and final norm in one launch
            auto* keys = static_cast<uint64_t*>(e.argmax_ws);
            argmax_partial_launch(e.logits, c.n_vocab, nc, c.n_vocab, keys, e.s);
            const NormOut no{e.x, e.out_norm, e.part, h, hp, c.n_embd, c.eps};
            const dim3 grid(1 + nc * ((c.n_embd + 255) / 256));
            if (tail == kTailVerify)
                hipLaunchKernelGGL(verify_tail_kernel, grid, dim3(256), 0, e.s, e.ints, e.ring, keys, no);
            else
                hipLaunchKernelGGL(single_tail_kernel, grid, dim3(256), 0, e.s, e.ints, e.ring, keys, no);
            return launch_status("decode tail");
        }
        RMI_TRY(rmi_argmax(e.logits, c.n_vocab, ncol, c.n_vocab, e.ints + kV0, e.argmax_ws, e.s));
    }
    return rmi_rms_norm_out(e.x, e.out_norm, e.part, h, hp, c.n_embd, c.eps, nc, e.s);
}

// trunk for the decode columns: tokens ints[kTok0 + c] at positions ints[kPos] + c, head on every column
int trunk(Engine& e, int nc) {
    return trunk_cols(e, nc, e.ints + kTok0, e.ints + kPos, e.hsave, e.hpart, kHeadAll,
                      nc == 2 ? kTailVerify : kTailSingle);
}

// draft (nextn) block for nc columns: tokens tok[c] at positions pos[0] + c (pos: see attn_block), previous hidden
// h / hp.  eh_proj's input = [enorm(emb) | hnorm(h)] per column (embedding first, qw:1327-1332).  Argmax to
// ints[kC0 + c] when with_head.
// what follows the draft's lm_head (with_head): the round's finalize (2 columns) or the first candidate (1)
enum DraftTail { kDraftFinalize, kDraftFirst };

int draft_cols(Engine& e, const int* tok, const int* pos, const float* h, const float* hp, int nc, bool with_head,
               DraftTail dtail = kDraftFinalize) {
    const auto& c = e.cfg;
    // [enorm(emb) | hnorm(h)] straight into the Q8_1 row of eh_proj's input, the embedding rows dequantized in the
    // same launch: the bits of embed, norm, norm, quantize
    RMI_TRY(rmi_embed_quant_apply_pair(e.emb_type, e.tok_embd, tok, e.enorm, h, e.hnorm, hp, e.q8f, c.n_embd,
                                       c.n_vocab, c.eps, nc, e.s));
    RMI_TRY(gemv(e, e.eh_proj, e.q8f, e.dx, nc));
    // dx's partials: formed by the draft layer's first norm itself (one launch fewer)
    e.norm_self = true;
    RMI_TRY(attn_block(e, e.draft, e.dx, e.dpart, pos, nc));
    if (!with_head) return RMI_OK;
    const uint8_t* xq = nullptr;
    RMI_TRY(norm_input(e, e.dx, e.dpart, e.shnorm, 0, nc, &xq));
    RMI_TRY(gemv(e, e.lm_head, xq, e.logits, nc));
    auto* keys = static_cast<uint64_t*>(e.argmax_ws);
    argmax_partial_launch(e.logits, c.n_vocab, nc, c.n_vocab, keys, e.s);
    if (dtail == kDraftFinalize)
        hipLaunchKernelGGL(draft_tail_kernel, dim3(1), dim3(256), 0, e.s, e.ints, keys, e.ref_tok, e.pattern,
                           e.hsave, e.hpart, c.n_embd, c.n_embd / 4);
    else
        hipLaunchKernelGGL(first_tail_kernel, dim3(1), dim3(256), 0, e.s, e.ints, keys, e.ref_tok, e.pattern);
    return launch_status("draft tail");
}

// the decode draft: tokens ints[kD0 + c] at positions ints[kDPos] + c
int draft_block(Engine& e, const float* h, const float* hp, int nc, bool with_head,
                DraftTail dtail = kDraftFinalize) {
    return draft_cols(e, e.ints + kD0, e.ints + kDPos, h, hp, nc, with_head, dtail);
}

// One ingest chunk of nc prompt tokens from position ints[kPos] (the row-batched serve_ingest_kernels, qw:2192-2502,
// plus the draft KV rows of the same positions): the trunk on nc columns, every GEMV one weight pass for all of them,
// then the draft block on the same tokens with the hidden shifted by one column.  Every kernel computes each column
// as the single-column call does, so the chunk leaves the state the per-token path leaves.
int ingest_chunk(Engine& e, int nc, bool head) {
    const auto& c = e.cfg;
    const size_t np = c.n_embd / 4;
    hipLaunchKernelGGL(chunk_setup_kernel, dim3(1), dim3(kChunk), 0, e.s, e.ints, e.prompt, e.cints, nc);
    RMI_TRY(launch_status("chunk_setup"));
    const int* tok = e.cints;
    const int* pos = e.cints + kChunk;
    RMI_TRY(trunk_cols(e, nc, tok, pos, e.hsave + c.n_embd, e.hpart + np, head ? kHeadLast : kHeadNone));
    RMI_TRY(draft_cols(e, tok, pos, e.hsave, e.hpart, nc, false));
    hipLaunchKernelGGL(chunk_finish_kernel, dim3(1), dim3(256), 0, e.s, e.ints, e.hsave, e.hpart, c.n_embd,
                       static_cast<int>(np), nc, head ? 1 : 0);
    return launch_status("chunk_finish");
}

// the greedy forward of the current token; its tail launch emits the token and advances
int single_step(Engine& e) {
    return trunk(e, 1);
}

// the verify round: the trunk on (current, candidate), whose tail launch accepts or rejects, then the 2-column draft,
// whose tail launch picks the next candidate and advances
int verify_round(Engine& e) {
    RMI_TRY(trunk(e, 2));
    return draft_block(e, e.hsave, e.hpart, 2, true, kDraftFinalize);
}

// the first candidate: 1-column draft with head of (current token, hidden of the last forward) at the current position
int first_draft(Engine& e) {
    HIP_TRY(hipMemcpyAsync(e.ints + kD0, e.ints + kTok0, sizeof(int), hipMemcpyDeviceToDevice, e.s));
    HIP_TRY(hipMemcpyAsync(e.ints + kDPos, e.ints + kPos, sizeof(int), hipMemcpyDeviceToDevice, e.s));
    return draft_block(e, e.hsave, e.hpart, 1, true, kDraftFirst);
}

template <typename F>
int capture(Engine& e, hipGraphExec_t* out, F&& body) {
    if (*out) return RMI_OK;
    HIP_TRY(hipStreamBeginCapture(e.s, hipStreamCaptureModeThreadLocal));
    const int rc = body();
    hipGraph_t g = nullptr;
    const hipError_t ec = hipStreamEndCapture(e.s, &g);
    if (rc != RMI_OK) {
        if (g) (void) hipGraphDestroy(g);
        return rc;
    }
    RMI_TRY(hip_check(ec, "hipStreamEndCapture"));
    const hipError_t ei = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
    (void) hipGraphDestroy(g);
    return hip_check(ei, "hipGraphInstantiate");
}

int set_int(Engine& e, int slot, int v) {
    hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(256), 0, e.s, e.ints + slot, static_cast<size_t>(1), v);
    return launch_status("set_int");
}

int get_ints(Engine& e, int* host, int n) {
    HIP_TRY(hipMemcpyAsync(host, e.ints, sizeof(int) * n, hipMemcpyDeviceToHost, e.s));
    HIP_TRY(hipStreamSynchronize(e.s));
    return RMI_OK;
}

// The split GDN kernel waits, with a bound, for the other workgroups of a value head; a wait that runs out leaves the
// launch's outputs untrustworthy and bumps a device counter.  Every call that runs the trunk samples the counter
// before its launches and checks it after its last synchronization, so a timed-out wait is an error of that call
// instead of silently wrong tokens.
struct ExchangeGuard {
    unsigned int before = 0;
    int begin() {
        before = rmi_gdn_exchange_timeouts();
        if (before == 0xffffffffu) return fail(RMI_ERR_LAUNCH, "engine: cannot read the GDN exchange counter");
        return RMI_OK;
    }
    // call after the stream has been synchronized
    int end(const char* who) const {
        const unsigned int now = rmi_gdn_exchange_timeouts();
        if (now == 0xffffffffu) return fail(RMI_ERR_LAUNCH, "engine: cannot read the GDN exchange counter");
        if (now != before) {
            char msg[160];
            std::snprintf(msg, sizeof msg, "%s: %u GDN exchange wait(s) timed out; the generated tokens are not valid",
                          who, now - before);
            return fail(RMI_ERR_STATE, msg);
        }
        return RMI_OK;
    }
};

}  // namespace
}  // namespace rmi

using namespace rmi;

struct rmi_engine {
    Engine e;
};

extern "C" rmi_model_config rmi_qwen35_9b_config(void) {
    rmi_model_config c{};
    c.n_embd = 4096;
    c.n_ff = 12288;
    c.n_vocab = 248320;
    c.n_layer = 32;
    c.ssm_h_k = 16;
    c.ssm_h_v = 32;
    c.n_head = 16;
    c.n_kv = 4;
    c.head_dim = 256;
    c.n_rot = 64;
    c.rope_theta = 1e7f;
    c.eps = 1e-6f;
    c.rope_factor = 1.0f;
    c.rope_orig_ctx = 262144.0f;
    return c;
}

namespace rmi {
namespace {

int validate_config(const rmi_model_config& c, int max_ctx) {
    if (c.n_embd <= 0 || c.n_embd % 256 || c.n_ff % 256 || c.n_ff <= 0 || c.n_vocab <= 0 || c.n_layer <= 0 ||
        c.ssm_h_k <= 0 || c.ssm_h_v % c.ssm_h_k || c.head_dim != 256 || c.n_kv <= 0 || c.n_head % c.n_kv ||
        c.n_head <= 0 || (c.n_head / c.n_kv) * 2 > 16 || (c.ssm_h_v * kS) % 256 ||
        ((2 * c.ssm_h_k + c.ssm_h_v) * kS) % 256 || (c.n_head * c.head_dim) % 256 || c.n_rot < 0 || c.n_rot > 256 ||
        c.n_rot % 2 || !(c.rope_theta > 1.0f) || max_ctx < 64)
        return fail(RMI_ERR_SHAPE, "rmi_engine_create: unsupported model shape");
    return RMI_OK;
}

// configuration, stream, derived sizes and RoPE parameters
int setup(Engine& e, const rmi_model_config& c, int max_ctx, void* stream) {
    e.cfg = c;
    e.max_ctx = (max_ctx + 63) / 64 * 64;
    {
        const char* v = std::getenv("RMI_FUSE_NORM");
        e.fuse_norm = !(v && v[0] == '0');
    }
    // attention chunk = 64 * nsub positions, sized so that a full cache is one partial workgroup per CU (n_kv heads
    // per chunk), at least 128 positions: nsub 2 at 4K-class caches, 16 at 65536 positions, 17 at 66048 on 256 CUs.
    // Measured on the 9B round at 64K: nsub 4 / 6 / 8 / 12 / 16 -> 2655 / 2571 / 2603 / 2589 / 2540 us; at 4K nsub
    // 1 / 2 / 3 / 4 -> 2223 / 2191 / 2203 / 2210 us.  No upper clamp below 64: a 66048-position cache at nsub 16 is 65
    // chunks, 260 workgroups, and four CUs then run two of them (64K round 2518 -> 2496 us at nsub 17).
    {
        int cus = 0, dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        const int chunks = std::max(1, cus / std::max(1, c.n_kv));
        e.nsub = std::max(2, std::min(64, (e.max_ctx + 64 * chunks - 1) / (64 * chunks)));
    }
    {
        const char* v = std::getenv("RMI_ATTN_NSUB");   // an explicit chunk size (64 x 1..64 positions)
        if (v && *v) e.nsub = std::max(1, std::min(64, std::atoi(v)));
    }
    if (stream) {
        e.s = static_cast<hipStream_t>(stream);
    } else {
        HIP_TRY(hipStreamCreateWithFlags(&e.s, hipStreamNonBlocking));
        e.own_stream = true;
    }
    e.qkvz_rows = 2 * c.ssm_h_k * kS + 2 * c.ssm_h_v * kS + 2 * c.ssm_h_v;   // q|k|v|z|beta|alpha
    e.gdn_v = c.ssm_h_v * kS;
    e.attn_q = c.n_head * c.head_dim;
    e.q3_rows = 2 * e.attn_q + 2 * c.n_kv * c.head_dim;                     // 16 x (q|gate) | k | v
    e.max_in = std::max({c.n_ff, 2 * c.n_embd, e.gdn_v, e.attn_q});
    // qw:1991-1999: YaRN with ext_factor 1, attn_factor 1, beta_fast 32, beta_slow 1
    e.rope = rmi_rope_params{c.rope_theta, c.rope_factor > 1.0f ? c.rope_factor : 1.0f,
                             c.rope_orig_ctx > 0.0f ? c.rope_orig_ctx : 262144.0f, 1.0f, 1.0f, 32.0f, 1.0f};
    e.gen_tmp_bytes = std::max({q6_bytes(c.n_vocab, c.n_embd), q6_bytes(2 * c.n_ff, c.n_embd), q6_bytes(c.n_embd, c.n_ff),
                                q6_bytes(std::max(e.qkvz_rows, e.q3_rows), c.n_embd),
                                q6_bytes(c.n_embd, std::max(e.gdn_v, e.attn_q)), q6_bytes(c.n_embd, 2 * c.n_embd)});
    HIP_TRY(hipMalloc(&e.gen_tmp, e.gen_tmp_bytes));
    return RMI_OK;
}

// seeded random-init Q6_K model of the configured shapes (the benchmark configs)
int weights_synthetic(Engine& e, uint64_t seed) {
    const auto& c = e.cfg;
    RMI_TRY(e.alloc(&e.tok_embd, q6_bytes(c.n_vocab, c.n_embd)));
    RMI_TRY(rmi_gen_q6_k(e.tok_embd, static_cast<size_t>(c.n_vocab) * (c.n_embd / 256), mix_seed(seed, -1, 1), 1e-3f,
                         e.s));
    RMI_TRY(make_mat(e, e.lm_head, c.n_vocab, c.n_embd, mix_seed(seed, -1, 2)));
    RMI_TRY(make_vec(e, &e.out_norm, c.n_embd, mix_seed(seed, -1, 3), 1.0f, 0.1f));
    e.layers.resize(c.n_layer);
    for (int il = 0; il < c.n_layer; ++il) {
        const bool gdn = ((il + 1) % 4) != 0;   // qw:2016
        RMI_TRY(gdn ? make_gdn(e, e.layers[il], il, seed) : make_attn(e, e.layers[il], il, seed));
        if (gdn) {
            hipLaunchKernelGGL(neg_exp_kernel, dim3(grid1(c.ssm_h_v)), dim3(256), 0, e.s, e.layers[il].ssm_a, c.ssm_h_v);
            RMI_TRY(launch_status("ssm_a"));
        }
    }
    RMI_TRY(make_attn(e, e.draft, c.n_layer, seed));
    RMI_TRY(make_mat(e, e.eh_proj, c.n_embd, 2 * c.n_embd, mix_seed(seed, c.n_layer, 10)));
    RMI_TRY(make_vec(e, &e.enorm, c.n_embd, mix_seed(seed, c.n_layer, 11), 1.0f, 0.1f));
    RMI_TRY(make_vec(e, &e.hnorm, c.n_embd, mix_seed(seed, c.n_layer, 12), 1.0f, 0.1f));
    return make_vec(e, &e.shnorm, c.n_embd, mix_seed(seed, c.n_layer, 13), 1.0f, 0.1f);
}

// ---- GGUF weights -------------------------------------------------------------------------------------------------
struct GTensor {
    const char* name = nullptr;
    int type = -1, n_dims = 0;
    int64_t dims[4] = {1, 1, 1, 1};
    size_t bytes = 0;
    const void* data = nullptr;
};

bool find_tensor(const rmi_gguf* g, const std::string& name, GTensor* t) {
    const int64_t i = rmi_gguf_find(g, name.c_str());
    if (i < 0) return false;
    if (t) (void) rmi_gguf_tensor_info(g, i, &t->name, &t->type, &t->n_dims, t->dims, &t->bytes, &t->data);
    return true;
}

int need_tensor(const rmi_gguf* g, const std::string& name, GTensor* t) {
    if (!find_tensor(g, name, t)) return fail(RMI_ERR_SHAPE, ("gguf: missing tensor " + name).c_str());
    if (!t->data) return fail(RMI_ERR_UNSUPPORTED, ("gguf: unsupported tensor type for " + name).c_str());
    return RMI_OK;
}

std::string blk(int il, const char* what) { return "blk." + std::to_string(il) + "." + what; }

// host -> device through two pinned staging buffers (hipHostMalloc), copies of one overlapping the fill of the other
struct Uploader {
    static constexpr size_t kBuf = 32u << 20;
    uint8_t* pin[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    int next = 0;
    ~Uploader() {
        for (int i = 0; i < 2; ++i) {
            if (ev[i]) (void) hipEventDestroy(ev[i]);
            if (pin[i]) (void) hipHostFree(pin[i]);
        }
    }
    int init() {
        for (int i = 0; i < 2; ++i) {
            HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&pin[i]), kBuf, hipHostMallocDefault));
            HIP_TRY(hipEventCreateWithFlags(&ev[i], hipEventDisableTiming));
        }
        return RMI_OK;
    }
    int put(void* dst, const void* src, size_t n, hipStream_t s) {
        const auto* h = static_cast<const uint8_t*>(src);
        auto* d = static_cast<uint8_t*>(dst);
        for (size_t off = 0; off < n;) {
            const size_t len = std::min(kBuf, n - off);
            HIP_TRY(hipEventSynchronize(ev[next]));   // the copy that last used this buffer is done
            std::memcpy(pin[next], h + off, len);
            HIP_TRY(hipMemcpyAsync(d + off, pin[next], len, hipMemcpyHostToDevice, s));
            HIP_TRY(hipEventRecord(ev[next], s));
            next ^= 1;
            off += len;
        }
        return RMI_OK;
    }
};

// rows of the named tensors, concatenated in order (the reference's try_cat groups, qw:2082-2087), into one engine
// matrix when every part has the same type (Q6_K packed when n_in % 2048 == 0, else GGUF blocks); a group whose parts
// differ in type keeps them as parts (try_cat leaves such a group unfused, qw:1284-1288)
int load_mat(Engine& e, Uploader& up, const rmi_gguf* g, Mat& m, std::initializer_list<std::string> names,
             bool swiglu = false) {
    int n_in = -1, n_out = 0, type = -1;
    bool mixed = false;
    std::vector<GTensor> parts;
    for (const auto& nm : names) {
        GTensor t;
        RMI_TRY(need_tensor(g, nm, &t));
        if (t.n_dims != 2 || !rmi_native_mmvq_supported(t.type))
            return fail(RMI_ERR_UNSUPPORTED, ("gguf: " + nm + " is not a Q6_K / Q5_K / Q4_K / Q8_0 matrix").c_str());
        if (n_in >= 0 && t.dims[0] != n_in) return fail(RMI_ERR_SHAPE, ("gguf: " + nm + " has another row length").c_str());
        if (type >= 0 && t.type != type) mixed = true;
        n_in = static_cast<int>(t.dims[0]);
        n_out += static_cast<int>(t.dims[1]);
        type = t.type;
        parts.push_back(t);
    }
    m.n_in = n_in;
    m.n_out = n_out;
    m.bytes = 0;
    for (const auto& t : parts) m.bytes += t.bytes;
    if (mixed) {
        for (const auto& nm : names) {
            Mat p;
            RMI_TRY(load_mat(e, up, g, p, {nm}));
            m.parts.push_back(std::move(p));
        }
        return RMI_OK;
    }
    m.type = type;
    static const bool use_packed = [] {
        const char* v = std::getenv("RMI_ENGINE_PACKED");
        return !(v && v[0] == '0');
    }();
    m.packed = type == 14 && use_packed && n_in % 2048 == 0;
    uint8_t* dst = nullptr;
    if (m.packed) {
        if (m.bytes > e.gen_tmp_bytes) return fail(RMI_ERR_STATE, "engine: generation buffer too small");
        dst = e.gen_tmp;
    } else {
        RMI_TRY(e.alloc(&m.w, m.bytes));
        dst = m.w;
    }
    size_t off = 0;
    for (const auto& t : parts) {
        RMI_TRY(up.put(dst + off, t.data, t.bytes, e.s));
        off += t.bytes;
    }
    if (!m.packed) return RMI_OK;
    RMI_TRY(e.alloc(&m.w, rmi_q6_k_packed_bytes(n_in, n_out)));
    RMI_TRY(pack_mat(e, m, swiglu));
    HIP_TRY(hipStreamSynchronize(e.s));   // the next matrix reuses the staging buffer
    return RMI_OK;
}

int load_f32(Engine& e, Uploader& up, const rmi_gguf* g, float** p, const std::string& name, size_t n) {
    GTensor t;
    RMI_TRY(need_tensor(g, name, &t));
    size_t elems = 1;
    for (int d = 0; d < t.n_dims; ++d) elems *= static_cast<size_t>(t.dims[d]);
    if (t.type != 0 || elems != n) return fail(RMI_ERR_SHAPE, ("gguf: " + name + " is not an F32 vector of the expected size").c_str());
    RMI_TRY(e.alloc(p, n));
    return up.put(*p, t.data, n * sizeof(float), e.s);
}

int load_attn(Engine& e, Uploader& up, const rmi_gguf* g, Layer& L, int il) {
    const auto& c = e.cfg;
    L.gdn = false;
    RMI_TRY(load_f32(e, up, g, &L.attn_norm, blk(il, "attn_norm.weight"), c.n_embd));
    RMI_TRY(load_f32(e, up, g, &L.post_norm, blk(il, "post_attention_norm.weight"), c.n_embd));
    RMI_TRY(load_mat(e, up, g, L.in_proj, {blk(il, "attn_q.weight"), blk(il, "attn_k.weight"), blk(il, "attn_v.weight")}));
    RMI_TRY(load_mat(e, up, g, L.out_proj, {blk(il, "attn_output.weight")}));
    RMI_TRY(load_mat(e, up, g, L.upgate, {blk(il, "ffn_up.weight"), blk(il, "ffn_gate.weight")}, true));
    RMI_TRY(load_mat(e, up, g, L.down, {blk(il, "ffn_down.weight")}));
    RMI_TRY(load_f32(e, up, g, &L.qn, blk(il, "attn_q_norm.weight"), c.head_dim));
    RMI_TRY(load_f32(e, up, g, &L.kn, blk(il, "attn_k_norm.weight"), c.head_dim));
    if (L.in_proj.n_out != e.q3_rows || L.out_proj.n_in != e.attn_q || L.upgate.n_out != 2 * c.n_ff ||
        L.down.n_in != c.n_ff || L.in_proj.n_in != c.n_embd)
        return fail(RMI_ERR_SHAPE, ("gguf: attention layer " + std::to_string(il) + " has unexpected shapes").c_str());
    return alloc_attn_state(e, L);
}

int load_gdn(Engine& e, Uploader& up, const rmi_gguf* g, Layer& L, int il) {
    const auto& c = e.cfg;
    L.gdn = true;
    RMI_TRY(load_f32(e, up, g, &L.attn_norm, blk(il, "attn_norm.weight"), c.n_embd));
    RMI_TRY(load_f32(e, up, g, &L.post_norm, blk(il, "post_attention_norm.weight"), c.n_embd));
    // qkv | z | beta | alpha: the reference's qkvz and ab groups (beta before alpha, qw:2085) as one GEMV
    RMI_TRY(load_mat(e, up, g, L.in_proj, {blk(il, "attn_qkv.weight"), blk(il, "attn_gate.weight"),
                                           blk(il, "ssm_beta.weight"), blk(il, "ssm_alpha.weight")}));
    RMI_TRY(load_mat(e, up, g, L.out_proj, {blk(il, "ssm_out.weight")}));
    RMI_TRY(load_mat(e, up, g, L.upgate, {blk(il, "ffn_up.weight"), blk(il, "ffn_gate.weight")}, true));
    RMI_TRY(load_mat(e, up, g, L.down, {blk(il, "ffn_down.weight")}));
    const int ch = 2 * c.ssm_h_k * kS + c.ssm_h_v * kS;
    RMI_TRY(load_f32(e, up, g, &L.conv_w, blk(il, "ssm_conv1d.weight"), static_cast<size_t>(4) * ch));
    RMI_TRY(load_f32(e, up, g, &L.dt, blk(il, "ssm_dt.bias"), c.ssm_h_v));
    RMI_TRY(load_f32(e, up, g, &L.ssm_a, blk(il, "ssm_a"), c.ssm_h_v));
    RMI_TRY(load_f32(e, up, g, &L.ssm_norm, blk(il, "ssm_norm.weight"), kS));
    if (L.in_proj.n_out != e.qkvz_rows || L.out_proj.n_in != e.gdn_v || L.upgate.n_out != 2 * c.n_ff ||
        L.down.n_in != c.n_ff || L.in_proj.n_in != c.n_embd)
        return fail(RMI_ERR_SHAPE, ("gguf: GDN layer " + std::to_string(il) + " has unexpected shapes").c_str());
    return alloc_gdn_state(e, L);
}

double meta_num(const rmi_gguf* g, const char* key, double def) {
    double v = def;
    return rmi_gguf_get_num(g, key, &v) == RMI_OK ? v : def;
}

// the model configuration from a qwen35 file: shapes from the tensors, eps / RoPE / YaRN from the metadata
int gguf_config(const rmi_gguf* g, rmi_model_config* c) {
    const char* arch = nullptr;
    if (rmi_gguf_get_str(g, "general.architecture", &arch) != RMI_OK || std::string(arch) != "qwen35")
        return fail(RMI_ERR_UNSUPPORTED, "gguf: not a qwen35 GGUF");
    double blocks = 0, nextn = 0;
    if (rmi_gguf_get_num(g, "qwen35.block_count", &blocks) != RMI_OK ||
        rmi_gguf_get_num(g, "qwen35.nextn_predict_layers", &nextn) != RMI_OK || nextn != 1)
        return fail(RMI_ERR_SHAPE, "gguf: qwen35 file without block_count / one nextn layer");
    *c = rmi_model_config{};
    c->n_layer = static_cast<int>(blocks - nextn);
    GTensor emb, up, qkv, ssma, qn, aq, ak, snorm;
    RMI_TRY(need_tensor(g, "token_embd.weight", &emb));
    c->n_embd = static_cast<int>(emb.dims[0]);
    c->n_vocab = static_cast<int>(emb.dims[1]);
    RMI_TRY(need_tensor(g, blk(0, "ffn_up.weight"), &up));
    c->n_ff = static_cast<int>(up.dims[1]);
    int first_attn = -1, first_gdn = -1;
    for (int il = 0; il < c->n_layer; ++il) {
        const bool a = find_tensor(g, blk(il, "attn_q.weight"), nullptr);
        const bool d = find_tensor(g, blk(il, "attn_qkv.weight"), nullptr);
        if (a == d) return fail(RMI_ERR_SHAPE, ("gguf: layer " + std::to_string(il) + " is neither GDN nor attention").c_str());
        if (a && first_attn < 0) first_attn = il;
        if (d && first_gdn < 0) first_gdn = il;
    }
    const int ai = first_attn >= 0 ? first_attn : c->n_layer;   // the draft block is an attention layer
    RMI_TRY(need_tensor(g, blk(ai, "attn_q_norm.weight"), &qn));
    RMI_TRY(need_tensor(g, blk(ai, "attn_q.weight"), &aq));
    RMI_TRY(need_tensor(g, blk(ai, "attn_k.weight"), &ak));
    c->head_dim = static_cast<int>(qn.dims[0]);
    c->n_head = static_cast<int>(aq.dims[1] / (2 * c->head_dim));
    c->n_kv = static_cast<int>(ak.dims[1] / c->head_dim);
    if (first_gdn >= 0) {
        RMI_TRY(need_tensor(g, blk(first_gdn, "ssm_a"), &ssma));
        RMI_TRY(need_tensor(g, blk(first_gdn, "attn_qkv.weight"), &qkv));
        RMI_TRY(need_tensor(g, blk(first_gdn, "ssm_norm.weight"), &snorm));
        if (snorm.dims[0] != kS) return fail(RMI_ERR_SHAPE, "gguf: GDN state size must be 128");
        c->ssm_h_v = static_cast<int>(ssma.dims[0]);
        c->ssm_h_k = static_cast<int>((qkv.dims[1] - static_cast<int64_t>(kS) * c->ssm_h_v) / (2 * kS));
    } else {
        c->ssm_h_k = 1;
        c->ssm_h_v = 2;
    }
    c->n_rot = static_cast<int>(meta_num(g, "qwen35.rope.dimension_count", 64));
    c->rope_theta = static_cast<float>(meta_num(g, "qwen35.rope.freq_base", 1e7));
    c->eps = static_cast<float>(meta_num(g, "qwen35.attention.layer_norm_rms_epsilon", 1e-6));
    c->rope_factor = static_cast<float>(meta_num(g, "qwen35.rope.scaling.factor", 1.0));
    c->rope_orig_ctx = static_cast<float>(meta_num(g, "qwen35.rope.scaling.original_context_length", 262144.0));
    return RMI_OK;
}

int weights_gguf(Engine& e, const rmi_gguf* g) {
    const auto& c = e.cfg;
    Uploader up;
    RMI_TRY(up.init());
    GTensor emb;
    RMI_TRY(need_tensor(g, "token_embd.weight", &emb));
    if (emb.type != 14 && emb.type != 13 && emb.type != 12)
        return fail(RMI_ERR_UNSUPPORTED, "gguf: token_embd must be Q6_K, Q5_K or Q4_K");
    e.emb_type = emb.type;
    RMI_TRY(e.alloc(&e.tok_embd, emb.bytes));
    RMI_TRY(up.put(e.tok_embd, emb.data, emb.bytes, e.s));
    RMI_TRY(load_mat(e, up, g, e.lm_head, {"output.weight"}));
    RMI_TRY(load_f32(e, up, g, &e.out_norm, "output_norm.weight", c.n_embd));
    if (e.lm_head.n_out != c.n_vocab || e.lm_head.n_in != c.n_embd) return fail(RMI_ERR_SHAPE, "gguf: bad output.weight");
    e.layers.resize(c.n_layer);
    for (int il = 0; il < c.n_layer; ++il) {
        if (find_tensor(g, blk(il, "attn_qkv.weight"), nullptr)) RMI_TRY(load_gdn(e, up, g, e.layers[il], il));
        else RMI_TRY(load_attn(e, up, g, e.layers[il], il));
    }
    const int d = c.n_layer;   // the nextn draft block (qw:2096-2126)
    RMI_TRY(load_attn(e, up, g, e.draft, d));
    RMI_TRY(load_mat(e, up, g, e.eh_proj, {blk(d, "nextn.eh_proj.weight")}));
    if (e.eh_proj.n_in != 2 * c.n_embd || e.eh_proj.n_out != c.n_embd) return fail(RMI_ERR_SHAPE, "gguf: bad eh_proj");
    RMI_TRY(load_f32(e, up, g, &e.hnorm, blk(d, "nextn.hnorm.weight"), c.n_embd));
    RMI_TRY(load_f32(e, up, g, &e.enorm, blk(d, "nextn.enorm.weight"), c.n_embd));
    RMI_TRY(load_f32(e, up, g, &e.shnorm, blk(d, "nextn.shared_head_norm.weight"), c.n_embd));
    HIP_TRY(hipStreamSynchronize(e.s));   // the staging buffers are freed on return
    return RMI_OK;
}

// round state and activations (kChunk columns), after the weights
int alloc_runtime(Engine& e) {
    const auto& c = e.cfg;
    HIP_TRY(hipStreamSynchronize(e.s));   // every pack has read the staging buffer
    HIP_TRY(hipFree(e.gen_tmp));
    e.gen_tmp = nullptr;
    RMI_TRY(e.alloc(&e.ints, 64));
    hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(256), 0, e.s, e.ints, static_cast<size_t>(64), 0);
    RMI_TRY(launch_status("fill"));
    RMI_TRY(set_int(e, kVocab, c.n_vocab));
    RMI_TRY(set_int(e, kMaxPos, e.max_ctx - 1));
    RMI_TRY(e.alloc(&e.ring, kRingCap));
    if (c.ssm_h_v > 0) {
        const size_t xb = rmi_gdn_exchange_bytes(c.ssm_h_v);
        RMI_TRY(e.alloc(&e.gdn_xch, xb / sizeof(unsigned long long)));
        HIP_TRY(hipMemsetAsync(e.gdn_xch, 0, xb, e.s));   // once, before any graph is captured
    }
    RMI_TRY(e.alloc(&e.ref_tok, static_cast<size_t>(e.max_ctx) + 1));
    RMI_TRY(e.alloc(&e.pattern, 4096));
    const size_t np = c.n_embd / 4;
    const size_t K = kChunk;
    RMI_TRY(e.alloc(&e.cints, 2 * K));
    RMI_TRY(e.alloc(&e.prompt, static_cast<size_t>(e.max_ctx)));
    RMI_TRY(e.alloc(&e.x, K * c.n_embd));
    RMI_TRY(e.alloc(&e.part, K * np));
    RMI_TRY(e.alloc(&e.proj, K * std::max(e.qkvz_rows, e.q3_rows)));
    RMI_TRY(e.alloc(&e.ug, K * 2 * c.n_ff));
    RMI_TRY(e.alloc(&e.y, K * std::max(e.gdn_v, e.attn_q)));
    RMI_TRY(e.alloc(&e.logits, 2 * static_cast<size_t>(c.n_vocab)));
    RMI_TRY(e.alloc(&e.hsave, (K + 1) * c.n_embd));
    RMI_TRY(e.alloc(&e.hpart, (K + 1) * np));
    RMI_TRY(e.alloc(&e.hzero, static_cast<size_t>(c.n_embd)));
    RMI_TRY(e.alloc(&e.pzero, np));
    RMI_TRY(zero_f32(e, e.hzero, c.n_embd));
    RMI_TRY(zero_f32(e, e.pzero, np));
    RMI_TRY(e.alloc(&e.qbuf, K * e.attn_q));
    RMI_TRY(e.alloc(&e.dx, K * c.n_embd));
    RMI_TRY(e.alloc(&e.dpart, K * np));
    RMI_TRY(e.alloc(&e.q8a, K * q81_bytes(c.n_embd)));
    RMI_TRY(e.alloc(&e.q8f, K * q81_bytes(e.max_in)));
    RMI_TRY(e.alloc(&e.q8y, K * q81_bytes(std::max(e.gdn_v, e.attn_q))));
    uint8_t* ws = nullptr;
    RMI_TRY(e.alloc(&ws, rmi_gqa_workspace_bytes(e.max_ctx, c.n_kv, e.nsub)));
    e.attn_ws = ws;
    RMI_TRY(e.alloc(&e.rope_cs, rmi_gqa_rope_table_bytes(c.n_rot) / sizeof(float)));
    uint8_t* aw = nullptr;
    RMI_TRY(e.alloc(&aw, rmi_argmax_workspace_bytes(2)));
    e.argmax_ws = aw;
    uint8_t* tw = nullptr;
    RMI_TRY(e.alloc(&tw, rmi_topk_workspace_bytes(c.n_vocab)));
    e.topk_ws = tw;
    RMI_TRY(e.alloc(&e.topk_out, 128));
    for (auto& L : e.layers) {
        if (!L.gdn) continue;
        float *s0 = nullptr, *h0 = nullptr;
        RMI_TRY(e.alloc(&s0, static_cast<size_t>(kS) * c.ssm_h_v * kS));
        RMI_TRY(e.alloc(&h0, hist_floats(c)));
        e.saved_state.push_back(s0);
        e.saved_hist.push_back(h0);
    }
    RMI_TRY(e.alloc(&e.saved_h, static_cast<size_t>(c.n_embd)));
    RMI_TRY(e.alloc(&e.saved_hp, np));
    HIP_TRY(hipEventCreate(&e.ev0));
    HIP_TRY(hipEventCreate(&e.ev1));
    HIP_TRY(hipStreamSynchronize(e.s));
    return RMI_OK;
}

}  // namespace
}  // namespace rmi

extern "C" int rmi_engine_create(const rmi_model_config* cfg, uint64_t seed, int max_ctx, void* stream,
                                 rmi_engine** out) {
    if (!cfg || !out) return fail(RMI_ERR_POINTER, "rmi_engine_create: null argument");
    RMI_TRY(validate_config(*cfg, max_ctx));
    std::unique_ptr<rmi_engine> h(new (std::nothrow) rmi_engine());
    if (!h) return fail(RMI_ERR_STATE, "rmi_engine_create: out of host memory");
    RMI_TRY(setup(h->e, *cfg, max_ctx, stream));
    RMI_TRY(weights_synthetic(h->e, seed));
    RMI_TRY(alloc_runtime(h->e));
    *out = h.release();
    return RMI_OK;
}

extern "C" int rmi_engine_create_gguf(const char* path, int max_ctx, void* stream, rmi_engine** out) {
    if (!path || !out) return fail(RMI_ERR_POINTER, "rmi_engine_create_gguf: null argument");
    rmi_gguf* g = nullptr;
    RMI_TRY(rmi_gguf_open(path, &g));
    std::unique_ptr<rmi_gguf, void (*)(rmi_gguf*)> file(g, rmi_gguf_close);
    rmi_model_config c{};
    RMI_TRY(gguf_config(g, &c));
    RMI_TRY(validate_config(c, max_ctx));
    std::unique_ptr<rmi_engine> h(new (std::nothrow) rmi_engine());
    if (!h) return fail(RMI_ERR_STATE, "rmi_engine_create_gguf: out of host memory");
    RMI_TRY(setup(h->e, c, max_ctx, stream));
    RMI_TRY(weights_gguf(h->e, g));
    RMI_TRY(alloc_runtime(h->e));
    *out = h.release();
    return RMI_OK;
}

extern "C" int rmi_engine_config(const rmi_engine* h, rmi_model_config* out) {
    if (!h || !out) return fail(RMI_ERR_POINTER, "rmi_engine_config: null argument");
    *out = h->e.cfg;
    return RMI_OK;
}

extern "C" int rmi_engine_destroy(rmi_engine* h) {
    if (!h) return RMI_OK;
    (void) hipStreamSynchronize(h->e.s);
    delete h;
    return RMI_OK;
}

extern "C" int rmi_engine_info(const rmi_engine* h, rmi_engine_info_t* info) {
    if (!h || !info) return fail(RMI_ERR_POINTER, "rmi_engine_info: null argument");
    const Engine& e = h->e;
    const auto& c = e.cfg;
    size_t trunk = 0;
    for (const auto& L : e.layers) trunk += L.in_proj.bytes + L.out_proj.bytes + L.upgate.bytes + L.down.bytes;
    const size_t head = e.lm_head.bytes;
    const size_t dblk = e.eh_proj.bytes + e.draft.in_proj.bytes + e.draft.out_proj.bytes + e.draft.upgate.bytes +
                        e.draft.down.bytes;
    info->trunk_weight_bytes = trunk;
    info->lm_head_bytes = head;
    info->draft_block_bytes = dblk;
    info->round_weight_bytes = trunk + head + dblk + head;
    info->token_weight_bytes = trunk + head;
    int n_attn = 0;
    for (const auto& L : e.layers) n_attn += L.gdn ? 0 : 1;
    info->kv_bytes_per_pos = static_cast<size_t>(n_attn) * 2 * c.n_kv * c.head_dim * 2;
    info->gdn_layers = c.n_layer - n_attn;
    info->attn_layers = n_attn;
    info->max_ctx = e.max_ctx;
    info->attn_chunk = 64 * e.nsub;
    return RMI_OK;
}

// Fill the context [0, n_ctx - 1) with seeded synthetic state (fp16 KV N(0,1) for trunk and draft layers, GDN state
// N(0, 0.05^2), conv history N(0, 0.5^2)), then run one real forward of `last_token` at position n_ctx - 1.
extern "C" int rmi_engine_synth_context(rmi_engine* h, int n_ctx, uint64_t seed, int last_token, int* first_out) {
    if (!h) return fail(RMI_ERR_POINTER, "rmi_engine_synth_context: null engine");
    Engine& e = h->e;
    e.stream_mode = -1;
    const auto& c = e.cfg;
    if (n_ctx < 1 || n_ctx >= e.max_ctx - 2 || last_token < 0 || last_token >= c.n_vocab)
        return fail(RMI_ERR_STATE, "rmi_engine_synth_context: context does not fit");
    const size_t kv = static_cast<size_t>(n_ctx - 1) * c.n_kv * c.head_dim;
    int il = 0;
    for (auto& L : e.layers) {
        if (L.gdn) {
            const size_t st = static_cast<size_t>(kS) * c.ssm_h_v * kS;
            // a [channels][3] history N(0, 0.5^2) (in the non-live buffer, overwritten by the next verify anyway),
            // expanded to the per-value-head layout of the live one
            const size_t hs = static_cast<size_t>(3) * (2 * c.ssm_h_k + c.ssm_h_v) * kS;
            RMI_TRY(rmi_gen_normal(L.state[0], st, mix_seed(seed, il, 20), 0.0f, 0.05f, e.s));
            RMI_TRY(rmi_gen_normal(L.hist[1], hs, mix_seed(seed, il, 21), 0.0f, 0.5f, e.s));
            hipLaunchKernelGGL(hist_expand_kernel, dim3(grid1(c.ssm_h_v * 3 * kS)), dim3(256), 0, e.s, L.hist[1],
                               L.hist[0], c.ssm_h_k, c.ssm_h_v);
            RMI_TRY(launch_status("hist_expand"));
        } else if (kv) {
            RMI_TRY(rmi_gen_normal_f16(L.kc, kv, mix_seed(seed, il, 22), 0.0f, 1.0f, e.s));
            RMI_TRY(rmi_gen_normal_f16(L.vc, kv, mix_seed(seed, il, 23), 0.0f, 1.0f, e.s));
        }
        ++il;
    }
    if (kv) {
        RMI_TRY(rmi_gen_normal_f16(e.draft.kc, kv + static_cast<size_t>(c.n_kv) * c.head_dim, mix_seed(seed, il, 22),
                                   0.0f, 1.0f, e.s));
        RMI_TRY(rmi_gen_normal_f16(e.draft.vc, kv + static_cast<size_t>(c.n_kv) * c.head_dim, mix_seed(seed, il, 23),
                                   0.0f, 1.0f, e.s));
    }
    RMI_TRY(set_int(e, kSel, 0));
    RMI_TRY(set_int(e, kPos, n_ctx - 1));
    RMI_TRY(set_int(e, kTok0, last_token));
    RMI_TRY(set_int(e, kNOut, 0));
    RMI_TRY(single_step(e));
    int st[kNumSlots];
    RMI_TRY(get_ints(e, st, kNumSlots));
    if (first_out) *first_out = st[kTok0];
    return RMI_OK;
}

// Empty context: zero GDN state and history (both buffers), selector 0, position 0, and a zero hidden as the input of
// the first draft row (the reference's serve reset, qw:2533-2549; KV rows need no clearing, attention reads only rows
// below the position it writes).
extern "C" int rmi_engine_reset(rmi_engine* h) {
    if (!h) return fail(RMI_ERR_POINTER, "rmi_engine_reset: null engine");
    Engine& e = h->e;
    const auto& c = e.cfg;
    for (auto& L : e.layers)
        if (L.gdn) {
            for (int b = 0; b < 2; ++b) {
                RMI_TRY(zero_f32(e, L.state[b], static_cast<size_t>(kS) * c.ssm_h_v * kS));
                RMI_TRY(zero_f32(e, L.hist[b], hist_floats(c)));
            }
        }
    RMI_TRY(zero_f32(e, e.hsave, c.n_embd));
    RMI_TRY(zero_f32(e, e.hpart, c.n_embd / 4));
    RMI_TRY(set_int(e, kSel, 0));
    RMI_TRY(set_int(e, kPos, 0));
    RMI_TRY(set_int(e, kTok0, 0));
    RMI_TRY(set_int(e, kNOut, 0));
    e.stream_mode = -1;
    HIP_TRY(hipStreamSynchronize(e.s));
    return RMI_OK;
}

// Feed n tokens from the current position, filling the draft's KV as the reference seeds it (slot 0 with a zero hidden,
// qw:2956-2958) and every later slot with (token, previous final-normed hidden).  batch 1: one token at a time (the
// trunk with its head, then the draft row, per token; forward_token, qw:1773-1824).  batch 2..16: chunks of `batch`
// tokens, each one pass over the weights (the ingest of qw:2658-2722), the head on the last token only; a full chunk is
// one hipGraph launch.  Both leave the same state.  *first_out = the greedy token after the last one fed (the current
// token).  After a generation the context continues at its position, as the reference's serve loop does.
extern "C" int rmi_engine_ingest(rmi_engine* h, const int* tokens, int n, int batch, int* first_out) {
    if (!h || !tokens) return fail(RMI_ERR_POINTER, "rmi_engine_ingest: null argument");
    Engine& e = h->e;
    const auto& c = e.cfg;
    if (batch < 1 || batch > kChunk) return fail(RMI_ERR_SHAPE, "rmi_engine_ingest: batch must be 1..16");
    for (int i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= c.n_vocab) return fail(RMI_ERR_STATE, "rmi_engine_ingest: bad token id");
    int st[kNumSlots];
    RMI_TRY(get_ints(e, st, kNumSlots));
    const int pos0 = st[kPos];
    if (n < 1 || pos0 + n >= e.max_ctx - 2) return fail(RMI_ERR_STATE, "rmi_engine_ingest: context does not fit");
    RMI_TRY(set_int(e, kNOut, 0));
    e.stream_mode = -1;
    ExchangeGuard xg;
    RMI_TRY(xg.begin());
    if (batch == 1) {
        for (int i = 0; i < n; ++i) {
            // draft KV slot p from (token, hidden of position p - 1) - the zero hidden at slot 0
            const int p = pos0 + i;
            RMI_TRY(set_int(e, kD0, tokens[i]));
            RMI_TRY(set_int(e, kDPos, p));
            RMI_TRY(draft_block(e, p == 0 ? e.hzero : e.hsave, p == 0 ? e.pzero : e.hpart, 1, false));
            RMI_TRY(set_int(e, kTok0, tokens[i]));
            RMI_TRY(set_int(e, kPos, p));
            RMI_TRY(single_step(e));
        }
    } else {
        // the chunk kernels read the tokens by position; hidden column 0 holds the hidden of position pos0 - 1 (zero
        // after a reset)
        HIP_TRY(hipMemcpyAsync(e.prompt + pos0, tokens, sizeof(int) * static_cast<size_t>(n), hipMemcpyHostToDevice,
                               e.s));
        int i = 0;
        if (batch == kChunk && n > kChunk) {
            RMI_TRY(capture(e, &e.g_chunk, [&] { return ingest_chunk(e, kChunk, false); }));
            for (; n - i > kChunk; i += kChunk) HIP_TRY(hipGraphLaunch(e.g_chunk, e.s));
        }
        for (; i < n; i += batch) {
            const int nc = std::min(batch, n - i);
            RMI_TRY(ingest_chunk(e, nc, i + nc == n));
        }
    }
    RMI_TRY(get_ints(e, st, kNumSlots));   // synchronizes: the host tokens are no longer read
    RMI_TRY(xg.end("rmi_engine_ingest"));
    if (first_out) *first_out = st[kTok0];
    return RMI_OK;
}

// the prompt from position 0: reset, then ingest
extern "C" int rmi_engine_prefill_batch(rmi_engine* h, const int* tokens, int n, int batch, int* first_out) {
    if (!h || !tokens) return fail(RMI_ERR_POINTER, "rmi_engine_prefill: null argument");
    if (n < 1 || n >= h->e.max_ctx - 2) return fail(RMI_ERR_STATE, "rmi_engine_prefill: context does not fit");
    if (batch < 1 || batch > kChunk) return fail(RMI_ERR_SHAPE, "rmi_engine_prefill: batch must be 1..16");
    RMI_TRY(rmi_engine_reset(h));
    return rmi_engine_ingest(h, tokens, n, batch, first_out);
}

extern "C" int rmi_engine_prefill(rmi_engine* h, const int* tokens, int n, int* first_out) {
    return rmi_engine_prefill_batch(h, tokens, n, kChunk, first_out);
}

// Copy bytes [offset, offset + bytes) of an engine buffer to host memory (synchronous).  layer indexes the trunk
// layers; n_layer names the draft block (K/V caches only).  GDN buffers are the live ones.
extern "C" int rmi_engine_read(rmi_engine* h, int which, int layer, size_t offset, void* dst, size_t bytes) {
    if (!h || !dst) return fail(RMI_ERR_POINTER, "rmi_engine_read: null argument");
    Engine& e = h->e;
    const auto& c = e.cfg;
    if (layer < 0 || layer > c.n_layer) return fail(RMI_ERR_SHAPE, "rmi_engine_read: bad layer");
    const Layer& L = layer == c.n_layer ? e.draft : e.layers[layer];
    int st[kNumSlots];
    RMI_TRY(get_ints(e, st, kNumSlots));
    const void* src = nullptr;
    size_t size = 0;
    switch (which) {
        case RMI_BUF_GDN_STATE:
        case RMI_BUF_GDN_HIST:
            if (!L.gdn || layer == c.n_layer) return fail(RMI_ERR_SHAPE, "rmi_engine_read: not a GDN layer");
            src = which == RMI_BUF_GDN_STATE ? static_cast<const void*>(L.state[st[kSel] & 1]) : L.hist[st[kSel] & 1];
            size = which == RMI_BUF_GDN_STATE ? sizeof(float) * kS * c.ssm_h_v * kS : sizeof(float) * hist_floats(c);
            break;
        case RMI_BUF_K_CACHE:
        case RMI_BUF_V_CACHE:
            if (L.gdn) return fail(RMI_ERR_SHAPE, "rmi_engine_read: not an attention layer");
            src = which == RMI_BUF_K_CACHE ? L.kc : L.vc;
            size = sizeof(uint16_t) * e.max_ctx * c.n_kv * c.head_dim;
            break;
        case RMI_BUF_HIDDEN:
            src = e.hsave;
            size = sizeof(float) * c.n_embd;
            break;
        case RMI_BUF_LOGITS:
            src = e.logits;
            size = sizeof(float) * 2 * static_cast<size_t>(c.n_vocab);
            break;
        case RMI_BUF_ROUND: {
            const int slots[8] = {st[kPos], st[kTok0], st[kTok1], st[kV0], st[kV1], st[kC0], st[kC1], st[kAccept]};
            if (offset > sizeof(slots) || bytes > sizeof(slots) - offset)
                return fail(RMI_ERR_SHAPE, "rmi_engine_read: range outside the buffer");
            std::memcpy(dst, reinterpret_cast<const uint8_t*>(slots) + offset, bytes);
            return RMI_OK;
        }
        default:
            return fail(RMI_ERR_SHAPE, "rmi_engine_read: bad buffer");
    }
    if (offset > size || bytes > size - offset) return fail(RMI_ERR_SHAPE, "rmi_engine_read: range outside the buffer");
    HIP_TRY(hipMemcpyAsync(dst, static_cast<const uint8_t*>(src) + offset, bytes, hipMemcpyDeviceToHost, e.s));
    HIP_TRY(hipStreamSynchronize(e.s));
    return RMI_OK;
}

extern "C" int rmi_engine_save_state(rmi_engine* h) {
    if (!h) return fail(RMI_ERR_POINTER, "null engine");
    Engine& e = h->e;
    const auto& c = e.cfg;
    int st[kNumSlots];
    RMI_TRY(get_ints(e, st, kNumSlots));
    size_t k = 0;
    for (auto& L : e.layers) {
        if (!L.gdn) continue;
        HIP_TRY(hipMemcpyAsync(e.saved_state[k], L.state[st[kSel]], sizeof(float) * kS * c.ssm_h_v * kS,
                               hipMemcpyDeviceToDevice, e.s));
        HIP_TRY(hipMemcpyAsync(e.saved_hist[k], L.hist[st[kSel]], sizeof(float) * hist_floats(c),
                               hipMemcpyDeviceToDevice, e.s));
        ++k;
    }
    HIP_TRY(hipMemcpyAsync(e.saved_h, e.hsave, sizeof(float) * c.n_embd, hipMemcpyDeviceToDevice, e.s));
    HIP_TRY(hipMemcpyAsync(e.saved_hp, e.hpart, sizeof(float) * (c.n_embd / 4), hipMemcpyDeviceToDevice, e.s));
    HIP_TRY(hipStreamSynchronize(e.s));
    return RMI_OK;
}

// restore the GDN state saved by rmi_engine_save_state and the token / position / hidden it was taken with
extern "C" int rmi_engine_restore_state(rmi_engine* h, int pos, int cur_token) {
    if (!h) return fail(RMI_ERR_POINTER, "null engine");
    Engine& e = h->e;
    e.stream_mode = -1;
    const auto& c = e.cfg;
    size_t k = 0;
    for (auto& L : e.layers) {
        if (!L.gdn) continue;
        HIP_TRY(hipMemcpyAsync(L.state[0], e.saved_state[k], sizeof(float) * kS * c.ssm_h_v * kS,
                               hipMemcpyDeviceToDevice, e.s));
        HIP_TRY(hipMemcpyAsync(L.hist[0], e.saved_hist[k], sizeof(float) * hist_floats(c),
                               hipMemcpyDeviceToDevice, e.s));
        ++k;
    }
    HIP_TRY(hipMemcpyAsync(e.hsave, e.saved_h, sizeof(float) * c.n_embd, hipMemcpyDeviceToDevice, e.s));
    HIP_TRY(hipMemcpyAsync(e.hpart, e.saved_hp, sizeof(float) * (c.n_embd / 4), hipMemcpyDeviceToDevice, e.s));
    RMI_TRY(set_int(e, kSel, 0));
    RMI_TRY(set_int(e, kPos, pos));
    RMI_TRY(set_int(e, kTok0, cur_token));
    HIP_TRY(hipStreamSynchronize(e.s));
    return RMI_OK;
}

extern "C" int rmi_engine_state(rmi_engine* h, int* pos, int* cur_token) {
    if (!h) return fail(RMI_ERR_POINTER, "null engine");
    int st[kNumSlots];
    RMI_TRY(get_ints(h->e, st, kNumSlots));
    if (pos) *pos = st[kPos];
    if (cur_token) *cur_token = st[kTok0];
    return RMI_OK;
}

// Generate n_gen tokens after the current token.  mode RMI_GEN_GREEDY: one forward per token (graph).  RMI_GEN_MTP:
// draft + 2-column verify rounds (graph).  RMI_GEN_MTP_FORCED: as MTP, but each round's candidate is replaced by
// ref_tokens[pos + 1 - ref_base] when pattern[round % pattern_len] is 1, and by another token when it is 0.
// Hidden state for the first draft: the final-normed hidden of the last forward (prefill / synth / previous run).
extern "C" int rmi_engine_generate(rmi_engine* h, const rmi_gen_request* req, int* out_tokens, rmi_gen_stats* stats) {
    if (!h || !req || !out_tokens) return fail(RMI_ERR_POINTER, "rmi_engine_generate: null argument");
    Engine& e = h->e;
    e.stream_mode = -1;
    const int n_gen = req->n_gen;
    if (n_gen < 1 || n_gen >= kRingCap - 2) return fail(RMI_ERR_STATE, "rmi_engine_generate: bad n_gen");
    int st[kNumSlots];
    RMI_TRY(get_ints(e, st, kNumSlots));
    if (st[kPos] + n_gen + 2 >= e.max_ctx) return fail(RMI_ERR_STATE, "context full");
    const bool mtp = req->mode != RMI_GEN_GREEDY;
    if (req->mode == RMI_GEN_MTP_FORCED) {
        if (!req->ref_tokens || req->ref_len < 1 || !req->pattern || req->pattern_len < 1 || req->pattern_len > 4096)
            return fail(RMI_ERR_STATE, "rmi_engine_generate: forced mode needs ref_tokens and a pattern");
        // ref_tokens[i] is the token at position ref_base + i; lay it out by absolute position
        std::vector<int> byp(static_cast<size_t>(e.max_ctx) + 1, 0);
        for (int i = 0; i < req->ref_len; ++i) {
            const int p = req->ref_base + i;
            if (p >= 0 && p <= e.max_ctx) byp[p] = req->ref_tokens[i];
        }
        HIP_TRY(hipMemcpyAsync(e.ref_tok, byp.data(), sizeof(int) * byp.size(), hipMemcpyHostToDevice, e.s));
        HIP_TRY(hipMemcpyAsync(e.pattern, req->pattern, req->pattern_len, hipMemcpyHostToDevice, e.s));
        HIP_TRY(hipStreamSynchronize(e.s));
    }
    RMI_TRY(set_int(e, kMode, req->mode == RMI_GEN_MTP_FORCED ? 1 : 0));
    RMI_TRY(set_int(e, kPatLen, req->mode == RMI_GEN_MTP_FORCED ? req->pattern_len : 0));
    RMI_TRY(set_int(e, kNOut, 0));
    RMI_TRY(set_int(e, kRound, 0));
    RMI_TRY(set_int(e, kNAcc, 0));
    const bool graph = req->use_graph != 0;
    if (graph) {
        if (mtp) RMI_TRY(capture(e, &e.g_round, [&] { return verify_round(e); }));
        else RMI_TRY(capture(e, &e.g_single, [&] { return single_step(e); }));
    }
    HIP_TRY(hipStreamSynchronize(e.s));
    ExchangeGuard xg;
    RMI_TRY(xg.begin());
    HIP_TRY(hipEventRecord(e.ev0, e.s));
    if (mtp) RMI_TRY(first_draft(e));
    int emitted = 0, launched = 0;
    while (emitted < n_gen) {
        const int batch = mtp ? std::max(1, (n_gen - emitted + 1) / 2) : n_gen - emitted;
        for (int i = 0; i < batch; ++i) {
            if (graph) HIP_TRY(hipGraphLaunch(mtp ? e.g_round : e.g_single, e.s));
            else RMI_TRY(mtp ? verify_round(e) : single_step(e));
        }
        launched += batch;
        HIP_TRY(hipEventRecord(e.ev1, e.s));
        RMI_TRY(get_ints(e, st, kNumSlots));
        emitted = st[kNOut];
        if (launched > 4 * n_gen + 8) return fail(RMI_ERR_STATE, "rmi_engine_generate: no progress");
    }
    RMI_TRY(xg.end("rmi_engine_generate"));
    float ms = 0.0f;
    HIP_TRY(hipEventElapsedTime(&ms, e.ev0, e.ev1));
    std::vector<int> ring(static_cast<size_t>(emitted));
    HIP_TRY(hipMemcpy(ring.data(), e.ring, sizeof(int) * ring.size(), hipMemcpyDeviceToHost));
    std::memcpy(out_tokens, ring.data(), sizeof(int) * static_cast<size_t>(n_gen));
    if (stats) {
        stats->tokens = n_gen;
        stats->emitted = emitted;
        stats->rounds = mtp ? st[kRound] : launched;
        stats->accepted = st[kNAcc];
        stats->gpu_ms = ms;
    }
    return RMI_OK;
}

// Token-at-a-time generation for a serving loop (the reference's serve_loop, qw:2740-2808): gen_begin prepares the
// mode (the captured graph; for MTP the first draft candidate of the current token), then each gen_step runs one
// greedy forward (1 token: the greedy token after the current one, which it feeds) or one verify round (c0, and c1
// when the candidate was accepted) and returns the emitted tokens.
extern "C" int rmi_engine_gen_begin(rmi_engine* h, int mode) {
    if (!h) return fail(RMI_ERR_POINTER, "rmi_engine_gen_begin: null engine");
    Engine& e = h->e;
    if (mode != RMI_GEN_GREEDY && mode != RMI_GEN_MTP) return fail(RMI_ERR_STATE, "rmi_engine_gen_begin: bad mode");
    RMI_TRY(set_int(e, kMode, 0));
    RMI_TRY(set_int(e, kPatLen, 0));
    RMI_TRY(set_int(e, kNOut, 0));
    RMI_TRY(set_int(e, kRound, 0));
    RMI_TRY(set_int(e, kNAcc, 0));
    if (mode == RMI_GEN_MTP) {
        RMI_TRY(capture(e, &e.g_round, [&] { return verify_round(e); }));
        RMI_TRY(first_draft(e));
    } else {
        RMI_TRY(capture(e, &e.g_single, [&] { return single_step(e); }));
    }
    HIP_TRY(hipStreamSynchronize(e.s));
    e.stream_mode = mode;
    return RMI_OK;
}

extern "C" int rmi_engine_gen_step(rmi_engine* h, int* out_tokens, int* n_out) {
    if (!h || !out_tokens || !n_out) return fail(RMI_ERR_POINTER, "rmi_engine_gen_step: null argument");
    Engine& e = h->e;
    if (e.stream_mode < 0) return fail(RMI_ERR_STATE, "rmi_engine_gen_step: no rmi_engine_gen_begin since the context changed");
    int st[kNumSlots];
    RMI_TRY(get_ints(e, st, kNumSlots));
    if (st[kPos] + 3 >= e.max_ctx) return fail(RMI_ERR_STATE, "context full");
    const bool mtp = e.stream_mode == RMI_GEN_MTP;
    ExchangeGuard xg;
    RMI_TRY(xg.begin());
    HIP_TRY(hipGraphLaunch(mtp ? e.g_round : e.g_single, e.s));
    RMI_TRY(get_ints(e, st, kNumSlots));
    RMI_TRY(xg.end("rmi_engine_gen_step"));
    out_tokens[0] = st[kV0];
    *n_out = 1;
    if (mtp && st[kAccept]) {
        out_tokens[1] = st[kV1];
        *n_out = 2;
    }
    return RMI_OK;
}

// The k largest logits of column col of the last head pass (column 0: the last forward or ingest, before any draft of
// a gen_begin / gen_step overwrites it) with their ids, logit descending, lower id first among equal logits
// (topk_out, qw:2513-2531).
extern "C" int rmi_engine_topk(rmi_engine* h, int col, int k, int* ids, float* logits) {
    if (!h || !ids || !logits) return fail(RMI_ERR_POINTER, "rmi_engine_topk: null argument");
    Engine& e = h->e;
    const int n = e.cfg.n_vocab;
    if (col < 0 || col > 1) return fail(RMI_ERR_SHAPE, "rmi_engine_topk: column must be 0 or 1");
    if (k < 1 || k > 64 || k > n) return fail(RMI_ERR_SHAPE, "rmi_engine_topk: k must be 1..min(64, n_vocab)");
    RMI_TRY(rmi_topk(e.logits + static_cast<size_t>(col) * n, n, k, e.topk_out,
                     reinterpret_cast<float*>(e.topk_out + 64), e.topk_ws, e.s));
    int buf[128];
    HIP_TRY(hipMemcpyAsync(buf, e.topk_out, sizeof buf, hipMemcpyDeviceToHost, e.s));
    HIP_TRY(hipStreamSynchronize(e.s));
    std::memcpy(ids, buf, sizeof(int) * k);
    std::memcpy(logits, buf + 64, sizeof(float) * k);
    return RMI_OK;
}
