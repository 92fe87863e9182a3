// gdn.hip - Gated DeltaNet decode chain for gfx950 (reference src/fused_gdn.cu:40-133, engine glue
// src/qwythos.cpp:1101-1127 and the verify pass 1438-1478).
//
// Kernels, for 1 token (the plain decode step), the 2 verify tokens or an ingest chunk of up to 16 tokens (the engine
// path runs the conv inside the step kernel's prologue, one launch per layer; the reference surface keeps them apart):
//   conv:  one lane per channel (8192 = q 2048 | k 2048 | v 4096): causal width-4 conv over [hist(3) | x], SiLU, and
//          the L2 norm of each 128-channel q/k head.  History is updated in place; with 2 tokens the history after
//          token 0 also goes to the rollback buffer.
//   step:  one workgroup per value head (128 columns x 4 row groups, 512 lanes), the head's 128x128 fp32 state held
//          in registers (32 rows per lane) across both tokens.  Per token: decay g = exp(softplus(a + dt) * ssm_a),
//          beta = sigmoid(b) (both from the raw beta|alpha GEMV output), kv = S^T k, delta = (v - g kv) beta,
//          S = g S + k delta^T, o = S^T q / sqrt(128), y = o * rsqrt(mean(o^2) + eps) * gamma * silu(z), Q8_1 of y.
//          With 2 tokens the state after token 0 is written to the rollback buffer, the final state in place.
// State layout [128 rows (k index)][h_v][128 cols (v index)], cols fastest (fgdn:60-61).  Conv history [c][3],
// conv weights [c][4] (fgdn:113-133).
//
// Rollback by selector: each GDN layer owns two state buffers and two history buffers; `sel` (device int) names the
// live one.  A verify writes the after-token-0 state/history into the other buffer, so rejecting the draft is a flip
// of `sel` (no copy).  A single-token step updates the live buffers in place.
#include "rmi_common.h"

namespace rmi {
namespace {

constexpr int S = 128;
constexpr int RG = 4;
constexpr int RPG = S / RG;

template <typename T>
__device__ __forceinline__ T* pick(T* a, T* b, const int* sel) {
    return (sel != nullptr && *sel != 0) ? b : a;
}

// ---- conv + SiLU + L2 -------------------------------------------------------------------------------------------------
// 256 lanes per workgroup = two 128-channel heads.  x of token t at x + t * tok_stride, output likewise at h.
template <int NT>
__global__ __launch_bounds__(256) void gdn_conv_kernel(float* hist_a, float* hist_b, const int* sel,
                                                       const float* x, const float* __restrict__ w, float* h,
                                                       int tok_stride, int qk_heads, float eps) {
    __shared__ float part[NT][4];
    const int c = blockIdx.x * 256 + threadIdx.x;
    float* hist = pick(hist_a, hist_b, sel);
    float* snap = pick(hist_b, hist_a, sel);
    const float h0 = hist[3 * c], h1 = hist[3 * c + 1], h2 = hist[3 * c + 2];
    const float w0 = w[4 * c], w1 = w[4 * c + 1], w2 = w[4 * c + 2], w3 = w[4 * c + 3];
    const float x0 = x[c];
    float y[NT];
    y[0] = silu(__builtin_fmaf(x0, w3, __builtin_fmaf(h2, w2, __builtin_fmaf(h1, w1, h0 * w0))));
    float x1 = 0.0f;
    if constexpr (NT == 2) {
        x1 = x[tok_stride + c];
        y[1] = silu(__builtin_fmaf(x1, w3, __builtin_fmaf(x0, w2, __builtin_fmaf(h2, w1, h1 * w0))));
    }
    const int head = c / S;   // uniform per wave (a head is two waves)
    if (head < qk_heads) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float sq = group_sum<64>(y[t] * y[t]);
            if ((threadIdx.x & 63) == 0) part[t][threadIdx.x >> 6] = sq;
        }
    }
    __syncthreads();
    if (head < qk_heads) {
        const int pair = (threadIdx.x >> 7) * 2;   // the two waves of this lane's head
#pragma unroll
        for (int t = 0; t < NT; ++t) y[t] *= rsqrtf((part[t][pair] + part[t][pair + 1]) + eps);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) h[static_cast<size_t>(t) * tok_stride + c] = y[t];
    if constexpr (NT == 2) {
        snap[3 * c] = h1;
        snap[3 * c + 1] = h2;
        snap[3 * c + 2] = x0;
        hist[3 * c] = h2;
        hist[3 * c + 1] = x0;
        hist[3 * c + 2] = x1;
    } else {
        hist[3 * c] = h1;
        hist[3 * c + 1] = h2;
        hist[3 * c + 2] = x0;
    }
}

// ---- delta-rule step + RMSNorm * SiLU gate + Q8_1 ----------------------------------------------------------------------
struct StepArgs {
    float* state_a;
    float* state_b;
    const int* sel;
    const float* q;        // token t at + t * tok_stride; head qh at + qh * 128
    const float* k;
    const float* v;        // head h at + h * 128
    const float* z;
    int tok_stride;
    // gates: RAW = raw beta|alpha GEMV output (beta at ab[h], alpha at ab[h_v + h], token t at + t * ab_stride)
    const float* ab;
    int ab_stride;
    const float* dt;
    const float* ssm_a;
    // gates, prepared (the reference API): decay logit gate[h], beta[h] after the sigmoid
    const float* gate;
    const float* beta;
    const float* gamma;
    float eps;
    float* y;              // token t at + t * y_stride
    int y_stride;
    uint8_t* q8;           // token t at + t * q8_stride bytes (may be null)
    int q8_stride;
    int h_k, h_v;
    // CONV: the layer's conv + SiLU + L2 runs in the step kernel's prologue on the raw q|k|v rows (q, k, v above)
    float* hist_a;
    float* hist_b;
    const float* conv_w;
    int ntok;              // tokens of this launch (<= the instantiation's NT)
    unsigned long long* xch;   // the split kernel's exchange words, kXchWords per value head
};

// CONV (engine path): lanes 0..383 first run the conv of the head's q (k-head qh), k and v channels for all tokens
// with the arithmetic of gdn_conv_kernel (same 64-lane partition of each 128-channel L2 sum) and keep the results in
// LDS.  The history is per value head, [h_v][q 128 | k 128 | v 128][3]: the heads qh and qh + h_k that share a k-head
// each carry their own (identical) copy of its q/k history, so no workgroup writes what another reads.  The raw
// q|k|v rows are only read.
//
// NT is the largest token count of the instantiation and a.ntok (<= NT) the count of this launch.  NT = 2 is the
// verify pair: the state and history after token 0 also go to the rollback buffers.  Otherwise (1 token, or an ingest
// chunk of up to 16) the state and history are updated in place after the last token.  Every token's arithmetic is
// that of the single-token step in the same order, so a chunk leaves the bits the per-token steps leave.
// v[l] + v[l ^ 16], then that plus its value in lane l ^ 32: the sum over a column's four row groups, in every lane of
// the column.  gfx950's lane swaps (v_permlane16_swap / v_permlane32_swap: each returns a half's even / odd rows, or
// the two 32-lane halves, side by side) keep it on the VALU; the sums are those of the xor-16 / xor-32 butterfly
// (the two addends of each lane are the same, in either order).
__device__ __forceinline__ float sum_row_groups(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// a zero the compiler cannot see through: indexing a uniform address with it keeps the load on the vector path, in
// issue order with the kernel's other loads (a scalar load gets a wait of its own at the next branch)
__device__ __forceinline__ int opaque_zero() {
    int z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    return z;
}

// decay and beta of token t from the raw beta|alpha GEMV output (qw:707-715)
__device__ __forceinline__ void gate_values(float b_raw, float a_raw, float dt, float ssm_a, float& g, float& b) {
    b = 1.0f / (1.0f + expf(-b_raw));
    const float vv = a_raw + dt;
    g = expf((vv > 20.0f ? vv : log1pf(expf(vv))) * ssm_a);
}

template <int NT, bool RAW, bool CONV>
__global__ __launch_bounds__(S * RG) void gdn_step_kernel(StepArgs a) {
    constexpr bool SNAP = NT == 2;
    // the engine path (decode, verify, ingest chunks): the launch's loads go out in one batch led by the selector
    // (both history buffers read, one kept), so the state loads wait for one memory round trip, not three; the gates
    // are derived by the conv's idle lanes and published by the conv's own barrier
    constexpr bool FAST = CONV && RAW;
    __shared__ float cq[NT][S], ck[NT][S], cv[CONV ? NT : 1][S];   // q, k (and v) of every token
    __shared__ float cpart[NT][4];
    __shared__ float gbt[NT][2];                                    // decay, beta per token
    __shared__ float wsum[NT][S * RG / 64];                         // per-wave sums of o^2
    __shared__ float ybuf[NT][S];
    __shared__ float szb[NT][S];                                    // the output gate's SiLU per token and column
    const int ntok = NT <= 2 ? NT : a.ntok;
    const int head = blockIdx.x;
    // lane (wave w, lane l): column 16 w + l % 16, row group l / 16 (rows 32 rg .. 32 rg + 31): a column's four row
    // groups share a wave, so the S^T k and S^T q column sums are two xor shuffles, not LDS round trips
    const int wv = threadIdx.x >> 6, ln = threadIdx.x & 63;
    const int col = 16 * wv + (ln & 15);
    const int rg = ln >> 4;
    const int qh = head % a.h_k;
    const size_t row_stride = static_cast<size_t>(a.h_v) * S;
    const size_t base = (static_cast<size_t>(rg * RPG) * a.h_v + head) * S + col;
    const int kind = threadIdx.x >> 7;   // CONV prologue: 0 q, 1 k, 2 v, 3 idle
    const int j = threadIdx.x & (S - 1);

    // FAST: the selector is the launch's first load (the state addresses depend on it)
    int selv = 0;
    if constexpr (FAST) selv = a.sel[opaque_zero()];

    // everything that does not depend on the selector is loaded next, in flight with it: the raw q|k|v rows and conv
    // taps (CONV), z and gamma (the norm lanes), the gate inputs, and (FAST) both history buffers
    const float* src = kind == 0 ? a.q + qh * S : kind == 1 ? a.k + qh * S : a.v + head * S;
    const int c = kind == 0 ? qh * S + j : kind == 1 ? (a.h_k + qh) * S + j : (2 * a.h_k + head) * S + j;
    // every lane loads every token's row (clamped to the last token; kind 3 and row groups 1..3 load and discard):
    // a load under a per-token branch is issued where it is first used, one memory round trip per token
    float xr[NT], w0 = 0.0f, w1 = 0.0f, w2 = 0.0f, w3 = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; ++t) xr[t] = 0.0f;
    if constexpr (CONV) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float v = src[static_cast<size_t>(min(t, ntok - 1)) * a.tok_stride + j];
            xr[t] = t < ntok && kind < 3 ? v : 0.0f;
        }
        w0 = a.conv_w[4 * c];
        w1 = a.conv_w[4 * c + 1];
        w2 = a.conv_w[4 * c + 2];
        w3 = a.conv_w[4 * c + 3];
    }
    // the output gate: lane (column, row group rg) takes tokens RG i + rg, so a lane computes NT / RG SiLUs where the
    // row-group-0 lanes alone would take all NT (a wave runs every token's code either way)
    constexpr int ZT = (NT + RG - 1) / RG;
    float zq[ZT];
    const float gam = a.gamma[col];
#pragma unroll
    for (int i = 0; i < ZT; ++i) {
        const int t = RG * i + rg;
        const float v = a.z[static_cast<size_t>(min(t, ntok - 1)) * a.tok_stride + head * S + col];
        zq[i] = t < ntok ? v : 0.0f;
    }
    float gin[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    // gate lane of token gt: lanes 0.. (FAST: the conv's idle lanes 3 S ..)
    const int gt = FAST ? static_cast<int>(threadIdx.x) - 3 * S : static_cast<int>(threadIdx.x);
    if (gt >= 0 && gt < ntok) {
        if constexpr (RAW) {
            const float* ab = a.ab + static_cast<size_t>(gt) * a.ab_stride;
            gin[0] = ab[head];
            gin[1] = ab[a.h_v + head];
            gin[2] = a.dt[head];
            gin[3] = a.ssm_a[head];
        } else {
            gin[0] = a.beta[head];
            gin[1] = a.gate[head];
        }
    }
    // CONV history slot: this head's own copy of the channel (the idle lanes read the q slot and ignore it: no branch
    // around the loads, so the compiler's wait for them counts the state loads issued after)
    const int ch = (3 * head + (kind < 3 ? kind : 0)) * S + j;
    float hA[3] = {0.0f, 0.0f, 0.0f}, hB[3] = {0.0f, 0.0f, 0.0f};
    if constexpr (FAST) {
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            hA[i] = a.hist_a[3 * ch + i];
            hB[i] = a.hist_b[3 * ch + i];
        }
    }

    // the selector: read once (FAST: it arrived first); the other paths read it here, with the history behind
    // it and ahead of the state's 32 loads, so the conv (which needs only the history) does not wait for the state
    // (a wave's loads complete in issue order)
    const bool sel_b = FAST ? selv != 0 : (a.sel != nullptr && *a.sel != 0);
    float* state = sel_b ? a.state_b : a.state_a;
    float* snap = sel_b ? a.state_a : a.state_b;
    float* hist = sel_b ? a.hist_b : a.hist_a;
    float* hsnap = sel_b ? a.hist_a : a.hist_b;
    float h0 = 0.0f, h1 = 0.0f, h2 = 0.0f;
    if constexpr (FAST) {
        h0 = sel_b ? hB[0] : hA[0];
        h1 = sel_b ? hB[1] : hA[1];
        h2 = sel_b ? hB[2] : hA[2];
    } else if constexpr (CONV) {
        h0 = hist[3 * ch];
        h1 = hist[3 * ch + 1];
        h2 = hist[3 * ch + 2];
    }
    __builtin_amdgcn_sched_barrier(0);
    // The state is read once and written once per launch (2 MiB per layer, 4 MiB with the rollback copy):
    // nontemporal loads and stores keep it from filling the L2 that the end of the kernel writes back
    // (measured: 2447 -> 2376 us per 4K round over 24 layers).
    float s[RPG];
#pragma unroll
    for (int r = 0; r < RPG; ++r) s[r] = __builtin_nontemporal_load(state + base + r * row_stride);

    // FAST: the gate lanes publish each token's decay and beta with the conv's first barrier
    if constexpr (FAST) {
        if (gt >= 0 && gt < ntok) gate_values(gin[0], gin[1], gin[2], gin[3], gbt[gt][0], gbt[gt][1]);
    }

    if constexpr (CONV) {
        float y[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) y[t] = 0.0f;
        // the conv input sequence [h0 h1 h2 | x_0 .. x_ntok-1]; i is a compile-time index after unrolling
        auto seq = [&](int i) { return i == 0 ? h0 : i == 1 ? h1 : i == 2 ? h2 : xr[i - 3]; };
        if (kind < 3) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                if (t < ntok)
                    y[t] = silu(__builtin_fmaf(seq(t + 3), w3,
                                               __builtin_fmaf(seq(t + 2), w2, __builtin_fmaf(seq(t + 1), w1, seq(t) * w0))));
            }
        }
        if (kind < 2) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                if (t < ntok) {   // uniform
                    const float sqs = group_sum<64>(y[t] * y[t]);
                    if ((threadIdx.x & 63) == 0) cpart[t][threadIdx.x >> 6] = sqs;
                }
            }
        }
        __syncthreads();
        if (kind < 3) {
            if (kind < 2) {
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    if (t < ntok) y[t] *= rsqrtf((cpart[t][2 * kind] + cpart[t][2 * kind + 1]) + a.eps);
            }
#pragma unroll
            for (int t = 0; t < NT; ++t)
                if (t < ntok) (kind == 0 ? cq : kind == 1 ? ck : cv)[t][j] = y[t];
            if constexpr (SNAP) {
                hsnap[3 * ch] = h1;
                hsnap[3 * ch + 1] = h2;
                hsnap[3 * ch + 2] = xr[0];
                hist[3 * ch] = h2;
                hist[3 * ch + 1] = xr[0];
                hist[3 * ch + 2] = xr[1];
            } else {
                float n0 = 0.0f, n1 = 0.0f, n2 = 0.0f;   // the last three inputs
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    if (t == ntok - 1) {
                        n0 = seq(t + 1);
                        n1 = seq(t + 2);
                        n2 = seq(t + 3);
                    }
                }
                hist[3 * ch] = n0;
                hist[3 * ch + 1] = n1;
                hist[3 * ch + 2] = n2;
            }
        }
        if constexpr (FAST) __syncthreads();   // cq / ck / cv are read by other lanes at the top of the token loop
    }

    if constexpr (!CONV) {
        if (threadIdx.x < S) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                if (t >= ntok) break;
                ck[t][threadIdx.x] = a.k[static_cast<size_t>(t) * a.tok_stride + qh * S + threadIdx.x];
                cq[t][threadIdx.x] = a.q[static_cast<size_t>(t) * a.tok_stride + qh * S + threadIdx.x];
            }
        }
    }
    float vreg[NT];
    if constexpr (!CONV) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
            vreg[t] = t < ntok ? a.v[static_cast<size_t>(t) * a.tok_stride + head * S + col] : 0.0f;
    }
    if constexpr (!FAST) {
        // the gate lane of each token publishes its decay and beta (the barrier also publishes cq / ck / cv)
        if (gt < ntok) {
            float g, b;
            if constexpr (RAW) {
                gate_values(gin[0], gin[1], gin[2], gin[3], g, b);
            } else {
                b = gin[0];
                g = expf(gin[1]);
            }
            gbt[gt][0] = g;
            gbt[gt][1] = b;
        }
        __syncthreads();
    }

    // The recurrence runs through all tokens without a workgroup barrier: the output norm of token t (a sum over the
    // head's 128 columns, across waves) feeds only y, so each token's o and per-wave sum of squares are kept and the
    // norms are taken after the loop, with the same operations in the same order.
    // the output gate's SiLU does not depend on the recurrence: taken before it, read after the loop's barrier
#pragma unroll
    for (int i = 0; i < ZT; ++i) {
        const int t = RG * i + rg;
        if (t < NT) szb[t][col] = silu(zq[i]);
    }
    float occ[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) occ[t] = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        if (t < ntok) {   // uniform
            const float g = gbt[t][0], beta = gbt[t][1];
            float kv = 0.0f;
#pragma unroll
            for (int r = 0; r < RPG; ++r) kv = __builtin_fmaf(s[r], ck[t][rg * RPG + r], kv);
            kv = sum_row_groups(kv);   // (rg 0 + rg 1) + (rg 2 + rg 3), the same bits in all four lanes
            const float vcol = CONV ? cv[CONV ? t : 0][col] : vreg[t];
            const float delta = (vcol - g * kv) * beta;
            float o = 0.0f;
#pragma unroll
            for (int r = 0; r < RPG; ++r) {
                s[r] = __builtin_fmaf(g, s[r], ck[t][rg * RPG + r] * delta);
                o = __builtin_fmaf(s[r], cq[t][rg * RPG + r], o);
            }
            o = sum_row_groups(o);
            const float oc = o * 0.08838834764831845f;   // 1 / sqrt(128)
            if constexpr (SNAP) {
                if (t == 0) {
#pragma unroll
                    for (int r = 0; r < RPG; ++r) __builtin_nontemporal_store(s[r], snap + base + r * row_stride);
                }
            }
            const float ss = group_sum<16>(oc * oc);   // the wave's 16 columns (row-group 0 lanes carry them)
            if (ln == 0) wsum[t][wv] = ss;
            occ[t] = oc;
        }
    }
    __syncthreads();
    // every token's scale in every lane (no per-token divergent branch), the products on the row-group-0 lanes
    float scl[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        scl[t] = 0.0f;
        if (t < ntok) {   // uniform
            float tot = 0.0f;
#pragma unroll
            for (int w = 0; w < S * RG / 64; ++w) tot += wsum[t][w];
            scl[t] = rsqrtf(tot / static_cast<float>(S) + a.eps);
        }
    }
    if (rg == 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
            if (t < ntok) ybuf[t][col] = occ[t] * scl[t] * gam * szb[t][col];
    }
    __syncthreads();
    // y and its Q8_1 blocks: lane -> (token, column); 32-lane groups are whole blocks, and ntok * 128 is a multiple of
    // the wave size, so every pass has whole waves active
    for (int i = threadIdx.x; i < ntok * S; i += S * RG) {
        const int t = i / S, cc = i - t * S;
        const float yv = ybuf[t][cc];
        a.y[static_cast<size_t>(t) * a.y_stride + head * S + cc] = yv;
        if (a.q8) q8_1_store_lane(yv, a.q8 + static_cast<size_t>(t) * a.q8_stride + (head * 4 + (cc >> 5)) * kQ8_1Bytes);
    }
#pragma unroll
    for (int r = 0; r < RPG; ++r) __builtin_nontemporal_store(s[r], state + base + r * row_stride);
}

// ---- decode / verify step split over four workgroups per value head ---------------------------------------------------
// The engine's 1- and 2-token layer launch (conv + SiLU + L2, gates, delta-rule step, RMSNorm * SiLU gate, Q8_1) with
// each value head's 128 state columns cut into four parts of 32: workgroup (head, part) holds the part's 32 columns x
// 128 rows in two waves (lane: column 32 part + 16 w + l % 16, row group l / 16), so 128 CUs carry the state instead
// of 32 and each SIMD one wave instead of two.  Every per-lane operation, and every reduction order, is that of
// gdn_step_kernel (the column sums over row groups, the conv's 64-lane L2 partials, the output norm's sum of the eight
// 16-column wave sums in wave order), so the results are bitwise those of the one-workgroup kernel, which the ingest
// chunks run.  The part's 32 columns are one Q8_1 block per token.
// Each part recomputes the head's q and k conv (all 128 channels: the step reads all of them); part 0 writes their
// history once the exchange shows that every other part has used the history it loaded.  The output norm needs the head's eight wave sums: each part publishes its two per token as {bits, epoch}
// 8-byte words (agent scope: value and tag land together) and reads the other parts' words.  The epoch is the number
// of launches the head's parts have completed: every launch writes every part's words with the next one, so at the
// start of a launch all four parts' words carry the same tag, and a part reads it from its own word (which only it
// writes), waits for the other parts' words to carry tag + 1, and needs no reset.  The grid is part-major (workgroup
// part * h_v + head): workgroups go to the XCDs round robin, so with h_v a multiple of 8 the four parts of a head run
// on one XCD (with h_k one too, the heads that share its k-head, head % h_k: h and h + 16 at the 9B shapes) and read
// the head's q / k rows, conv taps and history through one L2 (a head-major grid put the parts on four XCDs: 7.28 ->
// 6.70 us per 2-token layer).  Every workgroup of the grid is resident at once (h_v * 4 workgroups of 128 lanes), so
// every wait ends (it is bounded all the same: gdn_exchange_timeouts).  The words live in a caller-owned buffer
// (rmi_gdn_exchange_bytes), zeroed once and used by one stream at a time: launches that overlap on one buffer race.
constexpr int kParts = 4;
constexpr int kPartCols = S / kParts;   // 32
constexpr int kPartLanes = kPartCols * RG;   // 128
constexpr int kXchWords = kParts * 2 * 2;   // per value head: [part][token][wave]
__device__ unsigned int gdn_xch_timeouts;
// The wait's bound (polls per wave) and a test switch that makes every wait miss until the bound: set from the host by
// rmi_gdn_exchange_test, so a test can drive the timeout path with every kernel still ending normally.
__device__ unsigned int gdn_xch_spin_limit = 1u << 20;
__device__ unsigned int gdn_xch_force_miss = 0;

template <int NT>
__global__ __launch_bounds__(kPartLanes) void gdn_split_kernel(StepArgs a) {
    static_assert(NT == 1 || NT == 2, "decode or verify");
    constexpr bool SNAP = NT == 2;
    __shared__ float cq[NT][S], ck[NT][S], cv[NT][kPartCols];
    __shared__ float cpart[NT][2][2];   // [token][q | k][wave]
    __shared__ float gbt[NT][2];
    __shared__ float wsum[NT][2];       // this part's two wave sums
    __shared__ float allw[NT][S * RG / 64];   // the head's eight wave sums, in wave order
    __shared__ float ybuf[NT][kPartCols];
    const int head = static_cast<int>(blockIdx.x) % a.h_v, part = static_cast<int>(blockIdx.x) / a.h_v;
    const int wv = threadIdx.x >> 6, ln = threadIdx.x & 63;
    const int lcol = 16 * wv + (ln & 15);
    const int col = kPartCols * part + lcol;
    const int rg = ln >> 4;
    const int qh = head % a.h_k;
    const size_t row_stride = static_cast<size_t>(a.h_v) * S;
    const size_t base = (static_cast<size_t>(rg * RPG) * a.h_v + head) * S + col;
    const int j = threadIdx.x;                   // q and k channel j of the k-head; lanes < 32: v of column 32 part + j
    const bool vlane = j < kPartCols;
    const int jv = kPartCols * part + (vlane ? j : 0);

    const int selv = a.sel[opaque_zero()];      // first: the state addresses depend on it
    // the exchange epoch of this launch: the tag of this part's own first word (written by no one else)
    unsigned long long* xh = a.xch + static_cast<size_t>(head) * kXchWords;
    const unsigned long long own0 = __hip_atomic_load(xh + part * 4, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned int spin_limit = gdn_xch_spin_limit;
    const bool force_miss = gdn_xch_force_miss != 0;
    float qx[NT], kx[NT], vx[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        qx[t] = a.q[static_cast<size_t>(t) * a.tok_stride + qh * S + j];
        kx[t] = a.k[static_cast<size_t>(t) * a.tok_stride + qh * S + j];
        vx[t] = a.v[static_cast<size_t>(t) * a.tok_stride + head * S + jv];
    }
    const int cqc = qh * S + j, ckc = (a.h_k + qh) * S + j, cvc = (2 * a.h_k + head) * S + jv;
    float wq[4], wk[4], wvv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        wq[i] = a.conv_w[4 * cqc + i];
        wk[i] = a.conv_w[4 * ckc + i];
        wvv[i] = a.conv_w[4 * cvc + i];
    }
    // z, gamma and the gate inputs are loaded by every lane (the same addresses in range for all of them) and used by
    // the lanes that own them: loads under a branch make the wait for the selector, at the join, cover every load
    // issued before the branch
    const float gam = a.gamma[col];
    float zz[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) zz[t] = a.z[static_cast<size_t>(t) * a.tok_stride + head * S + col];
    float gin[4];
    const int gt = static_cast<int>(threadIdx.x) - 64;   // gate lane of token gt: the second wave's first lanes
    {
        const float* ab = a.ab + static_cast<size_t>(min(max(gt, 0), NT - 1)) * a.ab_stride;
        gin[0] = ab[head];
        gin[1] = ab[a.h_v + head];
        gin[2] = a.dt[head];
        gin[3] = a.ssm_a[head];
    }
    // history slots of this value head's copy: q, k (channel j), v (column 32 part + j), both buffers
    const int chq = (3 * head) * S + j, chk = (3 * head + 1) * S + j, chv = (3 * head + 2) * S + jv;
    float hq[2][3], hk[2][3], hv[2][3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        hq[0][i] = a.hist_a[3 * chq + i];
        hq[1][i] = a.hist_b[3 * chq + i];
        hk[0][i] = a.hist_a[3 * chk + i];
        hk[1][i] = a.hist_b[3 * chk + i];
        hv[0][i] = a.hist_a[3 * chv + i];
        hv[1][i] = a.hist_b[3 * chv + i];
    }
    const bool sel_b = selv != 0;
    float* state = sel_b ? a.state_b : a.state_a;
    float* snap = sel_b ? a.state_a : a.state_b;
    float* hist = sel_b ? a.hist_b : a.hist_a;
    float* hsnap = sel_b ? a.hist_a : a.hist_b;
    const int sb = sel_b ? 1 : 0;
    __builtin_amdgcn_sched_barrier(0);
    float s[RPG];
#pragma unroll
    for (int r = 0; r < RPG; ++r) s[r] = __builtin_nontemporal_load(state + base + r * row_stride);

    if (gt >= 0 && gt < NT) gate_values(gin[0], gin[1], gin[2], gin[3], gbt[gt][0], gbt[gt][1]);

    // conv + SiLU over [h0 h1 h2 | x_0 .. x_NT-1] (gdn_step_kernel's arithmetic), L2 of q and k over 128 channels
    auto conv = [&](const float (&h)[3], const float (&x)[NT], const float (&w)[4], float (&y)[NT]) {
        auto seq = [&](int i) { return i < 3 ? h[i] : x[i - 3]; };
#pragma unroll
        for (int t = 0; t < NT; ++t)
            y[t] = silu(__builtin_fmaf(seq(t + 3), w[3],
                                       __builtin_fmaf(seq(t + 2), w[2], __builtin_fmaf(seq(t + 1), w[1], seq(t) * w[0]))));
    };
    float yq[NT], yk[NT], yv[NT];
    conv(hq[sb], qx, wq, yq);
    conv(hk[sb], kx, wk, yk);
    conv(hv[sb], vx, wvv, yv);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float sq = group_sum<64>(yq[t] * yq[t]);
        const float sk = group_sum<64>(yk[t] * yk[t]);
        if (ln == 0) {
            cpart[t][0][wv] = sq;
            cpart[t][1][wv] = sk;
        }
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        cq[t][j] = yq[t] * rsqrtf((cpart[t][0][0] + cpart[t][0][1]) + a.eps);
        ck[t][j] = yk[t] * rsqrtf((cpart[t][1][0] + cpart[t][1][1]) + a.eps);
        if (vlane) cv[t][j] = yv[t];
    }
    // history: part 0 keeps the head's q / k copies, every part its own v columns
    auto put_hist = [&](int ch, const float (&h)[3], const float (&x)[NT]) {
        if constexpr (SNAP) {
            hsnap[3 * ch] = h[1];
            hsnap[3 * ch + 1] = h[2];
            hsnap[3 * ch + 2] = x[0];
            hist[3 * ch] = h[2];
            hist[3 * ch + 1] = x[0];
            hist[3 * ch + 2] = x[NT - 1];
        } else {
            hist[3 * ch] = h[1];
            hist[3 * ch + 1] = h[2];
            hist[3 * ch + 2] = x[0];
        }
    };
    __syncthreads();

    // the output gate's SiLU is taken inside the exchange (below): wave 0 while its loads of the other parts' words are
    // in flight, wave 1 before it waits at the barrier.  Left to the compiler it sinks to its use after the exchange,
    // onto the launch's critical path.
    float sz[NT];
    auto gate_silu = [&]() {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            sz[t] = silu(zz[t]);
            asm volatile("" : "+v"(sz[t]));
        }
    };
    float occ[NT];
    float s0[SNAP ? RPG : 1];   // the state after token 0 (stored with the others after the exchange)
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float g = gbt[t][0], beta = gbt[t][1];
        float kv = 0.0f;
#pragma unroll
        for (int r = 0; r < RPG; ++r) kv = __builtin_fmaf(s[r], ck[t][rg * RPG + r], kv);
        kv = sum_row_groups(kv);
        const float delta = (cv[t][lcol] - g * kv) * beta;
        float o = 0.0f;
#pragma unroll
        for (int r = 0; r < RPG; ++r) {
            s[r] = __builtin_fmaf(g, s[r], ck[t][rg * RPG + r] * delta);
            o = __builtin_fmaf(s[r], cq[t][rg * RPG + r], o);
        }
        o = sum_row_groups(o);
        const float oc = o * 0.08838834764831845f;   // 1 / sqrt(128)
        if constexpr (SNAP) {
            if (t == 0) {
#pragma unroll
                for (int r = 0; r < RPG; ++r) s0[r] = s[r];
            }
        }
        const float ss = group_sum<16>(oc * oc);
        if (ln == 0) wsum[t][wv] = ss;
        occ[t] = oc;
    }
    __syncthreads();
    // Every global store of the launch (history, the state after token 0, the final state) is issued after the
    // exchange's loads: stores count in the wave's vector memory counter, so a load issued behind them waits for
    // their completion, a memory round trip.  The counter is per wave: wave 1, which makes no exchange loads, stores
    // (and publishes) at once.
    // The head's q / k history (part 0's stores) waits until the exchange has seen every other part's words at this
    // launch's tag: a part publishes only after its conv has consumed the history it loaded at the start, so a part
    // dispatched late still reads the history of the previous launch.  The other stores touch only the part's own
    // columns and go out at once.
    auto put_qk = [&]() {
        if (part == 0) {
            put_hist(chq, hq[sb], qx);
            put_hist(chk, hk[sb], kx);
        }
    };
    auto put_all = [&]() {
        if (vlane) put_hist(chv, hv[sb], vx);
        if constexpr (SNAP) {
#pragma unroll
            for (int r = 0; r < RPG; ++r) __builtin_nontemporal_store(s0[r], snap + base + r * row_stride);
        }
#pragma unroll
        for (int r = 0; r < RPG; ++r) __builtin_nontemporal_store(s[r], state + base + r * row_stride);
    };
    // the exchange: wave 1 publishes this part's wave sums and then stores, wave 0 gathers the other parts' (lane i:
    // part i / (2 NT), token (i / 2) % NT, wave i % 2) and then stores
    const unsigned long long tag = ((own0 >> 32) + 1ull) << 32;   // this launch's epoch
    if (wv == 1) {
        if (ln < 4) {   // both tokens' words (a 1-token launch writes token 1's words too, so all stay in step)
            const int tt = ln >> 1, ww = ln & 1;
            __hip_atomic_store(xh + (part * 2 + tt) * 2 + ww, tag | __float_as_uint(wsum[tt < NT ? tt : 0][ww]),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        put_all();
        gate_silu();
    }
    if (wv == 0) {
        const int pp = ln / (2 * NT), t = (ln >> 1) % NT, w = ln & 1;
        const bool other = ln < kParts * 2 * NT && pp != part;
        unsigned long long v = tag;
        if (other) v = __hip_atomic_load(xh + (pp * 2 + t) * 2 + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        gate_silu();
        unsigned int n = 0;
        bool arrived;
        while (!(arrived = __all(!other || ((v >> 32) == (tag >> 32) && !force_miss))) && n < spin_limit) {
            if (other && (v >> 32) != (tag >> 32))
                v = __hip_atomic_load(xh + (pp * 2 + t) * 2 + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ++n;
        }
        if (!arrived && ln == 0) atomicAdd(&gdn_xch_timeouts, 1u);
        if (ln < kParts * 2 * NT) allw[t][2 * pp + w] = other ? __uint_as_float(static_cast<uint32_t>(v)) : wsum[t][w];
        put_all();
    }
    __syncthreads();   // wave 0's wait has ended: every other part has published, so its history loads are done
    put_qk();
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        float tot = 0.0f;
#pragma unroll
        for (int w = 0; w < S * RG / 64; ++w) tot += allw[t][w];
        if (rg == 0) {
            const float scale = rsqrtf(tot / static_cast<float>(S) + a.eps);
            ybuf[t][lcol] = occ[t] * scale * gam * sz[t];
        }
    }
    __syncthreads();
    // y and the part's Q8_1 block per token: lanes 32 t + i (one 32-lane group per token)
    if (threadIdx.x < kPartCols * NT) {
        const int t = threadIdx.x / kPartCols, cc = threadIdx.x % kPartCols;
        const float yv2 = ybuf[t][cc];
        a.y[static_cast<size_t>(t) * a.y_stride + head * S + kPartCols * part + cc] = yv2;
        if (a.q8) q8_1_store_lane(yv2, a.q8 + static_cast<size_t>(t) * a.q8_stride + (head * 4 + part) * kQ8_1Bytes);
    }
}

}  // namespace
}  // namespace rmi

using namespace rmi;

// ---- reference surface ----------------------------------------------------------------------------------------------

extern "C" int rmi_fused_gdn_conv_l2(float* history, const float* qkv, const float* conv_w, float* h, int channels,
                                     int qk_heads, float eps, void* stream) {
    if (channels <= 0 || channels % 256 != 0 || qk_heads < 0 || qk_heads > channels / S)
        return fail(RMI_ERR_SHAPE, "fused_gdn_conv_l2: invalid arguments");
    if (!aligned4(history) || !aligned4(qkv) || !aligned4(conv_w) || !aligned4(h))
        return fail(RMI_ERR_POINTER, "fused_gdn_conv_l2: invalid arguments");
    hipLaunchKernelGGL(gdn_conv_kernel<1>, dim3(channels / 256), dim3(256), 0, static_cast<hipStream_t>(stream), history,
                       history, nullptr, qkv, conv_w, h, 0, qk_heads, eps);
    return launch_status("fused_gdn_conv_l2");
}

extern "C" int rmi_fused_gdn_step_norm_silu_q8(float* state, const float* q, const float* k, const float* v,
                                               const float* gate, const float* beta, const float* z,
                                               const float* gamma, float eps, float* y, uint8_t* q8, int h_k, int h_v,
                                               void* stream) {
    if (h_k <= 0 || h_v <= 0 || h_v % h_k) return fail(RMI_ERR_SHAPE, "fused_gdn_step_norm: invalid arguments");
    if (!aligned4(state) || !aligned4(q) || !aligned4(k) || !aligned4(v) || !aligned4(gate) || !aligned4(beta) ||
        !aligned4(z) || !aligned4(gamma) || !aligned4(y) || (q8 && (reinterpret_cast<uintptr_t>(q8) & 3u)))
        return fail(RMI_ERR_POINTER, "fused_gdn_step_norm: invalid arguments");
    StepArgs a{};
    a.state_a = a.state_b = state;
    a.q = q; a.k = k; a.v = v; a.z = z;
    a.gate = gate; a.beta = beta; a.gamma = gamma; a.eps = eps;
    a.y = y; a.q8 = q8; a.h_k = h_k; a.h_v = h_v;
    hipLaunchKernelGGL((gdn_step_kernel<1, false, false>), dim3(h_v), dim3(S * RG), 0, static_cast<hipStream_t>(stream), a);
    return launch_status("fused_gdn_step_norm_silu_q8");
}

// ---- engine surface: qkv|z and beta|alpha GEMV outputs, 1..16 tokens, selector-based rollback buffers --------------
// ntok = 2 is the verify pair (after-token-0 state and history to the non-live buffers); 1 and 3..16 update the live
// buffers in place (3..16: an ingest chunk, the row-batched step of src/qwythos_ingest.cu).  Per token t: qkvz + t * qkvz_stride holds [q h_k*128 | k h_k*128 | v h_v*128 | z h_v*128]; ab + t * ab_stride holds
// [beta h_v | alpha h_v] (both read only).  History per value head, [h_v][3 * 128][3].  Output y + t * y_stride, q8
// + t * q8_stride.
namespace {
int gdn_layer(float* state_a, float* state_b, float* hist_a, float* hist_b, const int* sel, float* qkvz,
              int qkvz_stride, const float* ab, int ab_stride, const float* conv_w, const float* dt, const float* ssm_a,
              const float* gamma, float eps, float* y, int y_stride, uint8_t* q8, int q8_stride, int h_k, int h_v,
              int ntok, void* xch, void* stream) {
    if (h_k <= 0 || h_v <= 0 || h_v % h_k || ntok < 1 || ntok > kMaxCols)
        return fail(RMI_ERR_SHAPE, "gdn_layer_tokens: invalid arguments");
    const int channels = 2 * h_k * S + h_v * S;
    if (channels % 256 != 0 || qkvz_stride < channels + h_v * S)
        return fail(RMI_ERR_SHAPE, "gdn_layer_tokens: invalid arguments");
    if (!aligned4(state_a) || !aligned4(state_b) || !aligned4(hist_a) || !aligned4(hist_b) || !aligned4(qkvz) ||
        !aligned4(ab) || !aligned4(conv_w) || !aligned4(dt) || !aligned4(ssm_a) || !aligned4(gamma) || !aligned4(y) ||
        !aligned4(sel))
        return fail(RMI_ERR_POINTER, "gdn_layer_tokens: invalid arguments");
    const auto s = static_cast<hipStream_t>(stream);
    StepArgs a{};
    a.state_a = state_a; a.state_b = state_b; a.sel = sel;
    a.q = qkvz; a.k = qkvz + h_k * S; a.v = qkvz + 2 * h_k * S; a.z = qkvz + channels;
    a.tok_stride = qkvz_stride;
    a.ab = ab; a.ab_stride = ab_stride; a.dt = dt; a.ssm_a = ssm_a;
    a.gamma = gamma; a.eps = eps;
    a.y = y; a.y_stride = y_stride; a.q8 = q8; a.q8_stride = q8_stride;
    a.h_k = h_k; a.h_v = h_v;
    a.hist_a = hist_a; a.hist_b = hist_b; a.conv_w = conv_w;
    a.ntok = ntok;
    a.xch = static_cast<unsigned long long*>(xch);
    if (ntok <= 2 && xch) {
        // decode / verify: four workgroups per value head (bitwise the one-workgroup kernel)
        if (ntok == 2) hipLaunchKernelGGL((gdn_split_kernel<2>), dim3(h_v * kParts), dim3(kPartLanes), 0, s, a);
        else hipLaunchKernelGGL((gdn_split_kernel<1>), dim3(h_v * kParts), dim3(kPartLanes), 0, s, a);
    } else if (ntok == 2) {
        hipLaunchKernelGGL((gdn_step_kernel<2, true, true>), dim3(h_v), dim3(S * RG), 0, s, a);
    } else if (ntok == 1) {
        hipLaunchKernelGGL((gdn_step_kernel<1, true, true>), dim3(h_v), dim3(S * RG), 0, s, a);
    } else {
        hipLaunchKernelGGL((gdn_step_kernel<kMaxCols, true, true>), dim3(h_v), dim3(S * RG), 0, s, a);
    }
    return launch_status("gdn_layer_tokens");
}
}  // namespace

extern "C" int rmi_gdn_layer_tokens(float* state_a, float* state_b, float* hist_a, float* hist_b, const int* sel,
                                    float* qkvz, int qkvz_stride, const float* ab, int ab_stride, const float* conv_w,
                                    const float* dt, const float* ssm_a, const float* gamma, float eps, float* y,
                                    int y_stride, uint8_t* q8, int q8_stride, int h_k, int h_v, int ntok,
                                    void* stream) {
    return gdn_layer(state_a, state_b, hist_a, hist_b, sel, qkvz, qkvz_stride, ab, ab_stride, conv_w, dt, ssm_a, gamma,
                     eps, y, y_stride, q8, q8_stride, h_k, h_v, ntok, nullptr, stream);
}

extern "C" size_t rmi_gdn_exchange_bytes(int h_v) {
    return h_v > 0 ? static_cast<size_t>(h_v) * kXchWords * sizeof(unsigned long long) : 0;
}

extern "C" int rmi_gdn_layer_tokens_x(float* state_a, float* state_b, float* hist_a, float* hist_b, const int* sel,
                                      float* qkvz, int qkvz_stride, const float* ab, int ab_stride,
                                      const float* conv_w, const float* dt, const float* ssm_a, const float* gamma,
                                      float eps, float* y, int y_stride, uint8_t* q8, int q8_stride, int h_k, int h_v,
                                      int ntok, void* xch, void* stream) {
    if (!xch || (reinterpret_cast<uintptr_t>(xch) & 7u))
        return fail(RMI_ERR_POINTER, "gdn_layer_tokens_x: null or misaligned exchange buffer");
    return gdn_layer(state_a, state_b, hist_a, hist_b, sel, qkvz, qkvz_stride, ab, ab_stride, conv_w, dt, ssm_a, gamma,
                     eps, y, y_stride, q8, q8_stride, h_k, h_v, ntok, xch, stream);
}

extern "C" int rmi_gdn_exchange_test(unsigned int spin_limit, int force_miss) {
    if (spin_limit == 0) spin_limit = 1u << 20;
    const unsigned int miss = force_miss ? 1u : 0u;
    if (hipMemcpyToSymbol(HIP_SYMBOL(gdn_xch_spin_limit), &spin_limit, sizeof(spin_limit)) != hipSuccess ||
        hipMemcpyToSymbol(HIP_SYMBOL(gdn_xch_force_miss), &miss, sizeof(miss)) != hipSuccess)
        return fail(RMI_ERR_LAUNCH, "rmi_gdn_exchange_test: cannot set the wait's bound");
    return RMI_OK;
}

extern "C" unsigned int rmi_gdn_exchange_timeouts(void) {
    unsigned int h = 0;
    if (hipMemcpyFromSymbol(&h, HIP_SYMBOL(gdn_xch_timeouts), sizeof(h)) != hipSuccess) return 0xffffffffu;
    return h;
}
