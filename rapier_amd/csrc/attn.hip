// attn.hip - GQA decode attention for gfx950 over an fp16 KV cache (reference src/qwythos.cpp: split_qg_kernel
// 320-327, store_kv2_kernel 340-345, gqa_head_kernel 384-442, sig_mul_quant_kernel 692-704, glue 1530-1558).
//
//   attn_prep   one workgroup per (token, head): q heads get the per-head RMSNorm (weights qn) and NEOX RoPE on the
//               first n_rot dims -> fp32 q buffer; k heads get RMSNorm (kn) + RoPE and v heads nothing, both stored
//               as fp16 at cache[pos_t][kv][d].  pos_t = pos[0] + t is read on the device.
//   partial     split-K flash decode.  Workgroup (chunk, kv head, slot group) covers positions [chunk * 64 * nsub,
//               +64 * nsub) for 8 query vectors (slots t * G + gh, group heads x tokens; up to 8 groups, so an ingest
//               chunk of 16 tokens is one launch); each of its 4 waves streams a quarter of the chunk independently:
//               QK^T and P V both on MFMA 16x16x16 f16 with the fp32 operand (q, p) split into fp16 hi + lo rows of
//               the same MFMA, online softmax per query.  Writes (m, l, o[256]) per query.  A slot's arithmetic does
//               not depend on which group or launch it is in (a wave step past a slot's last position leaves its
//               running state unchanged), so every query is bitwise its single-token result.
//   merge       one workgroup per (token, head): merges that query's chunks 0..pos_t / chunk in order, divides, gates
//               with sigmoid(g) and writes fp32 y plus Q8_1 for the wo GEMV.
// Query t sees positions <= pos[0] + t.  Chunk boundaries depend only on the query's position, so a verify column's
// result is bitwise the single-token result at the same position.
#include "rmi_common.h"
#include "rope.h"

#include <cmath>
#include <mutex>

namespace rmi {
namespace {

constexpr int HD = 256;
constexpr int SUB = 64;            // positions per chunk unit (4 waves x 16); a chunk is SUB * nsub positions
constexpr int REC = HD + 4;        // workspace record: m, l, pad, pad, o[256]
constexpr int SLOTS = 8;           // query vectors per kv head one partial workgroup handles (tokens x group heads)
constexpr int kMaxSlots = 64;      // query vectors per kv head one launch handles: SLOTS per slot group, grid.z groups

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }

__device__ __forceinline__ float block_sum256(float v, float* red) {
    v = group_sum<64>(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const float s = ((red[0] + red[1]) + red[2]) + red[3];
    __syncthreads();
    return s;
}

// ---- attn_prep -------------------------------------------------------------------------------------------------------
// RoPE: rope.h (NEOX pairs with the YaRN ramp; plain NEOX when yarn.on == 0).

// q3 per token: [n_head x (q HD | gate HD) | k n_kv*HD | v n_kv*HD] at q3 + t * q3_stride.
__global__ __launch_bounds__(HD) void attn_prep_kernel(const float* __restrict__ q3, int q3_stride,
                                                       const float* __restrict__ qn, const float* __restrict__ kn,
                                                       uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                                       const int* __restrict__ pos, float* __restrict__ qout,
                                                       int n_head, int n_kv, int n_rot, int max_ctx, float theta,
                                                       float eps, Yarn yarn) {
    __shared__ float red[4];
    __shared__ float xs[HD];
    const int t = blockIdx.x;
    const int hh = blockIdx.y;   // [0, n_head) q, [n_head, n_head + n_kv) k, then v
    const int d = threadIdx.x;
    const float* src = q3 + static_cast<size_t>(t) * q3_stride;
    // the row value does not depend on the position: load it in parallel with pos
    const bool is_v = hh >= n_head + n_kv, is_q = hh < n_head;
    float x = is_v ? src[2 * n_head * HD + n_kv * HD + (hh - n_head - n_kv) * HD + d]
                   : is_q ? src[hh * 2 * HD + d] : src[2 * n_head * HD + (hh - n_head) * HD + d];
    float wn = is_q ? qn[d] : kn[d];   // the norm weight too (unused for v): not a round trip after the sum
    const int p = pos[0] + t;
    // held here: the compiler would otherwise sink both loads below the position check, one round trip after it
    asm volatile("" : "+v"(x), "+v"(wn));
    // the rotary frequency of this lane's pair (fp64 pow, independent of the position) while the loads are in flight:
    // left in place it runs after the norm's last barrier, on the launch's critical path
    const int half = n_rot / 2;
    const int ri = d < half ? d : d - half;
    double freq = 0.0;
    if (!is_v && d < n_rot) freq = rope_freq(ri, n_rot, theta);
    asm volatile("" : "+v"(freq));
    if (p < 0 || p >= max_ctx) return;   // uniform: a position outside the cache stores nothing
    if (is_v) {   // v: straight to the cache
        const int kv = hh - n_head - n_kv;
        vc[(static_cast<size_t>(p) * n_kv + kv) * HD + d] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
        return;
    }
    const float ss = block_sum256(x * x, red);
    const float inv = rsqrtf(ss / static_cast<float>(HD) + eps);
    float v = x * inv * wn;
    xs[d] = v;
    __syncthreads();
    if (d < n_rot) {
        float c, s;
        rope_cos_sin_f(p, freq, ri, yarn, &c, &s);
        v = d < half ? rope_lo(xs[d], xs[d + half], c, s) : rope_hi(xs[d - half], xs[d], c, s);
    }
    if (is_q) {
        qout[(static_cast<size_t>(t) * n_head + hh) * HD + d] = v;
    } else {
        const int kv = hh - n_head;
        kc[(static_cast<size_t>(p) * n_kv + kv) * HD + d] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
    }
}

// ---- split-K partial ---------------------------------------------------------------------------------------------------
// Workgroup (chunk, kv head), 4 waves.  Wave w streams positions [chunk * 64 nsub + w * 16 nsub, +16 nsub) in steps of
// 16 on its own (no workgroup barrier inside the loop); the 4 waves' (m, l, o) are combined in wave order at the end
// into one record per query slot.  Query slot q = t * G + gh (token t, head kv * G + gh), q < 8.
//
// Both products run on v_mfma_f32_16x16x16f16 (lane l: l16 = l % 16, g4 = l / 16; A rows / B cols / D cols are l16,
// the k index of A and B is 4 g4 + 0..3, D rows are 4 g4 + 0..3):
//   scores  D[pos][n] = K[pos][:] . qcol_n, with qcol_n = fp16 hi part of slot n for n < 8 and the fp16 lo part of
//           slot n - 8 for n >= 8, so one MFMA chain yields both halves and s = D[pos][q] + D[pos][q + 8] carries
//           ~fp32 precision against the exact fp16 K.  K is loaded coalesced (two 512-byte rows per wave load),
//           staged through a padded LDS tile and read back in the A layout.
//   P V     D[m][n] = P'[m][pos] . V[pos][c(n)], with P' rows m < 8 = fp16 hi of p for slot m and rows m >= 8 = fp16
//           lo of p for slot m - 8.  The score lane (n, g4) already holds p for slot n % 8 at positions 4 g4 + r, which
//           is exactly the A layout.  V comes straight from coalesced 16-byte loads: lane (l16, g4) loads positions
//           4 g4 + j, dims 128 dg + 8 l16 + [0, 8); MFMA (dg, e) takes dim c = 128 dg + 8 l16 + e, so its B operand is
//           the e-th half of the four loads.  hi and lo rows are added once at the end (xor-32 lanes).
// Rows past the last position re-read the last row (finite data) and are masked to p = 0.
constexpr int STEP = 16;                 // positions per MFMA step
constexpr int WAVES = 4;
constexpr int KROW = 2 * HD + 16;        // bytes per staged K row: 16-byte pad puts consecutive rows 4 banks apart
constexpr int KTILE = STEP * KROW;       // 8448 bytes per wave; reused for the wave's o[8][256] (8192 bytes)

__device__ __forceinline__ void lds_wave_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
// K / V rows are streamed once per step: nontemporal loads, as the GEMVs stream their weights
__device__ __forceinline__ uint4 load_kv(const uint16_t* p) {
    const u32x4v v = __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(p));
    return make_uint4(v[0], v[1], v[2], v[3]);
}

typedef uint32_t u32x32 __attribute__((ext_vector_type(32)));

__device__ __forceinline__ void set_u4(u32x32& v, int j, uint4 w) {
    v[4 * j] = w.x;
    v[4 * j + 1] = w.y;
    v[4 * j + 2] = w.z;
    v[4 * j + 3] = w.w;
}
__device__ __forceinline__ uint4 get_u4(const u32x32& v, int j) {
    return make_uint4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
}

__device__ __forceinline__ uint32_t word_of(const uint4& v, int w) {
    return w == 0 ? v.x : w == 1 ? v.y : w == 2 ? v.z : v.w;
}

// attn_prep folded into the partial (decode and verify: one slot group).  pr.q3 is the GEMV output attn_prep reads;
// every workgroup norms and ropes its own query rows (attn_prep's reduction tree and rotation, so the same bits) into
// the query stage, and the workgroup whose chunk holds a new position writes that row's K (normed, roped) and V to the
// cache before it issues any K / V load (a workgroup barrier orders its stores before its waves' loads; no other
// workgroup reads the row).
struct PrepIn {
    const float* q3;   // per token: [n_head x (q HD | gate HD) | k n_kv HD | v n_kv HD]
    int q3_stride;
    const float* qn;
    const float* kn;
    uint16_t* kc;      // the caches, written
    uint16_t* vc;
    int n_rot;
    float theta, eps;
    Yarn yarn;
    // the rotation's (cos, sin) per token and pair, [2][n_rot / 2] float2 at positions pos[0] + t: kRopeOwn computes
    // them (no table), kRopeWrite computes them and workgroup 0 stores them, kRopeRead loads them with the launch's
    // first loads (every attention layer of one trunk pass rotates at the same positions: the first writes, the others
    // read the same bits, and the fp64 angle and sincos leave their critical paths)
    float2* cs;
    int cs_mode;
};
constexpr int kRopeOwn = 0, kRopeWrite = 1, kRopeRead = 2;

template <bool PREP>
__global__ __launch_bounds__(256, 2) void gqa_partial_kernel(const float* __restrict__ qbuf, const uint16_t* __restrict__ kc,
                                                          const uint16_t* __restrict__ vc, const int* __restrict__ pos,
                                                          float* __restrict__ ws, int slot_stride, int n_head,
                                                          int n_kv, int ntok, int nsub, int max_ctx, float scale,
                                                          PrepIn pr) {
    __shared__ __attribute__((aligned(16))) uint8_t tiles[WAVES * KTILE];
    __shared__ float wstat[WAVES][2][SLOTS];
    __shared__ float pred[PREP ? 2 : 1][WAVES];   // PREP: wave sums of the new K rows
    // the KV heads of one chunk are neighbouring workgroups (dispatched together), so the four 512-byte head rows of a
    // position are read close in time
    const int chunk = static_cast<int>(blockIdx.x) / n_kv, kv = static_cast<int>(blockIdx.x) - chunk * n_kv;
    const int s0 = SLOTS * static_cast<int>(blockIdx.z);
    const int G = n_head / n_kv;
    const int nq = ntok * G;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int l16 = lane & 15, g4 = lane >> 4;
    const int slot = s0 + (l16 & 7);   // query slot t * G + gh of this lane's MFMA column / row
    const bool lo_row = l16 >= 8;

    // The workgroup's 8 query rows (8 KB) are staged once in the K tile area: loaded by every wave (a row read per lane
    // by each wave would put 16 KB per wave of cache hits ahead of the K / V stream in the CU's memory pipeline).
    // They do not depend on the position: their loads go out together with pos[0].
    float4* qst = reinterpret_cast<float4*>(tiles);   // [slot within the group][64 float4]
    float4 qin[2];   // float4s tid and tid + 256 of the group's rows, written to the stage after the K / V loads issue
    const int d = static_cast<int>(threadIdx.x);   // PREP: this lane's dim of every query row and new K / V row
    // PREP query rows: wave w holds slots 2 w and 2 w + 1, lane l dims l + 64 k (k = 0..3) of each
    float xq[PREP ? 2 : 1][4], wq4[4], xk[PREP ? 2 : 1], xv[PREP ? 2 : 1], wk = 0.0f;
    double freq = 0.0, qfreq = 0.0;
    float2 kcs[2] = {make_float2(1.0f, 0.0f), make_float2(1.0f, 0.0f)}, qcs = make_float2(1.0f, 0.0f);   // kRopeRead
    if constexpr (PREP) {
        // raw rows, independent of the position: in flight together with pos
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int qs = min(s0 + 2 * wv + r, nq - 1), t = qs / G, gh = qs - t * G;
            const float* row = pr.q3 + static_cast<size_t>(t) * pr.q3_stride + (kv * G + gh) * 2 * HD;
#pragma unroll
            for (int k = 0; k < 4; ++k) xq[r][k] = row[lane + 64 * k];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) wq4[k] = pr.qn[lane + 64 * k];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const float* src = pr.q3 + static_cast<size_t>(min(t, ntok - 1)) * pr.q3_stride + 2 * n_head * HD;
            xk[t] = src[kv * HD + d];
            xv[t] = src[n_kv * HD + kv * HD + d];
        }
        wk = pr.kn[d];
        {
            // the table's entries, loaded unconditionally (a load under a branch gets a wait of its own, at the branch's
            // end): from the table in kRopeRead, else from qn (any 2 n_rot floats of valid memory; the values go unused)
            const int half = pr.n_rot / 2;
            const int kp = min(d < half ? d : d - half, half - 1), qp = min(lane < half ? lane : lane - half, half - 1);
            const int tq = min(s0 + 2 * wv, nq - 1) / G;
            const float2* tab = pr.cs_mode == kRopeRead ? pr.cs : reinterpret_cast<const float2*>(pr.qn);
#pragma unroll
            for (int t = 0; t < 2; ++t) kcs[t] = tab[min(t, ntok - 1) * half + kp];
            qcs = tab[tq * half + qp];
        }
        if (pr.cs_mode != kRopeRead) {
            if (d < pr.n_rot) freq = rope_freq(d < pr.n_rot / 2 ? d : d - pr.n_rot / 2, pr.n_rot, pr.theta);
            // the query rows' rotated dims: lane l of group 0 (n_rot = 64)
            if (lane < pr.n_rot) qfreq = rope_freq(lane < pr.n_rot / 2 ? lane : lane - pr.n_rot / 2, pr.n_rot, pr.theta);
            asm volatile("" : "+v"(freq), "+v"(qfreq));
        }
    } else {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int f = static_cast<int>(threadIdx.x) + 256 * i, qs = s0 + (f >> 6);
            const bool ok = qs < nq;
            const int t = ok ? qs / G : 0, gh = ok ? qs - (qs / G) * G : 0;
            const float4* q = reinterpret_cast<const float4*>(qbuf + (static_cast<size_t>(t) * n_head + kv * G + gh) * HD);
            const float4 v = q[f & 63];   // unconditional (a load under a branch gets a wait of its own)
            qin[i] = ok ? v : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    const int p0 = pos[0];
    const int p_last = p0 + (min(s0 + SLOTS, nq) - 1) / G;   // the last position this group's slots see
    const int wlen = STEP * nsub;
    const int cbase = chunk * WAVES * wlen;
    if (cbase > p_last || p0 < 0 || p_last >= max_ctx) return;   // uniform: no visible position (or a bad pos)
    // attn_prep's rotation of dim d (and d +- n_rot / 2) of a normed row staged in LDS (row) at position p (the angle
    // in fp64, as attn_prep)
    auto rope_row = [&](const float* row, float v, int p, int t) {
        if (d < pr.n_rot) {
            const int half = pr.n_rot / 2;
            float c, sn;
            if (pr.cs_mode == kRopeRead) {
                const float2 e = t == 0 ? kcs[0] : kcs[1];   // selected, not indexed (an indexed array goes to memory)
                c = e.x;
                sn = e.y;
            } else {
                rope_cos_sin_f(p, freq, d < half ? d : d - half, pr.yarn, &c, &sn);
            }
            v = d < half ? rope_lo(row[d], row[d + half], c, sn) : rope_hi(row[d - half], row[d], c, sn);
        }
        return v;
    };
    if constexpr (PREP) {
        // the new rows of this chunk (tokens t < ntok at p0 + t within [cbase, cbase + WAVES wlen)): K normed (the
        // norm tree of attn_prep: 64-lane butterfly per wave, then the four wave sums in order) and roped, V as is
        const int cend = cbase + WAVES * wlen;
        const int tfirst = max(0, cbase - p0), tlast = min(ntok, cend - p0);   // tokens [tfirst, tlast)
        if (tfirst < tlast) {   // uniform
            float* krow = reinterpret_cast<float*>(tiles);   // [2][HD] normed K rows
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const float sq = group_sum<64>(xk[t] * xk[t]);
                if ((d & 63) == 0) pred[t][d >> 6] = sq;
            }
            __syncthreads();
            float kvn[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const float ss = ((pred[t][0] + pred[t][1]) + pred[t][2]) + pred[t][3];
                kvn[t] = xk[t] * rsqrtf(ss / static_cast<float>(HD) + pr.eps) * wk;
                krow[t * HD + d] = kvn[t];
            }
            __syncthreads();
            for (int t = tfirst; t < tlast; ++t) {
                const int p = p0 + t;
                const float kr = rope_row(krow + t * HD, kvn[t], p, t);
                pr.kc[(static_cast<size_t>(p) * n_kv + kv) * HD + d] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(kr));
                pr.vc[(static_cast<size_t>(p) * n_kv + kv) * HD + d] =
                    __builtin_bit_cast(uint16_t, static_cast<_Float16>(t == 0 ? xv[0] : xv[1]));
            }
            __syncthreads();   // the rows are stored (workgroup scope) before any wave issues its K / V loads
        }
    }

    const int wbase = cbase + wv * wlen;
    const int nsteps = wbase > p_last ? 0 : min(nsub, (p_last - wbase) / STEP + 1);
    // the wave's own last row: the prefetch after its last step re-reads it instead of the next wave's rows (those
    // would be a second HBM pass over 1 / nsub of the cache)
    const int wlast = min(wbase + wlen - 1, p_last);
    uint8_t* kt = tiles + wv * KTILE;
    const int lim = slot < nq ? p0 + slot / G : -1;   // last position slot `slot` may see

    floatx4 oacc[2][8];
#pragma unroll
    for (int dg = 0; dg < 2; ++dg)
#pragma unroll
        for (int e = 0; e < 8; ++e) oacc[dg][e] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -INFINITY, l_run = 0.0f;   // of slot `slot` (same value in every lane of that slot)

    const size_t rstride = static_cast<size_t>(n_kv) * HD;   // halves between consecutive positions
    const uint16_t* kb = kc + static_cast<size_t>(kv) * HD;
    const uint16_t* vb = vc + static_cast<size_t>(kv) * HD;
    const int krow = lane >> 5, kcol = lane & 31;

    // rows are clamped to wlast <= p_last, so every load is in bounds (a wave with no step re-reads row p_last)
    u32x32 kreg;   // one vector value (an array carried across iterations would live in scratch)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int p = min(wbase + 2 * j + krow, wlast);
        set_u4(kreg, j, load_kv(kb + p * rstride + kcol * 8));
    }
    // V of a step: [2 j + dg] = position sb + 4 g4 + j, dims 128 dg + 8 l16 + [0, 8); also one step ahead
    u32x32 vnext;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint16_t* vr = vb + min(wbase + 4 * g4 + j, wlast) * rstride + 8 * l16;
        set_u4(vnext, 2 * j, load_kv(vr));
        set_u4(vnext, 2 * j + 1, load_kv(vr + 128));
    }
    // the new rows' inputs and the table's K entries stay live until the K / V loads are out: reusing their registers
    // for the K / V addresses made those loads wait for every load of the prologue
    if constexpr (PREP)
        asm volatile("" ::"v"(xk[0]), "v"(xk[1]), "v"(xv[0]), "v"(xv[1]), "v"(wk), "v"(kcs[0]), "v"(kcs[1]));
    // B operand of the score MFMAs, from the staged query rows: step 2 sp + hlf covers dims
    // 32 sp + 8 g4 + 4 hlf + [0, 4); rows 0-7 the fp16 hi part, rows 8-15 the fp16 lo part of the same slot
    if constexpr (PREP) {
        // the wave's two query rows: attn_prep's norm (the four 64-lane butterflies of a row, summed in order), weights,
        // then its rotation (n_rot 64: dims l and l +- 32 of group 0 meet by one lane exchange), into the stage
        float* qf = reinterpret_cast<float*>(tiles);   // [slot][HD]
        const int tq = min(s0 + 2 * wv, nq - 1) / G;    // both rows' token (G >= 2)
        float qc = 1.0f, qs = 0.0f;
        if (pr.cs_mode == kRopeRead) {
            qc = qcs.x;
            qs = qcs.y;
        } else if (lane < pr.n_rot) {
            rope_cos_sin_f(p0 + tq, qfreq, lane < pr.n_rot / 2 ? lane : lane - pr.n_rot / 2, pr.yarn, &qc, &qs);
            // the table of the launches that follow: workgroup 0's waves, each its rows' token (tokens 0 and 1 from
            // waves 0 and 2 at two tokens; equal values from the others)
            if (pr.cs_mode == kRopeWrite && blockIdx.x == 0 && lane < pr.n_rot / 2)
                pr.cs[tq * (pr.n_rot / 2) + lane] = make_float2(qc, qs);
        }
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            // lane 0's butterfly result, as attn_prep takes it: with the square contracted into the first step's add
            // (fma(x, x, partner^2)) the lanes of a wave do not all end with the same sum
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                ss += __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(group_sum<64>(xq[r][k] * xq[r][k]))));
            const float inv = rsqrtf(ss / static_cast<float>(HD) + pr.eps);
            float v[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) v[k] = xq[r][k] * inv * wq4[k];
            const float other = xor_lane<32>(v[0]);
            if (lane < pr.n_rot) v[0] = lane < pr.n_rot / 2 ? rope_lo(v[0], other, qc, qs) : rope_hi(other, v[0], qc, qs);
            const bool live = s0 + 2 * wv + r < nq;
#pragma unroll
            for (int k = 0; k < 4; ++k) qf[(2 * wv + r) * HD + lane + 64 * k] = live ? v[k] : 0.0f;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 2; ++i) qst[static_cast<int>(threadIdx.x) + 256 * i] = qin[i];
    }
    __syncthreads();   // the staged rows are complete
    half4 qb[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float4 qr = qst[(l16 & 7) * 64 + 8 * (i >> 1) + 2 * g4 + (i & 1)];
        const float xs[4] = {qr.x, qr.y, qr.z, qr.w};
        half4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const _Float16 h = static_cast<_Float16>(xs[e]);
            v[e] = lo_row ? static_cast<_Float16>(xs[e] - static_cast<float>(h)) : h;
        }
        qb[i] = v;
    }
    __syncthreads();   // every wave has its query rows: the K tiles may overwrite the stage
    for (int s = 0; s < nsteps; ++s) {
        const int sb = wbase + s * STEP;
        uint4 vreg[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) vreg[j] = get_u4(vnext, j);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint16_t* vr = vb + min(sb + STEP + 4 * g4 + j, wlast) * rstride + 8 * l16;
            set_u4(vnext, 2 * j, load_kv(vr));
            set_u4(vnext, 2 * j + 1, load_kv(vr + 128));
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) *reinterpret_cast<uint4*>(kt + (2 * j + krow) * KROW + kcol * 16) = get_u4(kreg, j);
        // next step's K is in flight during this step's math (after the last step: row wlast again, a cache hit)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int p = min(sb + STEP + 2 * j + krow, wlast);
            set_u4(kreg, j, load_kv(kb + p * rstride + kcol * 8));
        }
        lds_wave_sync();
        floatx4 sacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int sp = 0; sp < 8; ++sp) {
            const uint4 kw = *reinterpret_cast<const uint4*>(kt + l16 * KROW + 64 * sp + 16 * g4);
            const half4 k0 = __builtin_bit_cast(half4, make_uint2(kw.x, kw.y));
            const half4 k1 = __builtin_bit_cast(half4, make_uint2(kw.z, kw.w));
            sacc = __builtin_amdgcn_mfma_f32_16x16x16f16(k0, qb[2 * sp], sacc, 0, 0, 0);
            sacc = __builtin_amdgcn_mfma_f32_16x16x16f16(k1, qb[2 * sp + 1], sacc, 0, 0, 0);
        }
        // lane (l16, g4): s for slot l16 % 8 at positions sb + 4 g4 + r
        float sc[4];
        float mloc = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float v = sacc[r] + xor_lane<8>(sacc[r]);
            sc[r] = sb + 4 * g4 + r <= lim ? v * scale : -INFINITY;
            mloc = fmaxf(mloc, sc[r]);
        }
        mloc = fmaxf(mloc, xor_lane<16>(mloc));
        mloc = fmaxf(mloc, xor_lane<32>(mloc));
        const float m_new = fmaxf(m_run, mloc);
        const float m_ref = m_new == -INFINITY ? 0.0f : m_new;   // nothing visible yet: exp(-inf) = 0, no NaN
        const float alpha = m_run == m_new ? 1.0f : expf(m_run - m_ref);
        float pr[4], lsum = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            pr[r] = expf(sc[r] - m_ref);
            lsum += pr[r];
        }
        lsum += xor_lane<16>(lsum);
        lsum += xor_lane<32>(lsum);
        l_run = l_run * alpha + lsum;
        m_run = m_new;
        if (__ballot(alpha != 1.0f)) {   // wave-uniform: some slot's running max moved
            float a[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) a[r] = __shfl(alpha, 4 * (g4 & 1) + r, 64);
#pragma unroll
            for (int dg = 0; dg < 2; ++dg)
#pragma unroll
                for (int e = 0; e < 8; ++e)
#pragma unroll
                    for (int r = 0; r < 4; ++r) oacc[dg][e][r] *= a[r];
        }
        half4 pa;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const _Float16 h = static_cast<_Float16>(pr[r]);
            pa[r] = lo_row ? static_cast<_Float16>(pr[r] - static_cast<float>(h)) : h;
        }
#pragma unroll
        for (int dg = 0; dg < 2; ++dg) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const uint32_t x0 = word_of(vreg[dg], w), x1 = word_of(vreg[2 + dg], w);
                const uint32_t x2 = word_of(vreg[4 + dg], w), x3 = word_of(vreg[6 + dg], w);
                const half4 b_even = __builtin_bit_cast(
                    half4, make_uint2((x0 & 0xffffu) | (x1 << 16), (x2 & 0xffffu) | (x3 << 16)));
                const half4 b_odd = __builtin_bit_cast(
                    half4, make_uint2((x0 >> 16) | (x1 & 0xffff0000u), (x2 >> 16) | (x3 & 0xffff0000u)));
                oacc[dg][2 * w] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, b_even, oacc[dg][2 * w], 0, 0, 0);
                oacc[dg][2 * w + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, b_odd, oacc[dg][2 * w + 1], 0, 0, 0);
            }
        }
    }
    // A use of the first step's K / V rows on the path that runs no step: with their only uses inside the loop the
    // compiler sinks the loads into its preheader, behind the wait for the query rows, and no K / V load would go out
    // before the queries arrive.
    if (nsteps == 0) {
        uint32_t x = 0;
#pragma unroll
        for (int j = 0; j < 32; ++j) x ^= kreg[j] ^ vnext[j];
        asm volatile("" ::"v"(x));
    }
    // hi rows + lo rows: lanes g4 < 2 end with o[slot 4 g4 + r][128 dg + 8 l16 + e]
#pragma unroll
    for (int dg = 0; dg < 2; ++dg)
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
            for (int r = 0; r < 4; ++r) oacc[dg][e][r] += xor_lane<32>(oacc[dg][e][r]);

    __syncthreads();   // every wave is done with its K tile: reuse it for the wave's o
    float* ob = reinterpret_cast<float*>(kt);
    if (g4 < 2) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int dg = 0; dg < 2; ++dg) {
                float4* dst = reinterpret_cast<float4*>(ob + (4 * g4 + r) * HD + 128 * dg + 8 * l16);
                dst[0] = make_float4(oacc[dg][0][r], oacc[dg][1][r], oacc[dg][2][r], oacc[dg][3][r]);
                dst[1] = make_float4(oacc[dg][4][r], oacc[dg][5][r], oacc[dg][6][r], oacc[dg][7][r]);
            }
    }
    if (g4 == 0 && l16 < SLOTS) {
        wstat[wv][0][l16] = m_run;
        wstat[wv][1][l16] = l_run;
    }   // indexed by the slot within the group
    __syncthreads();
    // thread: slot q = tid / 32, dims 8 (tid % 32) + [0, 8); waves combined in order 0..3
    const int q = threadIdx.x >> 5, d0 = 8 * (threadIdx.x & 31);
    if (s0 + q < nq) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) M = fmaxf(M, wstat[w][0][q]);
        const float M_ref = M == -INFINITY ? 0.0f : M;
        float wt[WAVES], L = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            wt[w] = expf(wstat[w][0][q] - M_ref);
            L = __builtin_fmaf(wstat[w][1][q], wt[w], L);
        }
        float o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            const float* src = reinterpret_cast<const float*>(tiles + w * KTILE) + q * HD + d0;
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = __builtin_fmaf(wt[w], src[i], o[i]);
        }
        float* rec = ws + ((static_cast<size_t>(chunk) * n_kv + kv) * slot_stride + s0 + q) * REC;
        reinterpret_cast<float4*>(rec + 4 + d0)[0] = make_float4(o[0], o[1], o[2], o[3]);
        reinterpret_cast<float4*>(rec + 4 + d0)[1] = make_float4(o[4], o[5], o[6], o[7]);
        if ((threadIdx.x & 31) == 0) {
            rec[0] = M;
            rec[1] = L;
        }
    }
}

// ---- merge + sigmoid gate + Q8_1 ---------------------------------------------------------------------------------------
// Workgroup (token, head, quarter) owns 64 of the head's 256 output dims.  (1) the 256 lanes load every chunk's (m, l)
// in parallel, M = max m, weights w_c = exp(m_c - M) to LDS, L = sum l_c w_c (lane-strided partial sums, butterfly,
// waves in order); (2) wave g sums O_g = sum w_c o_c[d] over the chunks c = g mod 4 in ascending order, every load of
// a batch of 16 issued before the first is used, and O = ((O_0 + O_1) + O_2) + O_3.  The order depends only on the
// chunk count, so a verify column is bitwise its single-query launch.  Four workgroups per head put the record reads
// (1 KB per chunk and query) on 4x the CUs with every load of a lane in flight at once: at 64K (129 chunks) the
// previous form, one workgroup per head walking the chunks 8 loads ahead, was a chain of 16 dependent reads.
constexpr int kMaxChunks = 2048;
constexpr int kMergeParts = 4;                 // workgroups per (token, head)
constexpr int kMergeDims = HD / kMergeParts;   // 64 dims each: two Q8_1 blocks
constexpr int kMergeBatch = 16;                // record loads in flight per lane

__global__ __launch_bounds__(HD) void gqa_merge_kernel(const float* __restrict__ ws, int slot_stride,
                                                       const float* __restrict__ gsrc, int gstride,
                                                       const int* __restrict__ pos, float* __restrict__ y,
                                                       int y_stride, uint8_t* __restrict__ q8, int q8_stride,
                                                       int n_head, int n_kv, int chunk_len) {
    __shared__ float wts[kMaxChunks];
    __shared__ float red[4];
    __shared__ float opart[4][kMergeDims];
    const int t = blockIdx.x, h = blockIdx.y, part = blockIdx.z, tid = threadIdx.x;
    const int lane = tid & 63, grp = tid >> 6;
    const int d = kMergeDims * part + lane;   // this lane's output dim
    const int G = n_head / n_kv;
    const int kv = h / G, qv = t * G + (h - kv * G);
    const float g = gsrc[static_cast<size_t>(t) * gstride + h * 2 * HD + HD + d];   // in flight with pos
    const int nchunk = min((pos[0] + t) / chunk_len + 1, kMaxChunks);
    const size_t cstride = static_cast<size_t>(n_kv) * slot_stride * REC;
    const float* base = ws + (static_cast<size_t>(kv) * slot_stride + qv) * REC;
    // in flight together before the first barrier: the lane's first (m, l) record and its group's first o values
    float m0 = 0.0f, l0 = 0.0f;
    if (tid < nchunk) {
        m0 = base[tid * cstride];
        l0 = base[tid * cstride + 1];
    }
    float oa[kMergeBatch];   // chunks grp + 4 k, clamped (unconditional: a load under a branch gets a wait of its own)
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) oa[k] = base[min(grp + 4 * k, nchunk - 1) * cstride + 4 + d];
    float mloc = -INFINITY;
    if (tid < nchunk) mloc = fmaxf(mloc, m0);
    for (int c = tid + HD; c < nchunk; c += HD) mloc = fmaxf(mloc, base[c * cstride]);
    mloc = group_max<64>(mloc);
    if ((tid & 63) == 0) red[tid >> 6] = mloc;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float lloc = 0.0f;
    if (tid < nchunk) {
        const float w = expf(m0 - M);
        wts[tid] = w;
        lloc = __builtin_fmaf(l0, w, lloc);
    }
    for (int c = tid + HD; c < nchunk; c += HD) {
        const float w = expf(base[c * cstride] - M);
        wts[c] = w;
        lloc = __builtin_fmaf(base[c * cstride + 1], w, lloc);
    }
    const float L = block_sum256(lloc, red);   // includes the barrier that publishes wts
    // O_grp over chunks grp, grp + 4, ... in ascending order, a batch of 16 loads in flight while the previous is summed
    float O = 0.0f;
    for (int c0 = 0; 4 * c0 < nchunk; c0 += kMergeBatch) {
        const bool more = 4 * (c0 + kMergeBatch) < nchunk;
        float nx[kMergeBatch];
        if (more) {
#pragma unroll
            for (int k = 0; k < kMergeBatch; ++k)
                nx[k] = base[min(grp + 4 * (c0 + kMergeBatch + k), nchunk - 1) * cstride + 4 + d];
        }
#pragma unroll
        for (int k = 0; k < kMergeBatch; ++k) {
            const int c = grp + 4 * (c0 + k);
            if (c < nchunk) O = __builtin_fmaf(wts[c], oa[k], O);
        }
        if (more) {
#pragma unroll
            for (int k = 0; k < kMergeBatch; ++k) oa[k] = nx[k];
        }
    }
    opart[grp][lane] = O;
    __syncthreads();
    if (grp != 0) return;
    const float o = ((opart[0][lane] + opart[1][lane]) + opart[2][lane]) + opart[3][lane];
    const float v = (o / L) * sigmoid(g);
    if (y) y[static_cast<size_t>(t) * y_stride + h * HD + d] = v;
    if (q8) q8_1_store_lane(v, q8 + static_cast<size_t>(t) * q8_stride + (h * (HD / 32) + d / 32) * kQ8_1Bytes);
}

}  // namespace
}  // namespace rmi

using namespace rmi;

extern "C" int rmi_attn_prep_rope(const float* q3, int q3_stride, const float* qn, const float* kn,
                                  uint16_t* kcache, uint16_t* vcache, const int* pos, float* qout, int n_head,
                                  int n_kv, int head_dim, int n_rot, const rmi_rope_params* rope, float eps, int ntok,
                                  int max_ctx, void* stream) {
    if (head_dim != HD || n_head <= 0 || n_kv <= 0 || n_head % n_kv || n_rot < 0 || n_rot > HD || n_rot % 2 ||
        ntok < 1 || ntok > kMaxCols || !rope || !(rope->freq_base > 1.0f))
        return fail(RMI_ERR_SHAPE, "attn_prep: invalid arguments");
    if (!aligned4(q3) || !aligned4(qn) || !aligned4(kn) || !kcache || !vcache || !aligned4(pos) || !aligned4(qout))
        return fail(RMI_ERR_POINTER, "attn_prep: invalid arguments");
    Yarn y{};
    if (!yarn_setup(*rope, n_rot, &y)) return fail(RMI_ERR_SHAPE, "attn_prep: invalid YaRN parameters");
    hipLaunchKernelGGL(attn_prep_kernel, dim3(ntok, n_head + 2 * n_kv), dim3(HD), 0, static_cast<hipStream_t>(stream),
                       q3, q3_stride, qn, kn, kcache, vcache, pos, qout, n_head, n_kv, n_rot, max_ctx, rope->freq_base,
                       eps, y);
    return launch_status("attn_prep");
}

extern "C" int rmi_attn_prep(const float* q3, int q3_stride, const float* qn, const float* kn, uint16_t* kcache,
                             uint16_t* vcache, const int* pos, float* qout, int n_head, int n_kv, int head_dim,
                             int n_rot, float theta, float eps, int ntok, int max_ctx, void* stream) {
    const rmi_rope_params rope{theta, 1.0f, 0.0f, 1.0f, 1.0f, 32.0f, 1.0f};
    return rmi_attn_prep_rope(q3, q3_stride, qn, kn, kcache, vcache, pos, qout, n_head, n_kv, head_dim, n_rot, &rope,
                              eps, ntok, max_ctx, stream);
}

extern "C" size_t rmi_gqa_workspace_bytes(int max_ctx, int n_kv, int nsub) {
    if (max_ctx <= 0 || n_kv <= 0 || nsub <= 0) return 0;
    const int chunk_len = SUB * nsub;
    const size_t nchunks = static_cast<size_t>((max_ctx + chunk_len - 1) / chunk_len);
    return nchunks * static_cast<size_t>(n_kv) * kMaxSlots * REC * sizeof(float);
}

namespace rmi {
namespace {

// Workspace records: [chunk][kv head][slot_stride][REC] floats.  Every record the merge reads (chunks 0 .. pos_t /
// chunk_len of its query) is written by the partial launch of the same call, so nothing needs to start at zero.
int flash_decode(const float* q, const uint16_t* kcache, const uint16_t* vcache, const int* pos, const float* gate_src,
                 int gate_stride, float* y, int y_stride, uint8_t* q8, int q8_stride, float* ws, int slot_stride,
                 int n_head, int n_kv, int ntok, int nchunks, int nsub, int max_ctx, float scale, hipStream_t s) {
    const int groups = (ntok * (n_head / n_kv) + SLOTS - 1) / SLOTS;
    hipLaunchKernelGGL(gqa_partial_kernel<false>, dim3(nchunks * n_kv, 1, groups), dim3(256), 0, s, q, kcache, vcache, pos,
                       ws, slot_stride, n_head, n_kv, ntok, nsub, max_ctx, scale, PrepIn{});
    hipLaunchKernelGGL(gqa_merge_kernel, dim3(ntok, n_head, kMergeParts), dim3(HD), 0, s, ws, slot_stride, gate_src, gate_stride,
                       pos, y, y_stride, q8, q8_stride, n_head, n_kv, SUB * nsub);
    return launch_status("gqa_flash_decode");
}

int flash_decode_check(const float* q, const uint16_t* kcache, const uint16_t* vcache, const int* pos,
                       const float* gate_src, float* y, uint8_t* q8, int n_head, int n_kv, int head_dim, int ntok,
                       int max_ctx, int nsub, int* nchunks) {
    if (head_dim != HD || n_head <= 0 || n_kv <= 0 || n_head % n_kv || ntok < 1 || ntok * (n_head / n_kv) > kMaxSlots ||
        max_ctx <= 0 || max_ctx % SUB || nsub <= 0)
        return fail(RMI_ERR_SHAPE, "gqa_flash_decode: invalid arguments");
    if (!aligned16(q) || !aligned16(kcache) || !aligned16(vcache) || !aligned4(pos) || !aligned4(gate_src) ||
        (!y && !q8))
        return fail(RMI_ERR_POINTER, "gqa_flash_decode: invalid arguments");
    const int chunk_len = SUB * nsub;
    *nchunks = (max_ctx + chunk_len - 1) / chunk_len;
    if (*nchunks > kMaxChunks) return fail(RMI_ERR_SHAPE, "gqa_flash_decode: max_ctx / (64 * nsub) exceeds 2048 chunks");
    return RMI_OK;
}

// ---- the allocation-free variant's scratch ----------------------------------------------------------------------------
// One array per GPU, in the library's code object, held until the process ends.  In host code `scratch` names a
// host-side stand-in, not the device array: its device address comes from hipGetSymbolAddress, once per device with
// that device current, and only that address reaches a kernel.
constexpr size_t kScratchBytes = size_t(16) << 20;
constexpr int kMaxDevices = 64;
__device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

// the device address of `scratch` on the device that owns `stream` (the current device for the null stream)
int scratch_address(hipStream_t stream, float** out) {
    int dev = -1, cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return fail(RMI_ERR_LAUNCH, "gqa_flash_decode_noalloc: no current device");
    if (!stream) dev = cur;
    else if (hipStreamGetDevice(stream, &dev) != hipSuccess)
        return fail(RMI_ERR_STREAM, "gqa_flash_decode_noalloc: cannot query the stream's device");
    if (dev < 0 || dev >= kMaxDevices) return fail(RMI_ERR_STATE, "gqa_flash_decode_noalloc: device ordinal too large");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        if (dev != cur && hipSetDevice(dev) != hipSuccess)
            return fail(RMI_ERR_LAUNCH, "gqa_flash_decode_noalloc: cannot select the stream's device");
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (dev != cur) (void) hipSetDevice(cur);
        if (e != hipSuccess || !p) return fail(RMI_ERR_LAUNCH, "gqa_flash_decode_noalloc: hipGetSymbolAddress failed");
        g_scratch_dev[dev] = p;
    }
    *out = static_cast<float*>(g_scratch_dev[dev]);
    return RMI_OK;
}

}  // namespace
}  // namespace rmi

extern "C" int rmi_gqa_flash_decode(const float* q, const uint16_t* kcache, const uint16_t* vcache, const int* pos,
                                    const float* gate_src, int gate_stride, float* y, int y_stride, uint8_t* q8,
                                    int q8_stride, void* workspace, int n_head, int n_kv, int head_dim, int ntok,
                                    int max_ctx, int nsub, float scale, void* stream) {
    int nchunks = 0;
    RMI_TRY(flash_decode_check(q, kcache, vcache, pos, gate_src, y, q8, n_head, n_kv, head_dim, ntok, max_ctx, nsub,
                               &nchunks));
    if (!aligned16(workspace)) return fail(RMI_ERR_POINTER, "gqa_flash_decode: invalid arguments");
    return flash_decode(q, kcache, vcache, pos, gate_src, gate_stride, y, y_stride, q8, q8_stride,
                        static_cast<float*>(workspace), kMaxSlots, n_head, n_kv, ntok, nchunks, nsub, max_ctx, scale,
                        static_cast<hipStream_t>(stream));
}

namespace rmi {
namespace {
int flash_decode_prep(const float* q3, int q3_stride, const float* qn, const float* kn, uint16_t* kcache,
                      uint16_t* vcache, const int* pos, float* y, int y_stride, uint8_t* q8, int q8_stride,
                      void* workspace, int n_head, int n_kv, int head_dim, int n_rot, const rmi_rope_params* rope,
                      float eps, int ntok, int max_ctx, int nsub, float scale, float* rope_cs, int cs_mode,
                      void* stream) {
    if (head_dim != HD || n_head <= 0 || n_kv <= 0 || n_head % n_kv || ntok < 1 || ntok * (n_head / n_kv) > SLOTS ||
        max_ctx <= 0 || max_ctx % SUB || nsub <= 0 || n_rot != 64 || (n_head / n_kv) % 2 || !rope ||
        !(rope->freq_base > 1.0f))
        return fail(RMI_ERR_SHAPE, "gqa_flash_decode_prep: invalid arguments (one slot group: ntok x heads per KV head "
                                   "<= 8, an even number of heads per KV head, 64 rotary dims)");
    if (!aligned4(q3) || !aligned4(qn) || !aligned4(kn) || !aligned16(kcache) || !aligned16(vcache) ||
        !aligned4(pos) || !aligned16(workspace) || (!y && !q8))
        return fail(RMI_ERR_POINTER, "gqa_flash_decode_prep: invalid arguments");
    const int chunk_len = SUB * nsub, nchunks = (max_ctx + chunk_len - 1) / chunk_len;
    if (nchunks > kMaxChunks) return fail(RMI_ERR_SHAPE, "gqa_flash_decode_prep: max_ctx / (64 * nsub) exceeds 2048 chunks");
    Yarn yarn{};
    if (!yarn_setup(*rope, n_rot, &yarn)) return fail(RMI_ERR_SHAPE, "gqa_flash_decode_prep: invalid YaRN parameters");
    if (cs_mode != kRopeOwn && (!rope_cs || (reinterpret_cast<uintptr_t>(rope_cs) & 7u) || cs_mode > kRopeRead))
        return fail(RMI_ERR_POINTER, "gqa_flash_decode_prep: rope table mode 1 or 2 needs an 8-byte aligned table");
    const PrepIn pr{q3,  q3_stride, qn,   kn, kcache, vcache, n_rot, rope->freq_base, eps, yarn,
                    reinterpret_cast<float2*>(rope_cs), cs_mode};
    const auto s = static_cast<hipStream_t>(stream);
    auto* ws = static_cast<float*>(workspace);
    hipLaunchKernelGGL(gqa_partial_kernel<true>, dim3(nchunks * n_kv, 1, 1), dim3(256), 0, s, nullptr, kcache, vcache,
                       pos, ws, kMaxSlots, n_head, n_kv, ntok, nsub, max_ctx, scale, pr);
    hipLaunchKernelGGL(gqa_merge_kernel, dim3(ntok, n_head, kMergeParts), dim3(HD), 0, s, ws, kMaxSlots, q3, q3_stride,
                       pos, y, y_stride, q8, q8_stride, n_head, n_kv, SUB * nsub);
    return launch_status("gqa_flash_decode_prep");
}
}  // namespace
}  // namespace rmi

extern "C" int rmi_gqa_flash_decode_prep(const float* q3, int q3_stride, const float* qn, const float* kn,
                                         uint16_t* kcache, uint16_t* vcache, const int* pos, float* y, int y_stride,
                                         uint8_t* q8, int q8_stride, void* workspace, int n_head, int n_kv,
                                         int head_dim, int n_rot, const rmi_rope_params* rope, float eps, int ntok,
                                         int max_ctx, int nsub, float scale, void* stream) {
    return flash_decode_prep(q3, q3_stride, qn, kn, kcache, vcache, pos, y, y_stride, q8, q8_stride, workspace, n_head,
                             n_kv, head_dim, n_rot, rope, eps, ntok, max_ctx, nsub, scale, nullptr, kRopeOwn, stream);
}

extern "C" size_t rmi_gqa_rope_table_bytes(int n_rot) {
    return n_rot > 0 && n_rot % 2 == 0 ? static_cast<size_t>(2) * (n_rot / 2) * 2 * sizeof(float) : 0;
}

extern "C" int rmi_gqa_flash_decode_prep_rt(const float* q3, int q3_stride, const float* qn, const float* kn,
                                            uint16_t* kcache, uint16_t* vcache, const int* pos, float* y,
                                            int y_stride, uint8_t* q8, int q8_stride, void* workspace, int n_head,
                                            int n_kv, int head_dim, int n_rot, const rmi_rope_params* rope, float eps,
                                            int ntok, int max_ctx, int nsub, float scale, float* rope_table,
                                            int table_mode, void* stream) {
    if (table_mode < kRopeOwn || table_mode > kRopeRead)
        return fail(RMI_ERR_SHAPE, "gqa_flash_decode_prep_rt: table_mode must be 0, 1 or 2");
    return flash_decode_prep(q3, q3_stride, qn, kn, kcache, vcache, pos, y, y_stride, q8, q8_stride, workspace, n_head,
                             n_kv, head_dim, n_rot, rope, eps, ntok, max_ctx, nsub, scale, rope_table, table_mode,
                             stream);
}

extern "C" size_t rmi_gqa_noalloc_scratch_bytes(int max_ctx, int n_kv, int nsub, int slots) {
    if (max_ctx <= 0 || n_kv <= 0 || nsub <= 0 || slots <= 0) return 0;
    const int chunk_len = SUB * nsub;
    const size_t nchunks = static_cast<size_t>((max_ctx + chunk_len - 1) / chunk_len);
    const size_t stride = static_cast<size_t>((slots + SLOTS - 1) / SLOTS) * SLOTS;
    return nchunks * static_cast<size_t>(n_kv) * stride * REC * sizeof(float);
}

extern "C" size_t rmi_gqa_noalloc_scratch_max(void) { return kScratchBytes; }

extern "C" int rmi_gqa_flash_decode_noalloc(const float* q, const uint16_t* kcache, const uint16_t* vcache,
                                            const int* pos, const float* gate_src, int gate_stride, float* y,
                                            int y_stride, uint8_t* q8, int q8_stride, int n_head, int n_kv,
                                            int head_dim, int ntok, int max_ctx, int nsub, float scale, void* stream) {
    int nchunks = 0;
    RMI_TRY(flash_decode_check(q, kcache, vcache, pos, gate_src, y, q8, n_head, n_kv, head_dim, ntok, max_ctx, nsub,
                               &nchunks));
    const int slots = ntok * (n_head / n_kv);
    const int slot_stride = (slots + SLOTS - 1) / SLOTS * SLOTS;
    if (rmi_gqa_noalloc_scratch_bytes(max_ctx, n_kv, nsub, slots) > kScratchBytes)
        return fail(RMI_ERR_SHAPE, "gqa_flash_decode_noalloc: the split-K records exceed the 16 MiB scratch "
                                   "(chunks x kv heads x query slots; use a larger nsub or rmi_gqa_flash_decode)");
    float* ws = nullptr;
    const auto s = static_cast<hipStream_t>(stream);
    RMI_TRY(scratch_address(s, &ws));
    return flash_decode(q, kcache, vcache, pos, gate_src, gate_stride, y, y_stride, q8, q8_stride, ws, slot_stride,
                        n_head, n_kv, ntok, nchunks, nsub, max_ctx, scale, s);
}
