// attn.hip - GQA decode attention for gfx950 over an fp16 KV cache (reference src/qwythos.cpp: split_qg_kernel
// 320-327, store_kv2_kernel 340-345, gqa_head_kernel 384-442, sig_mul_quant_kernel 692-704, glue 1530-1558).
//
//   attn_prep   one workgroup per (token, head): q heads get the per-head RMSNorm (weights qn) and NEOX RoPE on the
//               first n_rot dims -> fp32 q buffer; k heads get RMSNorm (kn) + RoPE and v heads nothing, both stored
//               as fp16 at cache[pos_t][kv][d].  pos_t = pos[0] + t is read on the device.
//   partial     split-K flash decode.  Workgroup (chunk, kv head) covers positions [chunk * 64 * nsub, +64 * nsub) for
//               every query vector of its group (group heads x tokens): QK^T on MFMA 16x16x16 f16 with q split into
//               fp16 hi + lo (so scores carry ~fp32 precision against the exact fp16 K), online softmax per query,
//               P V with fp32 FMAs over coalesced fp16 V rows.  Writes (m, l, o[256]) per query vector.
//   merge       one workgroup per (token, head): merges that query's chunks 0..pos_t / chunk in order, divides, gates
//               with sigmoid(g) and writes fp32 y plus Q8_1 for the wo GEMV.
// Query t sees positions <= pos[0] + t.  Chunk boundaries depend only on the query's position, so a verify column's
// result is bitwise the single-token result at the same position.
#include "rmi_common.h"

namespace rmi {
namespace {

constexpr int HD = 256;
constexpr int SUB = 64;            // positions per sub-tile (4 waves x 16)
constexpr int REC = HD + 4;        // workspace record: m, l, pad, pad, o[256]
constexpr int MAXQ = 16;           // query vectors per kv head one launch handles (MFMA N)

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
// q3 per token: [n_head x (q HD | gate HD) | k n_kv*HD | v n_kv*HD] at q3 + t * q3_stride.
__global__ __launch_bounds__(HD) void attn_prep_kernel(const float* __restrict__ q3, int q3_stride,
                                                       const float* __restrict__ qn, const float* __restrict__ kn,
                                                       uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                                       const int* __restrict__ pos, float* __restrict__ qout,
                                                       int n_head, int n_kv, int n_rot, int max_ctx, float theta,
                                                       float eps) {
    __shared__ float red[4];
    __shared__ float xs[HD];
    const int t = blockIdx.x;
    const int hh = blockIdx.y;   // [0, n_head) q, [n_head, n_head + n_kv) k, then v
    const int d = threadIdx.x;
    const float* src = q3 + static_cast<size_t>(t) * q3_stride;
    const int p = pos[0] + t;
    if (p < 0 || p >= max_ctx) return;   // uniform: a position outside the cache stores nothing
    if (hh >= n_head + n_kv) {   // v: straight to the cache
        const int kv = hh - n_head - n_kv;
        const float v = src[2 * n_head * HD + n_kv * HD + kv * HD + d];
        vc[(static_cast<size_t>(p) * n_kv + kv) * HD + d] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
        return;
    }
    const bool is_q = hh < n_head;
    const float x = is_q ? src[hh * 2 * HD + d] : src[2 * n_head * HD + (hh - n_head) * HD + d];
    const float ss = block_sum256(x * x, red);
    const float inv = rsqrtf(ss / static_cast<float>(HD) + eps);
    float v = x * inv * (is_q ? qn[d] : kn[d]);
    xs[d] = v;
    __syncthreads();
    const int half = n_rot / 2;
    if (d < n_rot) {
        const int i = d < half ? d : d - half;
        const double ang = static_cast<double>(p) * pow(static_cast<double>(theta), -2.0 * i / static_cast<double>(n_rot));
        double sn, cs;
        sincos(ang, &sn, &cs);
        const float c = static_cast<float>(cs), s = static_cast<float>(sn);
        v = d < half ? xs[d] * c - xs[d + half] * s : xs[d - half] * s + xs[d] * c;
    }
    if (is_q) {
        qout[(static_cast<size_t>(t) * n_head + hh) * HD + d] = v;
    } else {
        const int kv = hh - n_head;
        kc[(static_cast<size_t>(p) * n_kv + kv) * HD + d] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
    }
}

// ---- split-K partial ---------------------------------------------------------------------------------------------------
// Query vector qv = t * G + gh (token t, head kv * G + gh).  MFMA 16x16x16 f16, lane l: A rows (positions) l % 16 with
// k = 4 (l / 16) .. +3; B cols (query vectors) l % 16, same k; D col l % 16, rows 4 (l / 16) .. +3.  The head
// dimension is walked in 8 pairs of k-steps: in pair sp, lane group g = l / 16 supplies dims 32 sp + 8 g + 0..3 (first
// step) and + 4..7 (second step) for both operands, so one 16-byte K load feeds two MFMAs.
__global__ __launch_bounds__(256) void gqa_partial_kernel(const float* __restrict__ qbuf, const uint16_t* __restrict__ kc,
                                                          const uint16_t* __restrict__ vc, const int* __restrict__ pos,
                                                          float* __restrict__ ws, int n_head, int n_kv, int ntok,
                                                          int nsub, int max_ctx, float scale) {
    __shared__ float pbuf[SUB][MAXQ];
    __shared__ float red[4][MAXQ];
    __shared__ float msh[MAXQ];
    __shared__ float opart[MAXQ][128 * 2];
    const int chunk = blockIdx.x, kv = blockIdx.y;
    const int G = n_head / n_kv;
    const int nq = ntok * G;
    const int p0 = pos[0];
    const int p_last = p0 + ntok - 1;
    const int cbase = chunk * SUB * nsub;
    if (cbase > p_last || p0 < 0 || p_last >= max_ctx) return;   // uniform: no visible position (or a bad pos)

    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int l16 = lane & 15, g4 = lane >> 4;

    // B operand: q hi/lo for query vector l16
    half4 qhi[16], qlo[16];
    {
        const int qv = l16;
        const bool ok = qv < nq;
        const int t = ok ? qv / G : 0, gh = ok ? qv - (qv / G) * G : 0;
        const float* q = qbuf + (static_cast<size_t>(t) * n_head + kv * G + gh) * HD;
#pragma unroll
        for (int sp = 0; sp < 8; ++sp) {
#pragma unroll
            for (int hlf = 0; hlf < 2; ++hlf) {
                half4 hi, lo;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float x = ok ? q[32 * sp + 8 * g4 + 4 * hlf + e] : 0.0f;
                    const _Float16 h = static_cast<_Float16>(x);
                    hi[e] = h;
                    lo[e] = static_cast<_Float16>(x - static_cast<float>(h));
                }
                qhi[2 * sp + hlf] = hi;
                qlo[2 * sp + hlf] = lo;
            }
        }
    }

    // P V ownership: dims pair dp (2 dims), position half ph of each sub-tile
    const int dp = threadIdx.x & 127, ph = threadIdx.x >> 7;
    float o[MAXQ][2];
#pragma unroll
    for (int q = 0; q < MAXQ; ++q) o[q][0] = o[q][1] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;   // for query vector l16 (replicated across lane groups and waves)

    for (int sb = 0; sb < nsub; ++sb) {
        const int sbase = cbase + sb * SUB;
        if (sbase > p_last) break;   // uniform
        // ---- scores: wave wv owns positions sbase + 16 wv + [0, 16)
        floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        {
            const int prow = sbase + 16 * wv + l16;
            const uint16_t* krow = kc + (static_cast<size_t>(prow) * n_kv + kv) * HD;
#pragma unroll
            for (int sp = 0; sp < 8; ++sp) {
                const uint4 kw = *reinterpret_cast<const uint4*>(krow + 32 * sp + 8 * g4);
                half4 k0, k1;
                k0 = __builtin_bit_cast(half4, make_uint2(kw.x, kw.y));
                k1 = __builtin_bit_cast(half4, make_uint2(kw.z, kw.w));
                acc = __builtin_amdgcn_mfma_f32_16x16x16f16(k0, qhi[2 * sp], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x16f16(k0, qlo[2 * sp], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x16f16(k1, qhi[2 * sp + 1], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x16f16(k1, qlo[2 * sp + 1], acc, 0, 0, 0);
            }
        }
        // lane holds scores of query l16 at positions sbase + 16 wv + 4 g4 + r
        const int qv = l16;
        const int tq = qv < nq ? qv / G : 0;
        const int lim = qv < nq ? p0 + tq : -1;   // last visible position for this query vector
        float s[4];
        float mloc = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int pp = sbase + 16 * wv + 4 * g4 + r;
            s[r] = pp <= lim ? acc[r] * scale : -INFINITY;
            mloc = fmaxf(mloc, s[r]);
        }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
        if (g4 == 0) red[wv][qv] = mloc;
        __syncthreads();
        const float msub = fmaxf(fmaxf(red[0][qv], red[1][qv]), fmaxf(red[2][qv], red[3][qv]));
        const float m_new = fmaxf(m_run, msub);
        const float m_ref = m_new == -INFINITY ? 0.0f : m_new;   // all masked so far: exp(-inf) = 0, no NaN
        float lloc = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float pr = expf(s[r] - m_ref);
            pbuf[16 * wv + 4 * g4 + r][qv] = pr;
            lloc += pr;
        }
        lloc += __shfl_xor(lloc, 16, 64);
        lloc += __shfl_xor(lloc, 32, 64);
        __syncthreads();   // everyone has read red (max) before it holds the sums
        if (g4 == 0) red[wv][qv] = lloc;
        __syncthreads();
        const float lsub = ((red[0][qv] + red[1][qv]) + red[2][qv]) + red[3][qv];
        const float alpha = m_run == -INFINITY ? 0.0f : expf(m_run - m_ref);
        l_run = l_run * alpha + lsub;
        // rescale factor per query vector for the P V owners, via LDS
        if (threadIdx.x < MAXQ) msh[threadIdx.x] = alpha;
        m_run = m_new;
        __syncthreads();
        // ---- P V: positions sbase + 32 ph + [0, 32) that are <= p_last
        const int pend = min(32, p_last - (sbase + 32 * ph) + 1);
#pragma unroll
        for (int q = 0; q < MAXQ; ++q) {
            const float a = msh[q];
            o[q][0] *= a;
            o[q][1] *= a;
        }
        const uint32_t* vbase = reinterpret_cast<const uint32_t*>(vc + (static_cast<size_t>(sbase + 32 * ph) * n_kv + kv) * HD) + dp;
        // all 32 V rows of this half are loaded before the FMA chain (positions past p_last are not read)
        uint32_t vw[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) vw[i] = i < pend ? vbase[static_cast<size_t>(i) * n_kv * (HD / 2)] : 0u;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            if (i < pend) {
                const float v0 = half_bits_to_float(vw[i]), v1 = half_bits_to_float(vw[i] >> 16);
                const float* prow = pbuf[32 * ph + i];
#pragma unroll
                for (int q = 0; q < MAXQ; ++q) {
                    if (q < nq) {
                        o[q][0] = __builtin_fmaf(prow[q], v0, o[q][0]);
                        o[q][1] = __builtin_fmaf(prow[q], v1, o[q][1]);
                    }
                }
            }
        }
        __syncthreads();   // pbuf / msh reused by the next sub-tile
    }
    // combine the two position halves in order (half 0 + half 1) and write the records
    if (ph == 1) {
#pragma unroll
        for (int q = 0; q < MAXQ; ++q) {
            opart[q][2 * dp] = o[q][0];
            opart[q][2 * dp + 1] = o[q][1];
        }
    }
    __syncthreads();
    if (ph == 0) {
        for (int q = 0; q < nq; ++q) {
            float* rec = ws + ((static_cast<size_t>(chunk) * n_kv + kv) * MAXQ + q) * REC;
            rec[4 + 2 * dp] = o[q][0] + opart[q][2 * dp];
            rec[4 + 2 * dp + 1] = o[q][1] + opart[q][2 * dp + 1];
        }
    }
    if (threadIdx.x < nq) {   // lanes 0..15 of wave 0 hold m_run / l_run of query vector threadIdx.x
        float* rec = ws + ((static_cast<size_t>(chunk) * n_kv + kv) * MAXQ + threadIdx.x) * REC;
        rec[0] = m_run;
        rec[1] = l_run;
    }
}

// ---- merge + sigmoid gate + Q8_1 ---------------------------------------------------------------------------------------
// Two passes over the query's chunks 0..last: (1) the 256 lanes load every chunk's (m, l) in parallel, M = max m,
// weights w_c = exp(m_c - M) to LDS, L = sum l_c w_c (lane-strided partial sums, butterfly, waves in order);
// (2) lane d accumulates O = sum_c w_c o_c[d] in chunk order with the loads issued 8 chunks ahead.
constexpr int kMaxChunks = 2048;

__global__ __launch_bounds__(HD) void gqa_merge_kernel(const float* __restrict__ ws, const float* __restrict__ gsrc,
                                                       int gstride, const int* __restrict__ pos, float* __restrict__ y,
                                                       int y_stride, uint8_t* __restrict__ q8, int q8_stride,
                                                       int n_head, int n_kv, int chunk_len) {
    __shared__ float wts[kMaxChunks];
    __shared__ float red[4];
    const int t = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
    const int G = n_head / n_kv;
    const int kv = h / G, qv = t * G + (h - kv * G);
    const int nchunk = min((pos[0] + t) / chunk_len + 1, kMaxChunks);
    const size_t cstride = static_cast<size_t>(n_kv) * MAXQ * REC;
    const float* base = ws + (static_cast<size_t>(kv) * MAXQ + qv) * REC;
    float mloc = -INFINITY;
    for (int c = d; c < nchunk; c += HD) mloc = fmaxf(mloc, base[c * cstride]);
    mloc = group_max<64>(mloc);
    if ((d & 63) == 0) red[d >> 6] = mloc;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float lloc = 0.0f;
    for (int c = d; c < nchunk; c += HD) {
        const float w = expf(base[c * cstride] - M);
        wts[c] = w;
        lloc = __builtin_fmaf(base[c * cstride + 1], w, lloc);
    }
    const float L = block_sum256(lloc, red);   // includes the barrier that publishes wts
    float O = 0.0f;
    int c = 0;
    for (; c + 8 <= nchunk; c += 8) {
        float oc[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) oc[k] = base[(c + k) * cstride + 4 + d];
#pragma unroll
        for (int k = 0; k < 8; ++k) O = __builtin_fmaf(wts[c + k], oc[k], O);
    }
    for (; c < nchunk; ++c) O = __builtin_fmaf(wts[c], base[c * cstride + 4 + d], O);
    const float o = O / L;
    const float g = gsrc[static_cast<size_t>(t) * gstride + h * 2 * HD + HD + d];
    const float v = o * sigmoid(g);
    if (y) y[static_cast<size_t>(t) * y_stride + h * HD + d] = v;
    if (q8) q8_1_store_lane(v, q8 + static_cast<size_t>(t) * q8_stride + (h * (HD / 32) + d / 32) * kQ8_1Bytes);
}

}  // namespace
}  // namespace rmi

using namespace rmi;

extern "C" int rmi_attn_prep(const float* q3, int q3_stride, const float* qn, const float* kn, uint16_t* kcache,
                             uint16_t* vcache, const int* pos, float* qout, int n_head, int n_kv, int head_dim,
                             int n_rot, float theta, float eps, int ntok, int max_ctx, void* stream) {
    if (head_dim != HD || n_head <= 0 || n_kv <= 0 || n_head % n_kv || n_rot < 0 || n_rot > HD || n_rot % 2 ||
        ntok < 1 || ntok > 2)
        return fail(RMI_ERR_SHAPE, "attn_prep: invalid arguments");
    if (!aligned4(q3) || !aligned4(qn) || !aligned4(kn) || !kcache || !vcache || !aligned4(pos) || !aligned4(qout))
        return fail(RMI_ERR_POINTER, "attn_prep: invalid arguments");
    hipLaunchKernelGGL(attn_prep_kernel, dim3(ntok, n_head + 2 * n_kv), dim3(HD), 0, static_cast<hipStream_t>(stream),
                       q3, q3_stride, qn, kn, kcache, vcache, pos, qout, n_head, n_kv, n_rot, max_ctx, theta, eps);
    return launch_status("attn_prep");
}

extern "C" size_t rmi_gqa_workspace_bytes(int max_ctx, int n_kv, int nsub) {
    if (max_ctx <= 0 || n_kv <= 0 || nsub <= 0) return 0;
    const int chunk_len = SUB * nsub;
    const size_t nchunks = static_cast<size_t>((max_ctx + chunk_len - 1) / chunk_len);
    return nchunks * static_cast<size_t>(n_kv) * MAXQ * REC * sizeof(float);
}

extern "C" int rmi_gqa_flash_decode(const float* q, const uint16_t* kcache, const uint16_t* vcache, const int* pos,
                                    const float* gate_src, int gate_stride, float* y, int y_stride, uint8_t* q8,
                                    int q8_stride, void* workspace, int n_head, int n_kv, int head_dim, int ntok,
                                    int max_ctx, int nsub, float scale, void* stream) {
    if (head_dim != HD || n_head <= 0 || n_kv <= 0 || n_head % n_kv || ntok < 1 || ntok * (n_head / n_kv) > MAXQ ||
        max_ctx <= 0 || max_ctx % SUB || nsub <= 0)
        return fail(RMI_ERR_SHAPE, "gqa_flash_decode: invalid arguments");
    if (!aligned4(q) || !aligned4(kcache) || !aligned4(vcache) || !aligned4(pos) || !aligned4(gate_src) ||
        !aligned4(workspace) || (!y && !q8))
        return fail(RMI_ERR_POINTER, "gqa_flash_decode: invalid arguments");
    const int chunk_len = SUB * nsub;
    const int nchunks = (max_ctx + chunk_len - 1) / chunk_len;
    if (nchunks > kMaxChunks) return fail(RMI_ERR_SHAPE, "gqa_flash_decode: max_ctx / (64 * nsub) exceeds 2048 chunks");
    const auto s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(gqa_partial_kernel, dim3(nchunks, n_kv), dim3(256), 0, s, q, kcache, vcache, pos,
                       static_cast<float*>(workspace), n_head, n_kv, ntok, nsub, max_ctx, scale);
    hipLaunchKernelGGL(gqa_merge_kernel, dim3(ntok, n_head), dim3(HD), 0, s, static_cast<const float*>(workspace),
                       gate_src, gate_stride, pos, y, y_stride, q8, q8_stride, n_head, n_kv, chunk_len);
    return launch_status("gqa_flash_decode");
}
