// topk.hip - the k largest logits (k <= 64) with their token ids, on the device: the per-token list the serve protocol
// prints (reference qw:2513-2531, topk_out: a host scan over all n logits keeping the k largest in descending order; an
// incoming logit must be strictly greater than the current k-th to displace it, so among equal logits the lower id
// ranks first and is kept).  Here each logit becomes a 64-bit key (order-preserving float bits with -0 folded into +0,
// then the inverted id), all keys are distinct, and the list is the k largest keys in descending order: the same
// (logit descending, id ascending) order.
//
// Two launches.  topk_lists: one wave per 64*E consecutive logits; each lane sorts its E keys in registers (a bitonic
// network, compile-time indices), then k rounds of a wave max over the lanes' heads pop the wave's k largest into a
// sorted list (one key per lane, 0 past k); the four waves of a workgroup then merge their lists into one.
// topk_merge: one 512-lane workgroup merges the workgroups' lists pairwise, level by level, in LDS.  Two sorted lists
// merge in one wave: lane l takes max(A[l], B[63 - l]), the top half of the bitonic sequence A | reverse(B), i.e. the
// 64 largest keys of both, and a bitonic half-cleaner network (lane strides 32 .. 1) sorts them.
#include "rmi_common.h"

namespace rmi {
namespace {

constexpr int kTopkMax = 64;       // largest k
constexpr int kListStride = 64;    // keys per list in the workspace
constexpr int kMergeLanes = 512;   // waves of the list pass at most (4 per workgroup list)
constexpr int kMaxLists = kMergeLanes / 4;   // workgroup lists the merge holds in LDS (64 KB)

__device__ __forceinline__ uint64_t topk_key(float v, uint32_t idx) {
    uint32_t b = __float_as_uint(v);
    if (b == 0x80000000u) b = 0u;   // -0 compares equal to +0
    b ^= (b >> 31) ? 0xffffffffu : 0x80000000u;
    return (static_cast<uint64_t>(b) << 32) | (0xffffffffu - idx);   // > 0 for every real key; 0 = no entry
}

__device__ __forceinline__ uint64_t max64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// lane exchange by a DPP pattern (every lane active)
template <int CTRL>
__device__ __forceinline__ uint64_t dpp64(uint64_t v) {
    const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(v)), CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(v >> 32)), CTRL, 0xf, 0xf,
                                               false);
    return (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo);
}

__device__ __forceinline__ uint64_t readlane64(uint64_t v, int lane) {
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v)), lane));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v >> 32)),
                                                                        lane));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// wave-uniform max of a 64-bit key: DPP within each row of 16 lanes (xor 1, xor 2, half-row mirror, row mirror; max
// is symmetric, so a mirror partner serves as well as an xor one), then the four row maxima read into scalars.
// Called with every lane of the wave active.
__device__ __forceinline__ uint64_t wave_max64(uint64_t k) {
    k = max64(k, dpp64<0xb1>(k));    // quad_perm [1,0,3,2]
    k = max64(k, dpp64<0x4e>(k));    // quad_perm [2,3,0,1]
    k = max64(k, dpp64<0x141>(k));   // row_half_mirror
    k = max64(k, dpp64<0x140>(k));   // row_mirror
    return max64(max64(readlane64(k, 0), readlane64(k, 16)), max64(readlane64(k, 32), readlane64(k, 48)));
}

// key of lane l ^ K (the VALU lane exchange of rmi_common.h on both halves)
template <int K>
__device__ __forceinline__ uint64_t xor64(uint64_t v) {
    const uint32_t lo = xor_lane<K>(static_cast<uint32_t>(v)), hi = xor_lane<K>(static_cast<uint32_t>(v >> 32));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

template <int K>
__device__ __forceinline__ uint64_t half_clean(uint64_t v, int lane) {
    const uint64_t o = xor64<K>(v);
    return (lane & K) ? (v < o ? v : o) : (v > o ? v : o);
}

// The 64 largest keys of two descending lists, descending, one per lane: a = A[lane], b = B[63 - lane].  Called with
// every lane of the wave active.
__device__ __forceinline__ uint64_t merge_lists(uint64_t a, uint64_t b) {
    const int lane = __lane_id();
    uint64_t v = a > b ? a : b;
    v = half_clean<32>(v, lane);
    v = half_clean<16>(v, lane);
    v = half_clean<8>(v, lane);
    v = half_clean<4>(v, lane);
    v = half_clean<2>(v, lane);
    return half_clean<1>(v, lane);
}

template <int E>
__global__ __launch_bounds__(256) void topk_lists_kernel(const float* __restrict__ x, int n, int k,
                                                         uint64_t* __restrict__ lists) {
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t base = static_cast<int64_t>(wave) * 64 * E;
    // every load issued before the first use, from clamped indices (a load under a branch gets a wait of its own)
    float xv[E];
#pragma unroll
    for (int j = 0; j < E; ++j) xv[j] = x[min(base + lane + 64 * j, static_cast<int64_t>(n) - 1)];
    uint64_t v[E];
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int64_t i = base + lane + 64 * j;
        v[j] = i < n ? topk_key(xv[j], static_cast<uint32_t>(i)) : 0ull;
    }
    // bitonic sort of the lane's E keys, descending
#pragma unroll
    for (int size = 2; size <= E; size <<= 1) {
#pragma unroll
        for (int stride = size / 2; stride > 0; stride >>= 1) {
#pragma unroll
            for (int i = 0; i < E; ++i) {
                const int j = i ^ stride;
                if (j > i) {
                    const uint64_t a = v[i], b = v[j];
                    const bool swap = (i & size) == 0 ? a < b : a > b;
                    v[i] = swap ? b : a;
                    v[j] = swap ? a : b;
                }
            }
        }
    }
    uint64_t mine = 0;
    for (int it = 0; it < k; ++it) {
        const uint64_t m = wave_max64(v[0]);
        if (m == 0) break;              // the slice has fewer than k logits (uniform across the wave)
        if (lane == it) mine = m;
        if (v[0] == m) {                // keys are distinct: exactly one lane pops
#pragma unroll
            for (int j = 0; j + 1 < E; ++j) v[j] = v[j + 1];
            v[E - 1] = 0;
        }
    }
    // the workgroup's four lists into one: waves 0 / 1 merge lists (0, 1) / (2, 3), then wave 0 merges the two
    __shared__ uint64_t wl[4][64];
    const int w = threadIdx.x >> 6;
    wl[w][lane] = mine;
    __syncthreads();
    uint64_t m2 = 0;
    if (w < 2) m2 = merge_lists(wl[2 * w][lane], wl[2 * w + 1][63 - lane]);
    __syncthreads();
    if (w < 2) wl[w][lane] = m2;
    __syncthreads();
    if (w == 0) lists[static_cast<size_t>(blockIdx.x) * kListStride + lane] = merge_lists(wl[0][lane], wl[1][63 - lane]);
}

// Workgroup lists merged pairwise: each level reads every pair into registers (wave w takes pairs w, w + 8, ...), passes
// a barrier, and writes the merged lists to the first half of the slots; an odd last list moves down with them.
__global__ __launch_bounds__(kMergeLanes) void topk_merge_kernel(const float* __restrict__ x,
                                                                 const uint64_t* __restrict__ lists, int nlists, int k,
                                                                 int* __restrict__ out_idx, float* __restrict__ out_val) {
    __shared__ uint64_t buf[kMaxLists * kListStride];
    constexpr int kWaves = kMergeLanes / 64;
    constexpr int kPer = kMaxLists / 2 / kWaves;   // pairs per wave at the widest level
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    {   // every list entry of the lane loaded before the first store (a strided loop waits on each load in turn)
        constexpr int kLoads = kMaxLists * kListStride / kMergeLanes;
        const int total = nlists * kListStride;
        uint64_t lv[kLoads];
#pragma unroll
        for (int r = 0; r < kLoads; ++r) lv[r] = lists[min(t + kMergeLanes * r, total - 1)];
#pragma unroll
        for (int r = 0; r < kLoads; ++r)
            if (t + kMergeLanes * r < total) buf[t + kMergeLanes * r] = lv[r];
    }
    __syncthreads();
    for (int n = nlists; n > 1;) {
        const int pairs = n >> 1;
        uint64_t res[kPer], last = 0;
#pragma unroll
        for (int r = 0; r < kPer; ++r) {
            const int p = w + kWaves * r;
            res[r] = p < pairs ? merge_lists(buf[(2 * p) * kListStride + lane], buf[(2 * p + 1) * kListStride + 63 - lane])
                               : 0;
        }
        if ((n & 1) && w == 0) last = buf[(n - 1) * kListStride + lane];
        __syncthreads();
#pragma unroll
        for (int r = 0; r < kPer; ++r) {
            const int p = w + kWaves * r;
            if (p < pairs) buf[p * kListStride + lane] = res[r];
        }
        if ((n & 1) && w == 0) buf[pairs * kListStride + lane] = last;
        __syncthreads();
        n = pairs + (n & 1);
    }
    if (t < k) {
        const uint64_t key = buf[t];
        const int idx = key ? static_cast<int>(0xffffffffu - static_cast<uint32_t>(key)) : -1;
        out_idx[t] = idx;
        out_val[t] = idx >= 0 ? x[idx] : 0.0f;
    }
}

// logits per lane of the list pass: the smallest of 8, 16, 32 that keeps the lists within one merge workgroup
int lane_elems(int n) {
    for (int e = 8; e <= 32; e *= 2) {
        const int64_t waves = (static_cast<int64_t>(n) + 64 * e - 1) / (64 * e);
        if ((waves + 3) / 4 * 4 <= kMergeLanes) return e;
    }
    return 0;
}

}  // namespace
}  // namespace rmi

using namespace rmi;

extern "C" size_t rmi_topk_workspace_bytes(int n) {
    const int e = lane_elems(n);
    if (n <= 0 || e == 0) return 0;
    const int64_t waves = (static_cast<int64_t>(n) + 64 * e - 1) / (64 * e);
    return static_cast<size_t>((waves + 3) / 4 * 4) * kListStride * sizeof(uint64_t);
}

extern "C" int rmi_topk(const float* logits, int n, int k, int* out_idx, float* out_val, void* workspace,
                        void* stream) {
    const int e = lane_elems(n);
    if (n <= 0 || e == 0) return fail(RMI_ERR_SHAPE, "topk: n must be 1..1048576");
    if (k < 1 || k > kTopkMax || k > n) return fail(RMI_ERR_SHAPE, "topk: k must be 1..min(64, n)");
    if (!aligned4(logits) || !aligned4(out_idx) || !aligned4(out_val) || !workspace ||
        (reinterpret_cast<uintptr_t>(workspace) & 7u) != 0)
        return fail(RMI_ERR_POINTER, "topk: null or misaligned pointer");
    const int64_t waves = (static_cast<int64_t>(n) + 64 * e - 1) / (64 * e);
    const int blocks = static_cast<int>((waves + 3) / 4);
    auto* lists = static_cast<uint64_t*>(workspace);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (e == 8) hipLaunchKernelGGL(topk_lists_kernel<8>, dim3(blocks), dim3(256), 0, s, logits, n, k, lists);
    else if (e == 16) hipLaunchKernelGGL(topk_lists_kernel<16>, dim3(blocks), dim3(256), 0, s, logits, n, k, lists);
    else hipLaunchKernelGGL(topk_lists_kernel<32>, dim3(blocks), dim3(256), 0, s, logits, n, k, lists);
    const int rc = launch_status("topk_lists");
    if (rc != RMI_OK) return rc;
    hipLaunchKernelGGL(topk_merge_kernel, dim3(1), dim3(kMergeLanes), 0, s, logits, lists, blocks, k, out_idx, out_val);
    return launch_status("topk_merge");
}
