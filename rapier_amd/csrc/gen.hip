// gen.hip - seeded synthetic tensors generated in HBM (the stand-in for a GGUF file: random-init weights of the
// qwen35 shapes).  Counter-based: element i of stream `seed` is mix64(seed * K1 + (i + 1) * K2), so any element is
// drawn independently and the integer fields match the host generator bit for bit.
//   Q6_K: 256 codes U{0..63} (eight 6-bit codes per 64-bit draw), 16 sub-scales U[-32,31], d = fp16(|N(0, d_std)|)
//   normal: Box-Muller in fp64 over two draws.
#include "rmi_common.h"

namespace rmi {
namespace {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t rand_u64(uint64_t seed, uint64_t i) {
    return mix64(seed * 0xD1B54A32D192ED03ULL + (i + 1) * 0x9E3779B97F4A7C15ULL);
}
__device__ __forceinline__ double rand_unit(uint64_t seed, uint64_t i) {
    return static_cast<double>(rand_u64(seed, i) >> 11) * (1.0 / 9007199254740992.0);
}
__device__ __forceinline__ double rand_normal(uint64_t seed, uint64_t i) {
    const double u1 = 1.0 - rand_unit(seed, 2 * i);
    const double u2 = rand_unit(seed, 2 * i + 1);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

// one lane per Q6_K block; the block is assembled in registers and written as 105 u16 stores
__global__ __launch_bounds__(256) void gen_q6k_kernel(uint8_t* __restrict__ w, size_t nblocks, uint64_t seed,
                                                      float d_std) {
    const size_t bi = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    if (bi >= nblocks) return;
    const uint64_t s_codes = seed ^ 0x51ULL, s_sc = seed ^ 0x52ULL, s_d = seed ^ 0x53ULL;
    uint32_t ql[32], qh[16];
#pragma unroll
    for (int i = 0; i < 32; ++i) ql[i] = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) qh[i] = 0;
    for (int g = 0; g < 32; ++g) {   // codes e = 8g .. 8g+7
        const uint64_t r = rand_u64(s_codes, bi * 32 + g);
        for (int m = 0; m < 8; ++m) {
            const int e = 8 * g + m;
            const uint32_t c = static_cast<uint32_t>((r >> (8 * m)) & 63);
            const int n = e >> 7, k = (e & 127) >> 5, l = e & 31;
            const int qlb = 64 * n + 32 * (k & 1) + l;
            const uint32_t nib = (k >> 1) ? ((c & 15) << 4) : (c & 15);
            ql[qlb >> 2] |= nib << (8 * (qlb & 3));
            const int qhb = 32 * n + l;
            qh[qhb >> 2] |= ((c >> 4) << (2 * k)) << (8 * (qhb & 3));
        }
    }
    uint32_t sc[4];
    const uint64_t r0 = rand_u64(s_sc, 2 * bi), r1 = rand_u64(s_sc, 2 * bi + 1);
    for (int i = 0; i < 4; ++i) {
        const uint64_t r = i < 2 ? r0 : r1;
        uint32_t word = 0;
        for (int m = 0; m < 4; ++m) {
            const int byte = static_cast<int>((r >> (8 * (4 * (i & 1) + m))) & 63) - 32;
            word |= (static_cast<uint32_t>(byte) & 0xffu) << (8 * m);
        }
        sc[i] = word;
    }
    const uint16_t d = f32_to_f16_bits(static_cast<float>(fabs(d_std * rand_normal(s_d, bi))));
    uint16_t* o = reinterpret_cast<uint16_t*>(w + bi * kQ6KBytes);   // 210 * bi is even: u16-aligned
    for (int i = 0; i < 32; ++i) { o[2 * i] = ql[i] & 0xffff; o[2 * i + 1] = ql[i] >> 16; }
    for (int i = 0; i < 16; ++i) { o[64 + 2 * i] = qh[i] & 0xffff; o[64 + 2 * i + 1] = qh[i] >> 16; }
    for (int i = 0; i < 4; ++i) { o[96 + 2 * i] = sc[i] & 0xffff; o[96 + 2 * i + 1] = sc[i] >> 16; }
    o[104] = d;
}

__global__ __launch_bounds__(256) void gen_q8_0_kernel(uint8_t* __restrict__ w, size_t nblocks, uint64_t seed,
                                                       float d_std) {
    const size_t bi = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    if (bi >= nblocks) return;
    uint16_t* o = reinterpret_cast<uint16_t*>(w + bi * kQ8_0Bytes);
    o[0] = f32_to_f16_bits(static_cast<float>(fabs(d_std * rand_normal(seed ^ 0x61ULL, bi))));
    for (int m = 0; m < 4; ++m) {
        const uint64_t r = rand_u64(seed ^ 0x62ULL, bi * 4 + m);
        for (int t = 0; t < 4; ++t) o[1 + 4 * m + t] = static_cast<uint16_t>((r >> (16 * t)) & 0xffff);
    }
}

__global__ __launch_bounds__(256) void gen_normal_kernel(float* __restrict__ out, size_t n, uint64_t seed, float mean,
                                                         float std) {
    const size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    out[i] = static_cast<float>(static_cast<double>(mean) + static_cast<double>(std) * rand_normal(seed, i));
}

// fp16 variant (the KV cache): N(mean, std) rounded to fp16
__global__ __launch_bounds__(256) void gen_normal_f16_kernel(uint16_t* __restrict__ out, size_t n, uint64_t seed,
                                                             float mean, float std) {
    const size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    out[i] = f32_to_f16_bits(static_cast<float>(static_cast<double>(mean) + static_cast<double>(std) * rand_normal(seed, i)));
}

unsigned grid_of(size_t n) { return static_cast<unsigned>((n + 255) / 256); }

// the read-bandwidth reference of a single launch: grid-stride 16-byte nontemporal loads, eight per lane in flight,
// folded into one word that is stored only if it equals a sentinel (so the loads stay live)
typedef unsigned int rd_u32x4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void stream_read_kernel(const rd_u32x4* __restrict__ p, size_t n16, unsigned* out) {
    constexpr int U = 8;
    const size_t stride = static_cast<size_t>(gridDim.x) * 256;
    size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    unsigned acc = 0;
    for (; i + (U - 1) * stride < n16; i += U * stride) {
        rd_u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    for (; i < n16; i += stride) {
        const rd_u32x4 v = __builtin_nontemporal_load(p + i);
        acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
    }
    if (acc == 0x9e3779b9u) out[0] = acc;
}

}  // namespace
}  // namespace rmi

using namespace rmi;

extern "C" int rmi_gen_q6_k(void* w, size_t nblocks, uint64_t seed, float d_std, void* stream) {
    if (!aligned4(w)) return fail(RMI_ERR_POINTER, "rmi_gen_q6_k: null or misaligned pointer");
    if (nblocks == 0) return RMI_OK;
    hipLaunchKernelGGL(gen_q6k_kernel, dim3(grid_of(nblocks)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<uint8_t*>(w), nblocks, seed, d_std);
    return launch_status("gen_q6_k");
}

extern "C" int rmi_gen_q8_0(void* w, size_t nblocks, uint64_t seed, float d_std, void* stream) {
    if (!aligned4(w)) return fail(RMI_ERR_POINTER, "rmi_gen_q8_0: null or misaligned pointer");
    if (nblocks == 0) return RMI_OK;
    hipLaunchKernelGGL(gen_q8_0_kernel, dim3(grid_of(nblocks)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<uint8_t*>(w), nblocks, seed, d_std);
    return launch_status("gen_q8_0");
}

extern "C" int rmi_gen_normal(float* out, size_t n, uint64_t seed, float mean, float std, void* stream) {
    if (!aligned4(out)) return fail(RMI_ERR_POINTER, "rmi_gen_normal: null or misaligned pointer");
    if (n == 0) return RMI_OK;
    hipLaunchKernelGGL(gen_normal_kernel, dim3(grid_of(n)), dim3(256), 0, static_cast<hipStream_t>(stream), out, n,
                       seed, mean, std);
    return launch_status("gen_normal");
}

extern "C" int rmi_gen_normal_f16(uint16_t* out, size_t n, uint64_t seed, float mean, float std, void* stream) {
    if (!out || (reinterpret_cast<uintptr_t>(out) & 1u)) return fail(RMI_ERR_POINTER, "rmi_gen_normal_f16: bad pointer");
    if (n == 0) return RMI_OK;
    hipLaunchKernelGGL(gen_normal_f16_kernel, dim3(grid_of(n)), dim3(256), 0, static_cast<hipStream_t>(stream), out,
                       n, seed, mean, std);
    return launch_status("gen_normal_f16");
}

extern "C" int rmi_stream_read(const void* p, size_t bytes, int grid, unsigned* out, void* stream) {
    if (!p || (reinterpret_cast<uintptr_t>(p) & 15u) || bytes % 16 || !aligned4(out))
        return fail(RMI_ERR_POINTER, "rmi_stream_read: 16-byte aligned buffer of whole 16-byte words required");
    if (grid <= 0) return fail(RMI_ERR_SHAPE, "rmi_stream_read: grid must be positive");
    hipLaunchKernelGGL(stream_read_kernel, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const rd_u32x4*>(p), bytes / 16, out);
    return launch_status("stream_read");
}
