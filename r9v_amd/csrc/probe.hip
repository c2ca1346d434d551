/*
 * probe.hip -- ceilings measured on the device itself: a 128-bit streaming
 * read over a buffer and an MFMA-only loop (the MI355X counterpart of the
 * reference's spikes/dot4-gemv and spikes/wmma-l1 measurements).
 */
#include "r9vx_device.h"
#include "r9vx_expf.h"
#include "r9vx_probe.h"

namespace {

/* 128 threads x two 16-byte loads per thread: the fastest of the shapes
 * measured on MI355X for 5.6 MB (2.23 us, against 2.38 us for 256 x 8).
 * The checksum is stored only when it equals a value the fill pattern never
 * produces, so no workgroup writes memory: a store from every workgroup
 * costs ~0.4 us at the end of a launch, which is not part of a read. */
constexpr uint32_t kStreamThreads = 128;
constexpr uint32_t kStreamPerThread = 2;
constexpr uint32_t kStreamNever = 0x9E3779B9u;

__global__ __launch_bounds__(128) void stream_kernel(const r9vx_u32x4 *__restrict__ src, uint64_t n16,
                                                     uint32_t *__restrict__ sink) {
    const uint64_t base = (uint64_t)blockIdx.x * kStreamThreads * kStreamPerThread + threadIdx.x;
    r9vx_u32x4 v[kStreamPerThread];
#pragma unroll
    for (uint32_t i = 0; i < kStreamPerThread; ++i) {
        uint64_t j = base + (uint64_t)i * kStreamThreads;
        v[i] = j < n16 ? __builtin_nontemporal_load(src + j) : r9vx_u32x4{0u, 0u, 0u, 0u};
    }
    uint32_t x = 0;
#pragma unroll
    for (uint32_t i = 0; i < kStreamPerThread; ++i) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    if (x == kStreamNever) sink[blockIdx.x] = x;
}

typedef _Float16 half8 __attribute__((ext_vector_type(8)));

__global__ __launch_bounds__(256) void mfma_kernel(uint32_t iters, float *sink) {
    half8 a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = (_Float16)(0.001f * (threadIdx.x + i));
        b[i] = (_Float16)(0.002f * (blockIdx.x + i));
    }
    r9vx_f32x16 acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
    for (uint32_t it = 0; it < iters; ++it)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[j], 0, 0, 0);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[j][r];
    sink[(uint64_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

/* The three device forms of the routing exp, on the inputs whose bits are
 * first .. first + n - 1, against `want`: bad[f] counts the inputs where
 * form f (0 r9vx_expf, 1 r9vx_expf_tab, 2 r9vx_expf_tab_nb) gives other bits
 * (two NaNs count as equal).  One atomic add per form per workgroup. */
__global__ __launch_bounds__(256) void expf_check_kernel(uint32_t first, uint32_t n, const float *__restrict__ want,
                                                         uint32_t *__restrict__ bad) {
    __shared__ uint64_t tab[R9VX_EXP2F_N];
    __shared__ uint32_t cnt[3];
    r9vx_exp2_fill(tab, threadIdx.x, blockDim.x);
    if (threadIdx.x < 3) cnt[threadIdx.x] = 0;
    __syncthreads();
    uint32_t b[3] = {0, 0, 0};
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const float x = __builtin_bit_cast(float, first + i);
        const float w = want[i];
        const float got[3] = {r9vx_expf(x), r9vx_expf_tab(x, tab), r9vx_expf_tab_nb(x, tab)};
#pragma unroll
        for (int f = 0; f < 3; ++f) {
            const bool same = __builtin_bit_cast(uint32_t, got[f]) == __builtin_bit_cast(uint32_t, w) ||
                              (got[f] != got[f] && w != w);
            b[f] += same ? 0u : 1u;
        }
    }
#pragma unroll
    for (int f = 0; f < 3; ++f)
        if (b[f]) atomicAdd(&cnt[f], b[f]);
    __syncthreads();
    if (threadIdx.x < 3 && cnt[threadIdx.x]) atomicAdd(&bad[threadIdx.x], cnt[threadIdx.x]);
}

}  // namespace

extern "C" {

int r9vx_probe_expf_check_launch(uint32_t first_bits, uint32_t n, const float *want, uint32_t *bad,
                                 r9vx_stream_t stream) {
    if (!want || !bad || n == 0 || (uint64_t)first_bits + n > (1ull << 32)) return R9VX_ERR_INVALID;
    hipLaunchKernelGGL(expf_check_kernel, dim3(1024), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), first_bits,
                       n, want, bad);
    return (int)hipGetLastError();
}

uint32_t r9vx_probe_stream_blocks(uint64_t bytes) {
    uint64_t n16 = bytes / 16;
    return (uint32_t)((n16 + kStreamThreads * kStreamPerThread - 1) / (kStreamThreads * kStreamPerThread));
}

int r9vx_probe_stream_launch(const void *src, uint64_t bytes, uint32_t *sink, r9vx_stream_t stream) {
    if (!src || !sink || bytes % 16 || ((uintptr_t)src & 15)) return R9VX_ERR_INVALID;
    hipLaunchKernelGGL(stream_kernel, dim3(r9vx_probe_stream_blocks(bytes)), dim3(kStreamThreads), 0,
                       reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const r9vx_u32x4 *>(src), bytes / 16,
                       sink);
    return (int)hipGetLastError();
}

int r9vx_probe_mfma_launch(uint32_t blocks, uint32_t iters, float *sink, r9vx_stream_t stream) {
    if (!sink || blocks == 0) return R9VX_ERR_INVALID;
    hipLaunchKernelGGL(mfma_kernel, dim3(blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), iters, sink);
    return (int)hipGetLastError();
}

}  // extern "C"
