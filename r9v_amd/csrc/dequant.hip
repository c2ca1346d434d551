/*
 * dequant.hip -- bit-exact GGUF Q4_K / IQ4_XS decode to f32, and load-time
 * scale validation.
 *
 * Q4_K: crates/r9v-format/src/ggml.rs:744-790 (nibble order) and :1131-1150
 *   (w = (d*sc)*q - (dmin*mn), each product rounded, then the subtraction).
 * IQ4_XS: crates/r9v-format/src/iq.rs:578-598 (w = (d*(s-32))*kv[q]).
 * The library is compiled with -ffp-contract=off, so the multiply and the
 * subtract round separately exactly as the Rust source does.
 *
 * One thread decodes one 16-byte payload chunk (32 weights): a 64-lane wave
 * reads 1 KiB of contiguous payload with 128-bit loads and writes 8 KiB of
 * f32 with 128-bit stores.
 */
#include "r9vx_device.h"
#include "r9vx_internal.h"

namespace {

__device__ __forceinline__ void store16(float *dst, const float *v) {
    r9vx_f32x4 *d4 = reinterpret_cast<r9vx_f32x4 *>(dst);
#pragma unroll
    for (int i = 0; i < 4; ++i) d4[i] = r9vx_f32x4{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
}

template <int SCHEME>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t *__restrict__ wire,
                                                      uint64_t n_chunks,
                                                      float *__restrict__ out) {
    uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= n_chunks) return;
    const uint64_t blk = gid >> 3;
    const uint32_t c = (uint32_t)(gid & 7);
    float lo[16], hi[16];
    if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
        const uint8_t *b = wire + blk * R9VX_Q4K_BYTES;
        r9vx_u32x4 hdr = r9vx_ld128(b);
        r9vx_u32x4 qs = r9vx_ld128(b + 16 + 16 * c);
        float d = r9vx_f16_to_f32((uint16_t)(hdr.x & 0xFFFF));
        float dmin = r9vx_f16_to_f32((uint16_t)(hdr.x >> 16));
        uint32_t g = c >> 1;
        uint32_t sc[2], mn[2];
        r9vx_q4k_scale_pair(hdr, g, sc, mn);
        float dl0 = d * (float)sc[0], ml0 = dmin * (float)mn[0];
        float dl1 = d * (float)sc[1], ml1 = dmin * (float)mn[1];
        uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
#pragma unroll
        for (int p = 0; p < 16; ++p) {
            uint32_t byte = (q[p >> 2] >> ((p & 3) * 8)) & 0xFF;
            lo[p] = dl0 * (float)(byte & 0xF) - ml0;
            hi[p] = dl1 * (float)(byte >> 4) - ml1;
        }
        float *o = out + blk * 256;
        uint32_t pos = 16 * (c & 1);
        store16(o + 32 * (2 * g) + pos, lo);
        store16(o + 32 * (2 * g + 1) + pos, hi);
    } else {
        const uint8_t *b = wire + blk * R9VX_IQ4XS_BYTES;
        r9vx_u32x2 hdr = *reinterpret_cast<const r9vx_u32x2 *>(b);
        r9vx_u32x4 qs = r9vx_ld128(b + 8 + 16 * c);
        float d = r9vx_f16_to_f32((uint16_t)(hdr.x & 0xFFFF));
        float dl = d * r9vx_iq4xs_scale(hdr, c);
        uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
#pragma unroll
        for (int p = 0; p < 16; ++p) {
            uint32_t byte = (q[p >> 2] >> ((p & 3) * 8)) & 0xFF;
            lo[p] = dl * (float)r9vx_iq4_kvalue(byte & 0xF);
            hi[p] = dl * (float)r9vx_iq4_kvalue(byte >> 4);
        }
        float *o = out + blk * 256 + 32 * c;
        store16(o, lo);
        store16(o + 16, hi);
    }
}

template <int SCHEME>
__global__ __launch_bounds__(256) void validate_kernel(const uint8_t *__restrict__ wire,
                                                       uint64_t n_blocks, uint32_t *bad) {
    uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t isbad = 0;
    if (gid < n_blocks) {
        const uint32_t bb = SCHEME == R9VX_SCHEME_Q4_K ? R9VX_Q4K_BYTES : R9VX_IQ4XS_BYTES;
        uint32_t w = *reinterpret_cast<const uint32_t *>(wire + gid * bb);
        /* f16 exponent all ones = inf / nan (check_wire_f16, ggml.rs:421-445). */
        isbad = ((w & 0x7C00u) == 0x7C00u) ? 1u : 0u;
        if (SCHEME == R9VX_SCHEME_Q4_K) isbad |= ((w & 0x7C000000u) == 0x7C000000u) ? 1u : 0u;
    }
    uint64_t mask = __ballot(isbad);
    if ((threadIdx.x & 63) == 0 && mask) atomicAdd(bad, (uint32_t)__popcll(mask));
}

}  // namespace

int r9vx_launch_dequant(uint32_t scheme, const uint8_t *wire, uint32_t n_rows, uint32_t k,
                        float *out, hipStream_t stream) {
    uint64_t n_chunks = (uint64_t)n_rows * (k / 256) * 8;
    dim3 grid((unsigned)((n_chunks + 255) / 256));
    if (scheme == R9VX_SCHEME_Q4_K)
        hipLaunchKernelGGL(dequant_kernel<R9VX_SCHEME_Q4_K>, grid, dim3(256), 0, stream, wire, n_chunks, out);
    else
        hipLaunchKernelGGL(dequant_kernel<R9VX_SCHEME_IQ4_XS>, grid, dim3(256), 0, stream, wire, n_chunks, out);
    return (int)hipGetLastError();
}

int r9vx_launch_validate(uint32_t scheme, const uint8_t *wire, uint32_t n_rows, uint32_t k,
                         uint32_t *bad, hipStream_t stream) {
    uint64_t n_blocks = (uint64_t)n_rows * (k / 256);
    dim3 grid((unsigned)((n_blocks + 255) / 256));
    if (scheme == R9VX_SCHEME_Q4_K)
        hipLaunchKernelGGL(validate_kernel<R9VX_SCHEME_Q4_K>, grid, dim3(256), 0, stream, wire, n_blocks, bad);
    else
        hipLaunchKernelGGL(validate_kernel<R9VX_SCHEME_IQ4_XS>, grid, dim3(256), 0, stream, wire, n_blocks, bad);
    return (int)hipGetLastError();
}
