/*
 * dequant.hip -- bit-exact GGUF Q4_K / IQ4_XS / Q8_0 / Q6_K decode to f32,
 * load-time scale validation, and the Q8_0 / Q6_K split repack.
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

/* ------------------------------------------------------------------------
 * Q8_0 and Q6_K: wire decode (bit-exact), scale validation, and the
 * load-time split into the device layout the GEMV reads.  Wire blocks of 34
 * and 210 bytes are only 2-byte aligned, so these kernels read them as
 * 16-bit words; they run once per weight load, not per matmul.
 * ---------------------------------------------------------------------- */
namespace {

__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p) { return *reinterpret_cast<const uint16_t *>(p); }

/* Q8_0: one thread per block; w = d * (i8)v (crates/r9v-format/src/ggml.rs:1094-1100). */
__global__ __launch_bounds__(256) void dequant_q80_kernel(const uint8_t *__restrict__ wire, uint64_t n_blocks,
                                                          float *__restrict__ out) {
    const uint64_t blk = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= n_blocks) return;
    const uint8_t *b = wire + blk * R9VX_Q80_BYTES;
    const float d = r9vx_f16_to_f32((uint16_t)ld_u16(b));
    float v[32];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t two = ld_u16(b + 2 + 2 * i);
        v[2 * i] = d * (float)(int8_t)(two & 0xFF);
        v[2 * i + 1] = d * (float)(int8_t)(two >> 8);
    }
    store16(out + blk * 32, v);
    store16(out + blk * 32 + 16, v + 16);
}

/* Q6_K: one thread per group j of 16 weights; weight i of the block takes its
 * low nibble from byte (i/128)*64 + i%64 (nibble (i%128)/64) and its high
 * bits from byte 128 + (i/128)*32 + i%32 (pair (i%128)/32), then
 * w = (d * (i8)scales[j]) * (q - 32)  (ggml.rs:817-850, 1154-1172). */
__global__ __launch_bounds__(256) void dequant_q6k_kernel(const uint8_t *__restrict__ wire, uint64_t n_groups,
                                                          float *__restrict__ out) {
    const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= n_groups) return;
    const uint64_t blk = gid >> 4;
    const uint32_t j = (uint32_t)(gid & 15);
    const uint8_t *b = wire + blk * R9VX_Q6K_BYTES;
    const float d = r9vx_f16_to_f32((uint16_t)ld_u16(b + 208));
    const uint32_t scw = ld_u16(b + 192 + (j & ~1u));
    const float dl = d * (float)(int8_t)((scw >> (8 * (j & 1))) & 0xFF);
    const uint32_t i0 = 16 * j, half = i0 / 128, r = i0 % 128;
    const uint8_t *ql = b + half * 64 + r % 64;
    const uint8_t *qh = b + 128 + half * 32 + r % 32;
    const uint32_t nib = 4 * (r / 64), pair = 2 * (r / 32);
    float v[16];
#pragma unroll
    for (int p = 0; p < 16; p += 2) {
        const uint32_t l2 = ld_u16(ql + p), h2 = ld_u16(qh + p);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const uint32_t lo = (l2 >> (8 * e + nib)) & 0xF, hi = (h2 >> (8 * e + pair)) & 0x3;
            v[p + e] = dl * ((float)(lo | (hi << 4)) - 32.0f);
        }
    }
    store16(out + blk * 256 + i0, v);
}

/* IQ3_S: one thread per group g of 32 weights (crates/r9v-format/src/iq.rs:
 * 698-722): db = d * (1 + 2 s) with s = nibble g%2 of scales[g/2]; index i
 * of the group takes grid entry qs[8g+i] | (bit i of qh[g]) << 8, and weight
 * 4i + b is db * grid[b], negated when bit 4(i%2) + b of signs[4g + i/2] is
 * set. */
__global__ __launch_bounds__(256) void dequant_iq3s_kernel(const uint8_t *__restrict__ wire, uint64_t n_groups,
                                                           float *__restrict__ out) {
    const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= n_groups) return;
    const uint64_t blk = gid >> 3;
    const uint32_t g = (uint32_t)(gid & 7);
    const uint8_t *b = wire + blk * R9VX_IQ3S_BYTES;
    const float d = r9vx_f16_to_f32((uint16_t)ld_u16(b));
    /* scales[g/2] is byte (g/2)%2 of the 16-bit word at 106 + 2(g/4) */
    const uint32_t s = (ld_u16(b + 106 + 2 * (g >> 2)) >> (8 * ((g >> 1) & 1) + 4 * (g & 1))) & 0xF;
    const float db = d * (1.0f + 2.0f * (float)s);
    const uint32_t qh = (ld_u16(b + 66 + (g & ~1u)) >> (8 * (g & 1))) & 0xFF;
    const uint32_t sg = ld_u16(b + 74 + 4 * g) | (ld_u16(b + 76 + 4 * g) << 16); /* bit v signs weight v */
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
        const uint32_t two = ld_u16(b + 2 + 8 * g + i);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const uint32_t idx = ((two >> (8 * e)) & 0xFF) | (((qh >> (i + e)) & 1u) << 8);
            const uint32_t gw = kIq3sGrid[idx];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint32_t w = 4 * (i + e) + c;
                const float m = db * (float)((gw >> (8 * c)) & 0xFF);
                v[w] = ((sg >> w) & 1u) ? m * -1.0f : m;
            }
        }
    }
    store16(out + blk * 256 + 32 * g, v);
    store16(out + blk * 256 + 32 * g + 16, v + 16);
}

/* Non-finite d (check_wire_f16, ggml.rs:421-445) of Q8_0 / Q6_K / IQ3_S wire blocks. */
__global__ __launch_bounds__(256) void validate_split_kernel(const uint8_t *__restrict__ wire, uint64_t n_blocks,
                                                             uint32_t block_bytes, uint32_t d_offset,
                                                             uint32_t *bad) {
    const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t isbad = 0;
    if (gid < n_blocks) isbad = (ld_u16(wire + gid * block_bytes + d_offset) & 0x7C00u) == 0x7C00u;
    const uint64_t mask = __ballot(isbad);
    if ((threadIdx.x & 63) == 0 && mask) atomicAdd(bad, (uint32_t)__popcll(mask));
}

/* Wire -> split layout.  Q8_0: thread per block, the 32 quants to body
 * [blk*32, +32) and d to scales[blk].  Q6_K: thread per 16-byte piece of the
 * 208-byte body (13 per block); piece 0 also moves d. */
__global__ __launch_bounds__(256) void repack_q80_kernel(const uint8_t *__restrict__ wire, uint64_t n_blocks,
                                                         uint8_t *__restrict__ body, uint16_t *__restrict__ scales) {
    const uint64_t blk = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= n_blocks) return;
    const uint8_t *b = wire + blk * R9VX_Q80_BYTES;
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = ld_u16(b + 2 + 4 * i) | (ld_u16(b + 4 + 4 * i) << 16);
    r9vx_u32x4 *o = reinterpret_cast<r9vx_u32x4 *>(body + blk * 32);
    o[0] = r9vx_u32x4{w[0], w[1], w[2], w[3]};
    o[1] = r9vx_u32x4{w[4], w[5], w[6], w[7]};
    scales[blk] = (uint16_t)ld_u16(b);
}

__global__ __launch_bounds__(256) void repack_q6k_kernel(const uint8_t *__restrict__ wire, uint64_t n_pieces,
                                                         uint8_t *__restrict__ body, uint16_t *__restrict__ scales) {
    const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= n_pieces) return;
    const uint64_t blk = gid / 13;
    const uint32_t piece = (uint32_t)(gid % 13);
    const uint8_t *b = wire + blk * R9VX_Q6K_BYTES + 16 * piece;
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = ld_u16(b + 4 * i) | (ld_u16(b + 4 * i + 2) << 16);
    *reinterpret_cast<r9vx_u32x4 *>(body + blk * R9VX_Q6K_BODY + 16 * piece) = r9vx_u32x4{w[0], w[1], w[2], w[3]};
    if (piece == 0) scales[blk] = (uint16_t)ld_u16(wire + blk * R9VX_Q6K_BYTES + 208);
}

/* Wire -> IQ3_S device block: thread per 16-byte piece of the 112-byte
 * block (7 per block); device byte j takes wire byte 2 + j (qs, j < 64),
 * 10 + j (signs, j < 96), j - 30 (qh, j < 104), j + 2 (scales, j < 108),
 * j - 108 (d, j < 110), and zero. */

__global__ __launch_bounds__(256) void repack_iq3s_kernel(const uint8_t *__restrict__ wire, uint64_t n_pieces,
                                                          uint8_t *__restrict__ body) {
    const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= n_pieces) return;
    const uint64_t blk = gid / 7;
    const uint32_t piece = (uint32_t)(gid % 7);
    const uint8_t *b = wire + blk * R9VX_IQ3S_BYTES;
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t j = 16 * piece + i;
        if (j < 110) w[i >> 2] |= (uint32_t)b[r9vx_iq3s_wire_byte(j)] << (8 * (i & 3));
    }
    *reinterpret_cast<r9vx_u32x4 *>(body + blk * R9VX_IQ3S_DEV_BYTES + 16 * piece) = r9vx_u32x4{w[0], w[1], w[2], w[3]};
}

}  // namespace

int r9vx_launch_dequant_split(uint32_t scheme, const uint8_t *wire, uint32_t n_rows, uint32_t k, float *out,
                              hipStream_t stream) {
    if (scheme == R9VX_SCHEME_IQ3_S) {
        const uint64_t n = (uint64_t)n_rows * (k / 256) * 8;
        hipLaunchKernelGGL(dequant_iq3s_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, wire, n, out);
    } else if (scheme == R9VX_SCHEME_Q8_0) {
        const uint64_t n = (uint64_t)n_rows * (k / 32);
        hipLaunchKernelGGL(dequant_q80_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, wire, n, out);
    } else {
        const uint64_t n = (uint64_t)n_rows * (k / 256) * 16;
        hipLaunchKernelGGL(dequant_q6k_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, wire, n, out);
    }
    return (int)hipGetLastError();
}

int r9vx_launch_validate_split(uint32_t scheme, const uint8_t *wire, uint32_t n_rows, uint32_t k, uint32_t *bad,
                               hipStream_t stream) {
    const bool q8 = scheme == R9VX_SCHEME_Q8_0, iq3 = scheme == R9VX_SCHEME_IQ3_S;
    const uint64_t n = (uint64_t)n_rows * (k / (q8 ? 32 : 256));
    hipLaunchKernelGGL(validate_split_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, wire, n,
                       (uint32_t)(q8 ? R9VX_Q80_BYTES : iq3 ? R9VX_IQ3S_BYTES : R9VX_Q6K_BYTES),
                       (q8 || iq3) ? 0u : 208u, bad);
    return (int)hipGetLastError();
}

int r9vx_launch_repack(uint32_t scheme, const uint8_t *wire, uint32_t n_rows, uint32_t k, uint8_t *body,
                       uint16_t *scales, hipStream_t stream) {
    if (scheme == R9VX_SCHEME_IQ3_S) {
        const uint64_t n = (uint64_t)n_rows * (k / 256) * 7;
        hipLaunchKernelGGL(repack_iq3s_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, wire, n, body);
    } else if (scheme == R9VX_SCHEME_Q8_0) {
        const uint64_t n = (uint64_t)n_rows * (k / 32);
        hipLaunchKernelGGL(repack_q80_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, wire, n,
                           body, scales);
    } else {
        const uint64_t n = (uint64_t)n_rows * (k / 256) * 13;
        hipLaunchKernelGGL(repack_q6k_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, wire, n,
                           body, scales);
    }
    return (int)hipGetLastError();
}
