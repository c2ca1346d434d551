/*
 * r9vx_mfma.h -- building blocks of the MFMA dequant-GEMMs (dense prefill
 * matmul and the grouped MoE GEMMs).
 *
 * Operand precision: weight tiles are dequantized with the exact T0 formula
 * in f32 (crates/r9v-format/src/ggml.rs:1131-1150, iq.rs:578-598) and rounded
 * once to fp16; activations are bf16 (exact in fp16 after a per-row
 * power-of-two scale that keeps them below 2^15) or f32 rows scaled the same
 * way.  fp16 MFMA runs at the bf16 rate on gfx950 and carries 3 more mantissa
 * bits, which the matmul tolerance needs: bf16-rounded weights put
 * |err| above 1e-3*max|ref| + 2e-3*|ref| on the configs' synthetic weights.
 *
 * Two main loops build on these pieces: r9vx_mma.h dequantizes weights into
 * LDS (small dense tiles), r9vx_mma2.h decodes them straight into MFMA B
 * operands in registers (large dense tiles and the grouped MoE GEMMs).
 */
#ifndef R9VX_MFMA_H
#define R9VX_MFMA_H

#include "r9vx_device.h"
#include "r9vx_internal.h"

namespace r9vx {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));

constexpr int kTileK = 64; /* K step: one Q4_K sub-block pair, two IQ4_XS sub-blocks */

/* LDS byte offset of 16-byte chunk c (0..7) of row r. */
__device__ __forceinline__ uint32_t lds_chunk(uint32_t r, uint32_t c) {
    return r * 128u + ((c ^ (r & 7u)) << 4);
}

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    _Float16 ha = (_Float16)a, hb = (_Float16)b;
    return (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
}

/* Payload and header of one weight row for K step kt (global K offset 64*kt). */
template <int SCHEME>
__device__ __forceinline__ void load_w64(const uint8_t *row, uint32_t kt, r9vx_u32x4 &q0, r9vx_u32x4 &q1,
                                         r9vx_u32x4 &hdr) {
    uint32_t blk = kt >> 2, ks = kt & 3;
    if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
        const uint8_t *b = row + (uint64_t)blk * R9VX_Q4K_BYTES;
        hdr = r9vx_ld128(b);
        q0 = r9vx_ld128(b + 16 + 32 * ks);
        q1 = r9vx_ld128(b + 32 + 32 * ks);
    } else {
        const uint8_t *b = row + (uint64_t)blk * R9VX_IQ4XS_BYTES;
        r9vx_u32x2 h = *reinterpret_cast<const r9vx_u32x2 *>(b);
        hdr = r9vx_u32x4{h.x, h.y, 0u, 0u};
        q0 = r9vx_ld128(b + 8 + 32 * ks);
        q1 = r9vx_ld128(b + 24 + 32 * ks);
    }
}

/* IQ4_XS f32 codebook pairs: entry b = {kv[b & 15], kv[b >> 4]}. */
__device__ __forceinline__ void init_iq4_lut_f32(r9vx_f32x4 *lut2 /* 128 x (2 pairs) */, uint32_t tid) {
    if (tid < 128) {
        uint32_t b0 = 2 * tid, b1 = 2 * tid + 1;
        lut2[tid] = r9vx_f32x4{(float)r9vx_iq4_kvalue(b0 & 15), (float)r9vx_iq4_kvalue(b0 >> 4),
                               (float)r9vx_iq4_kvalue(b1 & 15), (float)r9vx_iq4_kvalue(b1 >> 4)};
    }
}

/* Per-row power-of-two scale that keeps max|row| * 2^-e below 2^15 (exact). */
__device__ __forceinline__ int row_shift(float maxabs) {
    if (!(maxabs >= 32768.0f)) return 0;
    int e = 0;
    (void)frexpf(maxabs, &e); /* maxabs = f * 2^e, f in [0.5, 1) */
    return e - 15;
}

}  // namespace r9vx

/* bf16 rows -> fp16 rows with a per-row power-of-two scale (gemm.hip); with
 * perm_scheme = a weight scheme the rows are stored in that scheme's K group
 * order (r9vx_mma2.h), with 0 in natural order. */
int r9vx_launch_x_to_f16(const uint16_t *x, uint32_t m, uint32_t k, _Float16 *x16, float *scale,
                         uint32_t perm_scheme, hipStream_t stream);

#endif
