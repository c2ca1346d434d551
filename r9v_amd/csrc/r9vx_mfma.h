/*
 * r9vx_mfma.h -- building blocks of the MFMA dequant-GEMMs (dense prefill
 * matmul and the grouped MoE GEMMs, both on the r9vx_mma3.h loop).
 *
 * Operand precision: weight tiles are dequantized with the exact T0 formula
 * in f32 (crates/r9v-format/src/ggml.rs:1131-1150, iq.rs:578-598) and rounded
 * once to fp16; activations are bf16 (exact in fp16 after a per-row
 * power-of-two scale that keeps them below 2^15) or f32 rows scaled the same
 * way.  fp16 MFMA runs at the bf16 rate on gfx950 and carries 3 more mantissa
 * bits, which the matmul tolerance needs: bf16-rounded weights put
 * |err| above 1e-3*max|ref| + 2e-3*|ref| on the configs' synthetic weights.
 */
#ifndef R9VX_MFMA_H
#define R9VX_MFMA_H

#include "r9vx_device.h"
#include "r9vx_internal.h"

namespace r9vx {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));

constexpr int kTileK = 64; /* K step: one Q4_K sub-block pair, two IQ4_XS sub-blocks */

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    _Float16 ha = (_Float16)a, hb = (_Float16)b;
    return (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
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
 * perm_scheme = a K order (r9vx_group_order of a weight scheme) the rows are
 * stored in that order (r9vx_x16.h order_pos), with 0 in natural order. */
int r9vx_launch_x_to_f16(const uint16_t *x, uint32_t m, uint32_t k, _Float16 *x16, float *scale,
                         uint32_t perm_scheme, hipStream_t stream);

#endif
