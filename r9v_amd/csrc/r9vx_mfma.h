/*
 * r9vx_mfma.h -- building blocks of the dequant-to-LDS MFMA GEMMs (dense
 * prefill matmul and the grouped MoE GEMM).
 *
 * Operand precision: weight tiles are dequantized with the exact T0 formula
 * in f32 (crates/r9v-format/src/ggml.rs:1131-1150, iq.rs:578-598) and rounded
 * once to fp16; activations are bf16 (exact in fp16 after a per-row
 * power-of-two scale that keeps them below 2^15) or f32 rows scaled the same
 * way.  fp16 MFMA runs at the bf16 rate on gfx950 and carries 3 more mantissa
 * bits, which the matmul tolerance needs: bf16-rounded weights put
 * |err| above 1e-3*max|ref| + 2e-3*|ref| on the configs' synthetic weights.
 *
 * Tile: 256 x 256 outputs per 256-thread workgroup (4 waves in 2 x 2, each
 * 128 x 128 = 4 x 4 v_mfma_f32_32x32x16_f16), K step 64 (one Q4_K sub-block
 * pair or two IQ4_XS sub-blocks = 32 payload bytes per weight row), LDS
 * double-buffered: A and B stages of 256 x 64 fp16 (32 KiB each).  LDS rows
 * are 128 bytes of eight 16-byte chunks stored at chunk ^ (row & 7) so that
 * the 32 rows an MFMA operand read touches spread over the banks.
 */
#ifndef R9VX_MFMA_H
#define R9VX_MFMA_H

#include "r9vx_device.h"
#include "r9vx_internal.h"

namespace r9vx {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));

constexpr int kTileM = 256;
constexpr int kTileN = 256;
constexpr int kTileK = 64;
constexpr int kStageHalfs = kTileM * kTileK; /* 16384 fp16 = 32 KiB */

/* LDS byte offset of 16-byte chunk c (0..7) of row r. */
__device__ __forceinline__ uint32_t lds_chunk(uint32_t r, uint32_t c) {
    return r * 128u + ((c ^ (r & 7u)) << 4);
}

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    _Float16 ha = (_Float16)a, hb = (_Float16)b;
    return (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
}

/* Dequantizes the 64 weights of one row for K step `ks` of its super-block
 * (ks = 0..3) into 8 chunks of 8 fp16 (chunk c = K offsets 8c..8c+7).
 *   q0, q1: the two 16-byte payload pieces for this K step
 *   hdr: the block header (Q4_K 16 bytes; IQ4_XS 8 bytes in .x/.y) */
template <int SCHEME>
__device__ __forceinline__ void dequant_row64(r9vx_u32x4 q0, r9vx_u32x4 q1, r9vx_u32x4 hdr, uint32_t ks,
                                              r9vx_u32x4 out[8]) {
    uint32_t b[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
        /* payload bytes 32g..32g+31: low nibble = sub-block 2g position p,
         * high nibble = sub-block 2g+1 position p. */
        float d = r9vx_f16_to_f32((uint16_t)(hdr.x & 0xFFFF));
        float dmin = r9vx_f16_to_f32((uint16_t)(hdr.x >> 16));
        uint32_t sc[2], mn[2];
        r9vx_q4k_scale_pair(hdr, ks, sc, mn);
        float dl0 = d * (float)sc[0], ml0 = dmin * (float)mn[0];
        float dl1 = d * (float)sc[1], ml1 = dmin * (float)mn[1];
        uint32_t lo[16], hi[16];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t w = b[i];
            float l[4], h[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t byte = (w >> (8 * j)) & 0xFFu;
                l[j] = dl0 * (float)(byte & 0xFu) - ml0;
                h[j] = dl1 * (float)(byte >> 4) - ml1;
            }
            lo[2 * i] = pack_h2(l[0], l[1]);
            lo[2 * i + 1] = pack_h2(l[2], l[3]);
            hi[2 * i] = pack_h2(h[0], h[1]);
            hi[2 * i + 1] = pack_h2(h[2], h[3]);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            out[c] = r9vx_u32x4{lo[4 * c], lo[4 * c + 1], lo[4 * c + 2], lo[4 * c + 3]};
            out[4 + c] = r9vx_u32x4{hi[4 * c], hi[4 * c + 1], hi[4 * c + 2], hi[4 * c + 3]};
        }
    } else {
        /* two sub-blocks s = 2ks, 2ks+1; byte p of sub-block s: position p
         * (low nibble) and p+16 (high nibble). */
        float d = r9vx_f16_to_f32((uint16_t)(hdr.x & 0xFFFF));
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            float dl = d * r9vx_iq4xs_scale(r9vx_u32x2{hdr.x, hdr.y}, 2 * ks + s);
            uint32_t lo[8], hi[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t w = b[4 * s + i];
                float l[4], h[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    uint32_t byte = (w >> (8 * j)) & 0xFFu;
                    l[j] = dl * (float)r9vx_iq4_kvalue(byte & 0xFu);
                    h[j] = dl * (float)r9vx_iq4_kvalue(byte >> 4);
                }
                lo[2 * i] = pack_h2(l[0], l[1]);
                lo[2 * i + 1] = pack_h2(l[2], l[3]);
                hi[2 * i] = pack_h2(h[0], h[1]);
                hi[2 * i + 1] = pack_h2(h[2], h[3]);
            }
            out[4 * s + 0] = r9vx_u32x4{lo[0], lo[1], lo[2], lo[3]};
            out[4 * s + 1] = r9vx_u32x4{lo[4], lo[5], lo[6], lo[7]};
            out[4 * s + 2] = r9vx_u32x4{hi[0], hi[1], hi[2], hi[3]};
            out[4 * s + 3] = r9vx_u32x4{hi[4], hi[5], hi[6], hi[7]};
        }
    }
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

/* Per-row power-of-two scale that keeps max|row| * 2^-e below 2^15 (exact). */
__device__ __forceinline__ int row_shift(float maxabs) {
    if (!(maxabs >= 32768.0f)) return 0;
    int e = 0;
    (void)frexpf(maxabs, &e); /* maxabs = f * 2^e, f in [0.5, 1) */
    return e - 15;
}

}  // namespace r9vx

/* bf16 rows -> fp16 rows with a per-row power-of-two scale (gemm.hip). */
int r9vx_launch_x_to_f16(const uint16_t *x, uint32_t m, uint32_t k, _Float16 *x16, float *scale,
                         hipStream_t stream);

#endif
