/*
 * r9vx_gemv_core.h -- the per-lane pieces of the dequant-fused GEMV shared by
 * the dense GEMV (gemv.hip) and the MoE decode kernels (moe.hip).
 *
 * A lane owns 16-byte payload chunks (32 weights); chunk ci of a row covers
 * K positions klo..klo+15 (low nibbles of its 16 bytes) and khi..khi+15
 * (high nibbles).  Q4_K: byte (j/2)*32+p holds sub-blocks 2g/2g+1
 * (crates/r9v-format/src/ggml.rs:744-790); IQ4_XS: byte 8+16g+(j%16) holds
 * positions j and j+16 of sub-block g (crates/r9v-format/src/iq.rs:274-293).
 */
#ifndef R9VX_GEMV_CORE_H
#define R9VX_GEMV_CORE_H

#include "r9vx_device.h"
#include "r9vx_internal.h"

namespace r9vx {

/* Activation registers of one chunk for one token. */
template <int SCHEME, bool XF32>
struct XChunk;

template <int SCHEME>
struct XChunk<SCHEME, false> {
    uint32_t p[16]; /* bf16 pairs arranged to match the weight decode */
    float slo, shi; /* sum of the 16 low-/high-nibble activations (Q4_K) */
};

template <int SCHEME>
struct XChunk<SCHEME, true> {
    r9vx_f32x4 v[8]; /* v[0..3]: low-nibble positions, v[4..7]: high */
    float slo, shi;
    __device__ __forceinline__ float lo(int i) const { return v[i >> 2][i & 3]; }
    __device__ __forceinline__ float hi(int i) const { return v[4 + (i >> 2)][i & 3]; }
};

/* K offset of byte 0 low nibble / high nibble of chunk ci. */
template <int SCHEME>
__device__ __forceinline__ void chunk_k(uint32_t ci, uint32_t &klo, uint32_t &khi) {
    uint32_t b = ci >> 3, c = ci & 7;
    if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
        klo = 256 * b + 64 * (c >> 1) + 16 * (c & 1);
        khi = klo + 32;
    } else {
        klo = 256 * b + 32 * c;
        khi = klo + 16;
    }
}

/* Raw activation bytes of one chunk for one row: the 16 low- and 16
 * high-nibble K positions (bf16: 2 x 32 bytes, f32: 2 x 64 bytes). */
template <bool XF32>
struct XRaw;
template <>
struct XRaw<false> {
    r9vx_u32x4 v[4];
};
template <>
struct XRaw<true> {
    r9vx_f32x4 v[8];
};

template <bool XF32>
__device__ __forceinline__ void load_x_raw(const void *xbase, uint32_t klo, uint32_t khi, XRaw<XF32> &r) {
    if constexpr (XF32) {
        const r9vx_f32x4 *l4 = reinterpret_cast<const r9vx_f32x4 *>(reinterpret_cast<const float *>(xbase) + klo);
        const r9vx_f32x4 *h4 = reinterpret_cast<const r9vx_f32x4 *>(reinterpret_cast<const float *>(xbase) + khi);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            r.v[i] = l4[i];
            r.v[4 + i] = h4[i];
        }
    } else {
        const r9vx_u32x4 *l4 = reinterpret_cast<const r9vx_u32x4 *>(reinterpret_cast<const uint16_t *>(xbase) + klo);
        const r9vx_u32x4 *h4 = reinterpret_cast<const r9vx_u32x4 *>(reinterpret_cast<const uint16_t *>(xbase) + khi);
        r.v[0] = l4[0];
        r.v[1] = l4[1];
        r.v[2] = h4[0];
        r.v[3] = h4[1];
    }
}

template <int SCHEME, bool XF32>
__device__ __forceinline__ void arrange_x(const XRaw<XF32> &r, XChunk<SCHEME, XF32> &xc) {
    if constexpr (XF32) {
#pragma unroll
        for (int i = 0; i < 8; ++i) xc.v[i] = r.v[i];
        if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
            float slo = 0.f, shi = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                slo += (r.v[i].x + r.v[i].y) + (r.v[i].z + r.v[i].w);
                shi += (r.v[4 + i].x + r.v[4 + i].y) + (r.v[4 + i].z + r.v[4 + i].w);
            }
            xc.slo = slo;
            xc.shi = shi;
        }
    } else {
        uint32_t L[8], H[8];
        L[0] = r.v[0].x; L[1] = r.v[0].y; L[2] = r.v[0].z; L[3] = r.v[0].w;
        L[4] = r.v[1].x; L[5] = r.v[1].y; L[6] = r.v[1].z; L[7] = r.v[1].w;
        H[0] = r.v[2].x; H[1] = r.v[2].y; H[2] = r.v[2].z; H[3] = r.v[2].w;
        H[4] = r.v[3].x; H[5] = r.v[3].y; H[6] = r.v[3].z; H[7] = r.v[3].w;
        if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
            float slo = 0.f, shi = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                slo += __builtin_bit_cast(float, L[j] << 16) + __builtin_bit_cast(float, L[j] & 0xFFFF0000u);
                shi += __builtin_bit_cast(float, H[j] << 16) + __builtin_bit_cast(float, H[j] & 0xFFFF0000u);
            }
            xc.slo = slo;
            xc.shi = shi;
        }
        if constexpr (SCHEME == R9VX_SCHEME_IQ4_XS) {
            /* pair i = {x_lo(i), x_hi(i)}: byte i's two nibbles */
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                xc.p[2 * j] = (L[j] & 0xFFFFu) | (H[j] << 16);
                xc.p[2 * j + 1] = (L[j] >> 16) | (H[j] & 0xFFFF0000u);
            }
        } else {
            /* dword d of the payload holds positions 4d..4d+3:
             * p[4d+0] = {lo(4d), lo(4d+2)}, p[4d+1] = {lo(4d+1), lo(4d+3)},
             * p[4d+2] = {hi(4d), hi(4d+2)}, p[4d+3] = {hi(4d+1), hi(4d+3)} */
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                xc.p[4 * d + 0] = (L[2 * d] & 0xFFFFu) | (L[2 * d + 1] << 16);
                xc.p[4 * d + 1] = (L[2 * d] >> 16) | (L[2 * d + 1] & 0xFFFF0000u);
                xc.p[4 * d + 2] = (H[2 * d] & 0xFFFFu) | (H[2 * d + 1] << 16);
                xc.p[4 * d + 3] = (H[2 * d] >> 16) | (H[2 * d + 1] & 0xFFFF0000u);
            }
        }
    }
}

template <int SCHEME, bool XF32>
__device__ __forceinline__ void load_x(const void *xbase, uint32_t klo, uint32_t khi, XChunk<SCHEME, XF32> &xc) {
    XRaw<XF32> r;
    load_x_raw<XF32>(xbase, klo, khi, r);
    arrange_x<SCHEME, XF32>(r, xc);
}

/* Block header of the chunk's super-block. */
struct Hdr {
    r9vx_u32x4 v;
};

template <int SCHEME>
__device__ __forceinline__ void load_chunk(const uint8_t *row, uint32_t ci, r9vx_u32x4 &qs, Hdr &h) {
    uint32_t b = ci >> 3, c = ci & 7;
    if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
        const uint8_t *blk = row + (uint64_t)b * R9VX_Q4K_BYTES;
        h.v = r9vx_ld128(blk);
        qs = r9vx_ld128_nt(blk + 16 + 16 * c);
    } else {
        const uint8_t *blk = row + (uint64_t)b * R9VX_IQ4XS_BYTES;
        r9vx_u32x2 hh = *reinterpret_cast<const r9vx_u32x2 *>(blk);
        h.v = r9vx_u32x4{hh.x, hh.y, 0u, 0u};
        qs = r9vx_ld128_nt(blk + 8 + 16 * c);
    }
}

/* One chunk of one row against M activation rows: acc[t] += chunk dot. */
/* `m` (<= M, wave-uniform) limits the activation rows that are live. */
template <int SCHEME, bool XF32, int M>
__device__ __forceinline__ void chunk_dot(const r9vx_u32x4 &qs, const Hdr &h, uint32_t c,
                                          const XChunk<SCHEME, XF32> (&xc)[M], float (&acc)[M],
                                          const uint32_t *lut, int m = M) {
    uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
    if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
        float d = r9vx_f16_to_f32((uint16_t)(h.v.x & 0xFFFF));
        float dmin = r9vx_f16_to_f32((uint16_t)(h.v.x >> 16));
        uint32_t sc[2], mn[2];
        r9vx_q4k_scale_pair(h.v, c >> 1, sc, mn);
        float dl0 = d * (float)sc[0], dl1 = d * (float)sc[1];
        float ml0 = dmin * (float)mn[0], ml1 = dmin * (float)mn[1];
        if constexpr (XF32) {
#pragma unroll
            for (int t = 0; t < M; ++t) {
                if (t >= m) break;
                float dlo = 0.f, dhi = 0.f;
#pragma unroll
                for (int dw = 0; dw < 4; ++dw) {
                    uint32_t lo4 = q[dw] & 0x0F0F0F0Fu, hi4 = (q[dw] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        dlo = fmaf((float)((lo4 >> (8 * i)) & 0xFF), xc[t].lo(4 * dw + i), dlo);
                        dhi = fmaf((float)((hi4 >> (8 * i)) & 0xFF), xc[t].hi(4 * dw + i), dhi);
                    }
                }
                acc[t] += dl0 * dlo + dl1 * dhi - (ml0 * xc[t].slo + ml1 * xc[t].shi);
            }
        } else {
            uint32_t v[16];
#pragma unroll
            for (int dw = 0; dw < 4; ++dw) {
                v[4 * dw + 0] = (q[dw] & 0x000F000Fu) | 0x43004300u;
                v[4 * dw + 1] = ((q[dw] >> 8) & 0x000F000Fu) | 0x43004300u;
                v[4 * dw + 2] = ((q[dw] >> 4) & 0x000F000Fu) | 0x43004300u;
                v[4 * dw + 3] = ((q[dw] >> 12) & 0x000F000Fu) | 0x43004300u;
            }
            /* sum (128+q)x = sum qx + 128 sum x; fold the offset into the min. */
            float off0 = fmaf(128.f, dl0, ml0), off1 = fmaf(128.f, dl1, ml1);
#pragma unroll
            for (int t = 0; t < M; ++t) {
                if (t >= m) break;
                float dlo = 0.f, dhi = 0.f;
#pragma unroll
                for (int dw = 0; dw < 4; ++dw) {
                    dlo = r9vx_dot2_bf16(v[4 * dw + 0], xc[t].p[4 * dw + 0], dlo);
                    dlo = r9vx_dot2_bf16(v[4 * dw + 1], xc[t].p[4 * dw + 1], dlo);
                    dhi = r9vx_dot2_bf16(v[4 * dw + 2], xc[t].p[4 * dw + 2], dhi);
                    dhi = r9vx_dot2_bf16(v[4 * dw + 3], xc[t].p[4 * dw + 3], dhi);
                }
                acc[t] += dl0 * dlo + dl1 * dhi - (off0 * xc[t].slo + off1 * xc[t].shi);
            }
        }
    } else {
        float d = r9vx_f16_to_f32((uint16_t)(h.v.x & 0xFFFF));
        float dl = d * r9vx_iq4xs_scale(r9vx_u32x2{h.v.x, h.v.y}, c);
        uint32_t lv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) lv[i] = lut[(q[i >> 2] >> (8 * (i & 3))) & 0xFF];
#pragma unroll
        for (int t = 0; t < M; ++t) {
            if (t >= m) break;
            float s = 0.f;
            if constexpr (XF32) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    s = fmaf(__builtin_bit_cast(float, lv[i] << 16), xc[t].lo(i), s);
                    s = fmaf(__builtin_bit_cast(float, lv[i] & 0xFFFF0000u), xc[t].hi(i), s);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 16; ++i) s = r9vx_dot2_bf16(lv[i], xc[t].p[i], s);
            }
            acc[t] = fmaf(dl, s, acc[t]);
        }
    }
}


/* Sums each of the V values over the `width` lanes of its aligned lane
 * group (width a power of two, 8..64), halving the live values at every
 * butterfly step: the lane whose step bit is set keeps the upper half and
 * sends the lower half, the other keeps the lower half.  Afterwards the lane
 * holds ceil-halved subsets of fully reduced values; owner(i, lane_in_group)
 * tells which original index ends in slot 0..  This costs about 4 ops per
 * value in total instead of 2 per value per step.
 *
 * Returns the number of live slots; idx[s] = original index of slot s. */
template <int V>
__device__ __forceinline__ int reduce_scatter(float (&v)[V], int (&idx)[V], uint32_t lane, int width) {
#pragma unroll
    for (int i = 0; i < V; ++i) idx[i] = i;
    int c = V;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        if (d >= width) continue;
        const bool up = (lane & (uint32_t)d) != 0;
        const int h = c / 2;
#pragma unroll
        for (int i = 0; i < V / 2 + 1; ++i) {
            if (i >= h) break;
            float a = v[i], b = v[i + h];
            float send = up ? a : b;
            float keep = up ? b : a;
            v[i] = keep + __shfl_xor(send, d, 64);
            idx[i] = up ? idx[i + h] : idx[i];
        }
        if (c & 1) { /* odd leftover: reduce it whole, keep it as slot h */
            float a = v[c - 1];
            v[h] = a + __shfl_xor(a, d, 64);
            idx[h] = idx[c - 1];
            c = h + 1;
        } else {
            c = h;
        }
    }
    return c;
}

/* IQ4_XS bf16 codebook-pair table: entry b = {kv[b & 15], kv[b >> 4]}. */
__device__ __forceinline__ void init_iq4_lut(uint32_t *lut, uint32_t tid, uint32_t nthreads) {
    for (uint32_t i = tid; i < 256; i += nthreads) {
        uint32_t lo = __builtin_bit_cast(uint32_t, (float)r9vx_iq4_kvalue(i & 15)) >> 16;
        uint32_t hi = __builtin_bit_cast(uint32_t, (float)r9vx_iq4_kvalue(i >> 4)) >> 16;
        lut[i] = lo | (hi << 16);
    }
}

}  // namespace r9vx

#endif
