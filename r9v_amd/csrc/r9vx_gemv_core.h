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
    } else if constexpr (SCHEME == R9VX_SCHEME_Q6_K) {
        /* chunk = 16 ql bytes of half c/4: low nibbles at 128h + 16(c%4),
         * high nibbles 64 further */
        klo = 256 * b + 128 * (c >> 2) + 16 * (c & 3);
        khi = klo + 64;
    } else if constexpr (SCHEME == R9VX_SCHEME_Q8_0) {
        /* chunk = one Q8_0 block of 32 quants */
        klo = 32 * ci;
        khi = klo + 16;
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
        if constexpr (SCHEME == R9VX_SCHEME_IQ3_S) {
            /* natural order: p[j] = positions 2j, 2j+1 of the 32 */
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                xc.p[j] = L[j];
                xc.p[8 + j] = H[j];
            }
        } else if constexpr (SCHEME == R9VX_SCHEME_IQ4_XS) {
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
            /* sums of the 16 low- and 16 high-position activations (the
             * min and 128-offset terms): dot products with the bf16 pair
             * (1, 1), two activations per instruction */
            constexpr uint32_t kOnes = 0x3F803F80u;
            float slo = 0.f, shi = 0.f;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                slo = r9vx_dot2_bf16(xc.p[4 * d + 0], kOnes, slo);
                slo = r9vx_dot2_bf16(xc.p[4 * d + 1], kOnes, slo);
                shi = r9vx_dot2_bf16(xc.p[4 * d + 2], kOnes, shi);
                shi = r9vx_dot2_bf16(xc.p[4 * d + 3], kOnes, shi);
            }
            xc.slo = slo;
            xc.shi = shi;
        }
    }
}

template <int SCHEME, bool XF32>
__device__ __forceinline__ void load_x(const void *xbase, uint32_t klo, uint32_t khi, XChunk<SCHEME, XF32> &xc) {
    XRaw<XF32> r;
    load_x_raw<XF32>(xbase, klo, khi, r);
    arrange_x<SCHEME, XF32>(r, xc);
}

/* Block header of the chunk's super-block; `e` holds the f16 d of the
 * split-layout schemes (Q8_0 / Q6_K), whose d lives in a separate array. */
struct Hdr {
    r9vx_u32x4 v;
    uint32_t e;
};

/* The payload and the header of a block share cache lines, so both take the
 * same path: a non-temporal payload load beside a cached header load of the
 * same line measured 4.0 TB/s on the configs[3] expert set against 5.2 TB/s
 * for cached loads (a plain 16-byte stream: 5.6).  NT: both non-temporal --
 * the one-shot GEMV's form (configs[1] M = 1: 4.14 -> 3.55 us, M = 5: 5.26 ->
 * 4.75, configs[0] 5.24 -> 4.89, same box); the streaming form and the MoE
 * decode GEMVs keep cached loads (streaming Q4_K 32768 x 4096: 16.0 -> 17.5
 * us with NT; configs[3] unchanged). */
template <int SCHEME, bool NT = false>
__device__ __forceinline__ void load_chunk(const uint8_t *row, uint32_t ci, r9vx_u32x4 &qs, Hdr &h) {
    uint32_t b = ci >> 3, c = ci & 7;
    if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
        const uint8_t *blk = row + (uint64_t)b * R9VX_Q4K_BYTES;
        h.v = NT ? r9vx_ld128_nt(blk) : r9vx_ld128(blk);
        qs = NT ? r9vx_ld128_nt(blk + 16 + 16 * c) : r9vx_ld128(blk + 16 + 16 * c);
    } else {
        const uint8_t *blk = row + (uint64_t)b * R9VX_IQ4XS_BYTES;
        typedef uint32_t u32x2a4 __attribute__((ext_vector_type(2), aligned(4)));
        const u32x2a4 hh = NT ? __builtin_nontemporal_load(reinterpret_cast<const u32x2a4 *>(blk))
                              : *reinterpret_cast<const u32x2a4 *>(blk);
        h.v = r9vx_u32x4{hh.x, hh.y, 0u, 0u};
        qs = NT ? r9vx_ld128_nt(blk + 8 + 16 * c) : r9vx_ld128(blk + 8 + 16 * c);
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
        const uint32_t sm = r9vx_q4k_pair_bytes(h.v, c >> 1);
        float dl0 = d * (float)(sm & 0xFFu), dl1 = d * (float)((sm >> 8) & 0xFFu);
        float ml0 = dmin * (float)((sm >> 16) & 0xFFu), ml1 = dmin * (float)(sm >> 24);
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
                v[4 * dw + 0] = r9vx_and_or(q[dw], 0x000F000Fu, 0x43004300u);
                v[4 * dw + 1] = r9vx_and_or(q[dw] >> 8, 0x000F000Fu, 0x43004300u);
                v[4 * dw + 2] = r9vx_and_or(q[dw] >> 4, 0x000F000Fu, 0x43004300u);
                v[4 * dw + 3] = r9vx_and_or(q[dw] >> 12, 0x000F000Fu, 0x43004300u);
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


/* ---- Q8_0 / Q6_K in the split device layout ---------------------------------
 *
 * A chunk is 32 weights here too, but 32 payload bytes: Q8_0 reads one
 * block's quants (body row = int8 [K]), Q6_K reads 16 ql bytes and the 16 qh
 * bytes holding their high bits (body row = K/256 blocks of 208 bytes:
 * ql 128, qh 64, scales 16).  d comes from the f16 scale row.  The
 * activations use the Q4_K arrangement (pairs of positions 4d+{0,2} and
 * 4d+{1,3}, plus the sums of the 16 low and 16 high positions). */
struct Payload2 {
    r9vx_u32x4 a, b;
};

template <int SCHEME>
__device__ __forceinline__ void load_chunk_split(const uint8_t *row, const uint16_t *srow, uint32_t ci,
                                                 Payload2 &p, Hdr &h) {
    if constexpr (SCHEME == R9VX_SCHEME_Q8_0) {
        p.a = r9vx_ld128_nt(row + 32 * (uint64_t)ci);
        p.b = r9vx_ld128_nt(row + 32 * (uint64_t)ci + 16);
        h.e = srow[ci];
    } else {
        const uint32_t b = ci >> 3, c = ci & 7;
        const uint8_t *blk = row + (uint64_t)b * R9VX_Q6K_BODY;
        p.a = r9vx_ld128(blk + 64 * (c >> 2) + 16 * (c & 3));                /* ql */
        p.b = r9vx_ld128(blk + 128 + 32 * (c >> 2) + 16 * (c & 1));          /* qh */
        h.v = r9vx_ld128(blk + 192);                                        /* 16 int8 scales */
        h.e = srow[b];
    }
}

/* One split-layout chunk of one row against M bf16 activation rows. */
template <int SCHEME, int M>
__device__ __forceinline__ void chunk_dot_split(const Payload2 &pl, const Hdr &h, uint32_t c,
                                                const XChunk<SCHEME, false> (&xc)[M], float (&acc)[M], int m = M) {
    const float d = r9vx_f16_to_f32((uint16_t)h.e);
    if constexpr (SCHEME == R9VX_SCHEME_Q8_0) {
        /* u = q + 128 (bytes XOR 0x80) = 16*hi + lo; 0x4300|n is the bf16 of
         * 128 + n, so sl = sum (128+lo) x and sh = sum (128+hi) x give
         * sum q x = 16 sh + sl - 2304 sum x. */
        const uint32_t q[8] = {pl.a.x, pl.a.y, pl.a.z, pl.a.w, pl.b.x, pl.b.y, pl.b.z, pl.b.w};
        uint32_t L[16], H[16];
#pragma unroll
        for (int dw = 0; dw < 8; ++dw) {
            const uint32_t u = q[dw] ^ 0x80808080u;
            L[2 * dw + 0] = (u & 0x000F000Fu) | 0x43004300u;
            L[2 * dw + 1] = ((u >> 8) & 0x000F000Fu) | 0x43004300u;
            H[2 * dw + 0] = ((u >> 4) & 0x000F000Fu) | 0x43004300u;
            H[2 * dw + 1] = ((u >> 12) & 0x000F000Fu) | 0x43004300u;
        }
#pragma unroll
        for (int t = 0; t < M; ++t) {
            if (t >= m) break;
            float sl = 0.f, sh = 0.f;
#pragma unroll
            for (int dw = 0; dw < 4; ++dw) {
                /* first 16 bytes: low positions; last 16: high positions */
                sl = r9vx_dot2_bf16(L[2 * dw + 0], xc[t].p[4 * dw + 0], sl);
                sl = r9vx_dot2_bf16(L[2 * dw + 1], xc[t].p[4 * dw + 1], sl);
                sh = r9vx_dot2_bf16(H[2 * dw + 0], xc[t].p[4 * dw + 0], sh);
                sh = r9vx_dot2_bf16(H[2 * dw + 1], xc[t].p[4 * dw + 1], sh);
                sl = r9vx_dot2_bf16(L[8 + 2 * dw + 0], xc[t].p[4 * dw + 2], sl);
                sl = r9vx_dot2_bf16(L[8 + 2 * dw + 1], xc[t].p[4 * dw + 3], sl);
                sh = r9vx_dot2_bf16(H[8 + 2 * dw + 0], xc[t].p[4 * dw + 2], sh);
                sh = r9vx_dot2_bf16(H[8 + 2 * dw + 1], xc[t].p[4 * dw + 3], sh);
            }
            acc[t] = fmaf(d, fmaf(16.f, sh, sl) - 2304.f * (xc[t].slo + xc[t].shi), acc[t]);
        }
    } else {
        /* 6-bit q = ql nibble | (qh bit pair << 4); low positions take pair
         * (c%4)/2, high positions pair 2 + (c%4)/2, and scales 8h + c%4 and
         * 8h + 4 + c%4 (h = c/4).  0x4300|q is the bf16 of 128 + q, so
         * sum (q - 32) x = sum (128 + q) x - 160 sum x. */
        const uint32_t cc = c & 3, hsel = c >> 2;
        const uint32_t j0 = 8 * hsel + cc, j1 = j0 + 4;
        const uint32_t sv[4] = {h.v.x, h.v.y, h.v.z, h.v.w};
        const float dl0 = d * (float)(int8_t)((sv[j0 >> 2] >> (8 * (j0 & 3))) & 0xFF);
        const float dl1 = d * (float)(int8_t)((sv[j1 >> 2] >> (8 * (j1 & 3))) & 0xFF);
        const uint32_t pair_lo = 2 * (cc >> 1), pair_hi = pair_lo + 4;
        const uint32_t ql[4] = {pl.a.x, pl.a.y, pl.a.z, pl.a.w};
        const uint32_t qh[4] = {pl.b.x, pl.b.y, pl.b.z, pl.b.w};
        uint32_t v[16];
#pragma unroll
        for (int dw = 0; dw < 4; ++dw) {
            const uint32_t lo6 = (ql[dw] & 0x0F0F0F0Fu) | (((qh[dw] >> pair_lo) & 0x03030303u) << 4);
            const uint32_t hi6 = ((ql[dw] >> 4) & 0x0F0F0F0Fu) | (((qh[dw] >> pair_hi) & 0x03030303u) << 4);
            v[4 * dw + 0] = (lo6 & 0x00FF00FFu) | 0x43004300u;
            v[4 * dw + 1] = ((lo6 >> 8) & 0x00FF00FFu) | 0x43004300u;
            v[4 * dw + 2] = (hi6 & 0x00FF00FFu) | 0x43004300u;
            v[4 * dw + 3] = ((hi6 >> 8) & 0x00FF00FFu) | 0x43004300u;
        }
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
            acc[t] += dl0 * (dlo - 160.f * xc[t].slo) + dl1 * (dhi - 160.f * xc[t].shi);
        }
    }
}

/* ---- IQ3_S in its 112-byte device blocks ------------------------------------
 *
 * Chunk c of a block is 32-weight group c in natural K order: index bytes
 * 8c..8c+7 (index i covers weights 4i..4i+3), the sign word at 64 + 4c (bit v
 * signs weight v), and the block's side word at 96 (qh bytes 0..7, scale
 * nibbles, d).  Weights come from an LDS table of the codebook as bf16
 * quads (entry e at lut[2e], lut[2e+1]); a sign flips the bf16 sign bit. */
__device__ __forceinline__ void build_iq3s_lut(uint32_t *lut, uint32_t tid, uint32_t nthreads) {
    for (uint32_t e = tid; e < 512; e += nthreads) {
        const uint32_t gw = kIq3sGrid[e];
        uint32_t h[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) h[b] = __builtin_bit_cast(uint32_t, (float)((gw >> (8 * b)) & 0xFF)) >> 16;
        lut[2 * e] = h[0] | (h[1] << 16);
        lut[2 * e + 1] = h[2] | (h[3] << 16);
    }
}

__device__ __forceinline__ void load_chunk_iq3s(const uint8_t *row, uint32_t ci, Payload2 &p, Hdr &h) {
    const uint32_t b = ci >> 3, c = ci & 7;
    const uint8_t *blk = row + (uint64_t)b * R9VX_IQ3S_DEV_BYTES;
    const r9vx_u32x2 q = *reinterpret_cast<const r9vx_u32x2 *>(blk + 8 * c);
    const uint32_t sg = *reinterpret_cast<const uint32_t *>(blk + 64 + 4 * c);
    p.a = r9vx_u32x4{q.x, q.y, sg, 0u};
    h.v = r9vx_ld128(blk + 96);
}

/* acc[t] += db * sum_v (sign_v grid_v) x_v with db = d (1 + 2 s_c)
 * (crates/r9v-format/src/iq.rs:698-722 for the weight law). */
template <int M>
__device__ __forceinline__ void chunk_dot_iq3s(const Payload2 &pl, const Hdr &h, uint32_t c,
                                               const XChunk<R9VX_SCHEME_IQ3_S, false> (&xc)[M], float (&acc)[M],
                                               const uint32_t *lut, int m = M) {
    const uint32_t qh = ((c < 4 ? h.v.x : h.v.y) >> (8 * (c & 3))) & 0xFF;
    const uint32_t sc = (h.v.z >> (4 * c)) & 0xF;
    const float db = r9vx_f16_to_f32((uint16_t)(h.v.w & 0xFFFF)) * (1.0f + 2.0f * (float)sc);
    const uint32_t sg = pl.a.z;
    uint32_t w[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t idx = (((i < 4 ? pl.a.x : pl.a.y) >> (8 * (i & 3))) & 0xFF) | (((qh >> i) & 1u) << 8);
        const r9vx_u32x2 e = *reinterpret_cast<const r9vx_u32x2 *>(lut + 2 * idx);
        const uint32_t nib = sg >> (4 * i);
        w[2 * i] = e.x ^ (((nib & 1u) << 15) | ((nib & 2u) << 30));
        w[2 * i + 1] = e.y ^ (((nib & 4u) << 13) | ((nib & 8u) << 28));
    }
#pragma unroll
    for (int t = 0; t < M; ++t) {
        if (t >= m) break;
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) s = r9vx_dot2_bf16(w[j], xc[t].p[j], s);
        acc[t] = fmaf(db, s, acc[t]);
    }
}

/* ---- f32 activations against Q8_0 / Q6_K (split) and IQ3_S chunks ----------
 *
 * acc += the chunk's dot product with f32 activations (XChunk<SCHEME, true>:
 * lo(i) the K position of the chunk's first 16 weights, hi(i) of its last
 * 16), every weight taken as its exact value before the multiply: Q8_0
 * d q, Q6_K d sc (q - 32), IQ3_S d (1 + 2 s) (sign grid) -- the laws of
 * chunk_dot_split and chunk_dot_iq3s, kept in f32 for activations that are
 * not bf16 (the MoE down projection's SwiGLU rows). */
template <int SCHEME>
__device__ __forceinline__ float chunk_dot_f32x(const Payload2 &pl, const Hdr &h, uint32_t c,
                                                const XChunk<SCHEME, true> &xc, const uint32_t *lut) {
    if constexpr (SCHEME == R9VX_SCHEME_Q8_0) {
        const float d = r9vx_f16_to_f32((uint16_t)h.e);
        const uint32_t q[8] = {pl.a.x, pl.a.y, pl.a.z, pl.a.w, pl.b.x, pl.b.y, pl.b.z, pl.b.w};
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) s = fmaf((float)(int8_t)((q[i >> 2] >> (8 * (i & 3))) & 0xFF), xc.lo(i), s);
#pragma unroll
        for (int i = 0; i < 16; ++i) s = fmaf((float)(int8_t)((q[4 + (i >> 2)] >> (8 * (i & 3))) & 0xFF), xc.hi(i), s);
        return d * s;
    } else if constexpr (SCHEME == R9VX_SCHEME_Q6_K) {
        const float d = r9vx_f16_to_f32((uint16_t)h.e);
        const uint32_t cc = c & 3, hsel = c >> 2;
        const uint32_t j0 = 8 * hsel + cc, j1 = j0 + 4;
        const uint32_t sv[4] = {h.v.x, h.v.y, h.v.z, h.v.w};
        const float dl0 = d * (float)(int8_t)((sv[j0 >> 2] >> (8 * (j0 & 3))) & 0xFF);
        const float dl1 = d * (float)(int8_t)((sv[j1 >> 2] >> (8 * (j1 & 3))) & 0xFF);
        const uint32_t pair_lo = 2 * (cc >> 1), pair_hi = pair_lo + 4;
        const uint32_t ql[4] = {pl.a.x, pl.a.y, pl.a.z, pl.a.w};
        const uint32_t qh[4] = {pl.b.x, pl.b.y, pl.b.z, pl.b.w};
        float slo = 0.f, shi = 0.f;
#pragma unroll
        for (int dw = 0; dw < 4; ++dw) {
            const uint32_t lo6 = (ql[dw] & 0x0F0F0F0Fu) | (((qh[dw] >> pair_lo) & 0x03030303u) << 4);
            const uint32_t hi6 = ((ql[dw] >> 4) & 0x0F0F0F0Fu) | (((qh[dw] >> pair_hi) & 0x03030303u) << 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                slo = fmaf((float)((int)((lo6 >> (8 * i)) & 0xFF) - 32), xc.lo(4 * dw + i), slo);
                shi = fmaf((float)((int)((hi6 >> (8 * i)) & 0xFF) - 32), xc.hi(4 * dw + i), shi);
            }
        }
        return dl0 * slo + dl1 * shi;
    } else {
        const uint32_t qh = ((c < 4 ? h.v.x : h.v.y) >> (8 * (c & 3))) & 0xFF;
        const uint32_t sc = (h.v.z >> (4 * c)) & 0xF;
        const float db = r9vx_f16_to_f32((uint16_t)(h.v.w & 0xFFFF)) * (1.0f + 2.0f * (float)sc);
        const uint32_t sg = pl.a.z;
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t idx = (((i < 4 ? pl.a.x : pl.a.y) >> (8 * (i & 3))) & 0xFF) | (((qh >> i) & 1u) << 8);
            const r9vx_u32x2 e = *reinterpret_cast<const r9vx_u32x2 *>(lut + 2 * idx);
            const uint32_t nib = sg >> (4 * i);
            /* weights 4i .. 4i + 3 of the 32: bf16 grid values, sign bits of nib */
            const uint32_t w2[4] = {e.x << 16, e.x & 0xFFFF0000u, e.y << 16, e.y & 0xFFFF0000u};
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float w = __builtin_bit_cast(float, w2[v] ^ (((nib >> v) & 1u) << 31));
                const int pos = 4 * i + v;
                s = fmaf(w, pos < 16 ? xc.lo(pos) : xc.hi(pos - 16), s);
            }
        }
        return db * s;
    }
}

/* ---- cross-lane sums of per-lane partials --------------------------------
 *
 * A row's partial sums sit in WIDTH consecutive lanes (an aligned group of 8,
 * 16, 32 or 64).  lane_reduce sums N arrays of V partials over the group:
 *  - across 32 and 16 lanes it reduce-scatters with the gfx950 permlane
 *    swaps: v_permlane32_swap(a, b) leaves {a[0..31], b[0..31]} and
 *    {a[32..63], b[32..63]}, so one add gives lanes 0..31 the sum of a and
 *    lanes 32..63 the sum of b (permlane16_swap does the same between
 *    neighbouring 16-lane rows).  Each step halves the live values; an odd
 *    leftover is swapped with itself and so reduced whole in both halves.
 *  - inside a 16-lane row it finishes with a DPP butterfly (row mirror, half-
 *    row mirror, quad reversal, quad pair swap), after which all lanes of the
 *    row hold the same live values.
 * Lane l of each row then emits the live slots s with s % G == l % G (G =
 * min(WIDTH, 16)) as emit(original index, values[N]); a leftover is emitted
 * once, by the half that kept the lower values. */
__device__ __forceinline__ float swap_sum32(float a, float b) {
    auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                              false, false);
    /* copy the elements out first: __builtin_bit_cast of r[1] in place
     * reads element 0 with this compiler */
    const uint32_t lo = r[0], hi = r[1];
    return __builtin_bit_cast(float, lo) + __builtin_bit_cast(float, hi);
}
__device__ __forceinline__ float swap_sum16(float a, float b) {
    auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                              false, false);
    /* copy the elements out first: __builtin_bit_cast of r[1] in place
     * reads element 0 with this compiler */
    const uint32_t lo = r[0], hi = r[1];
    return __builtin_bit_cast(float, lo) + __builtin_bit_cast(float, hi);
}
template <int CTRL>
__device__ __forceinline__ float dpp_add(float x) {
    return x + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF,
                                                                     false));
}

template <int V, int WIDTH>
struct LaneReduce {
    static constexpr int kC32 = WIDTH > 32 ? (V + 1) / 2 : V;    /* live after the 32-lane step */
    static constexpr int kLive = WIDTH > 16 ? (kC32 + 1) / 2 : kC32;
    static constexpr int kG = WIDTH < 16 ? WIDTH : 16;
};

template <int V, int WIDTH, int N, typename Emit>
__device__ __forceinline__ void lane_reduce(float (&v)[N][V], uint32_t lane, Emit &&emit) {
    using LR = LaneReduce<V, WIDTH>;
    if constexpr (WIDTH > 32) {
        constexpr int h = V / 2;
#pragma unroll
        for (int n = 0; n < N; ++n) {
#pragma unroll
            for (int i = 0; i < h; ++i) v[n][i] = swap_sum32(v[n][i], v[n][i + h]);
            if constexpr (V & 1) v[n][h] = swap_sum32(v[n][V - 1], v[n][V - 1]);
        }
    }
    if constexpr (WIDTH > 16) {
        constexpr int C = LR::kC32, h = C / 2;
#pragma unroll
        for (int n = 0; n < N; ++n) {
#pragma unroll
            for (int i = 0; i < h; ++i) v[n][i] = swap_sum16(v[n][i], v[n][i + h]);
            if constexpr (C & 1) v[n][h] = swap_sum16(v[n][C - 1], v[n][C - 1]);
        }
    }
    constexpr int C = LR::kLive;
#pragma unroll
    for (int n = 0; n < N; ++n)
#pragma unroll
        for (int i = 0; i < C; ++i) {
            float x = v[n][i];
            if constexpr (WIDTH > 8) x = dpp_add<0x140>(x); /* row_mirror: l <-> 15 - l */
            x = dpp_add<0x141>(x);                          /* row_half_mirror: l <-> 7 - l */
            x = dpp_add<0x1B>(x);                           /* quad_perm 3,2,1,0 */
            x = dpp_add<0xB1>(x);                           /* quad_perm 1,0,3,2 */
            v[n][i] = x;
        }
    constexpr int G = LR::kG;
    const int gl = (int)(lane & (uint32_t)(G - 1));
#pragma unroll
    for (int q = 0; q < (C + G - 1) / G; ++q) {
        const int s = gl + q * G;
        if (s >= C) break;
        float val[N];
#pragma unroll
        for (int n = 0; n < N; ++n) {
            val[n] = v[n][0];
#pragma unroll
            for (int i = 1; i < C; ++i)
                if (s == i) val[n] = v[n][i];
        }
        int j = s;
        bool dup = false;
        if constexpr (WIDTH > 16) {
            constexpr int h = LR::kC32 / 2;
            if (j < h) {
                if (lane & 16u) j += h;
            } else {
                j = LR::kC32 - 1;
                dup = dup || (lane & 16u) != 0;
            }
        }
        if constexpr (WIDTH > 32) {
            constexpr int h = V / 2;
            if (j < h) {
                if (lane & 32u) j += h;
            } else {
                j = V - 1;
                dup = dup || (lane & 32u) != 0;
            }
        }
        if (!dup) emit(j, val);
    }
}

/* lane_reduce for a runtime group width (8, 16, 32 or 64 = 1 << log2). */
template <int V, int N, typename Emit>
__device__ __forceinline__ void lane_reduce_w(float (&v)[N][V], uint32_t lane, uint32_t width_log2, Emit &&emit) {
    switch (width_log2) {
    case 6: lane_reduce<V, 64, N>(v, lane, emit); break;
    case 5: lane_reduce<V, 32, N>(v, lane, emit); break;
    case 4: lane_reduce<V, 16, N>(v, lane, emit); break;
    default: lane_reduce<V, 8, N>(v, lane, emit); break;
    }
}

/* IQ4_XS bf16 codebook-pair table: entry b = {kv[b & 15], kv[b >> 4]}
 * (codebook crates/r9v-format/src/iq_lut.rs:23-25; every value is a small
 * integer, so its bf16 is the top half of its f32 exactly).  Built at compile
 * time; a workgroup copies it to LDS with one 16-byte load per thread
 * (computing it per workgroup cost ~60 VALU per wave). */
struct Iq4PairLut {
    uint32_t v[256];
};
constexpr Iq4PairLut make_iq4_pair_lut() {
    constexpr int kv[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
    Iq4PairLut t{};
    for (int b = 0; b < 256; ++b) {
        const uint32_t lo = __builtin_bit_cast(uint32_t, (float)kv[b & 15]) >> 16;
        const uint32_t hi = __builtin_bit_cast(uint32_t, (float)kv[b >> 4]) >> 16;
        t.v[b] = lo | (hi << 16);
    }
    return t;
}
__device__ const Iq4PairLut kIq4PairLut = make_iq4_pair_lut();

__device__ __forceinline__ void init_iq4_lut(uint32_t *lut, uint32_t tid, uint32_t nthreads) {
    const r9vx_u32x4 *src = reinterpret_cast<const r9vx_u32x4 *>(kIq4PairLut.v);
    for (uint32_t i = tid; i < 64; i += nthreads) reinterpret_cast<r9vx_u32x4 *>(lut)[i] = src[i];
}

/* The table computed in VALU instead (r9vx_iq4_kvalue per nibble), for the
 * latency-bound dense GEMV, which builds it while its HBM loads are in
 * flight: any memory operation there (the copy above, issued before or after
 * the HBM loads) measured 0.2-0.6 us slower per launch at configs[1]. */
__device__ __forceinline__ void build_iq4_lut(uint32_t *lut, uint32_t tid, uint32_t nthreads) {
    for (uint32_t i = tid; i < 256; i += nthreads) {
        uint32_t lo = __builtin_bit_cast(uint32_t, (float)r9vx_iq4_kvalue(i & 15)) >> 16;
        uint32_t hi = __builtin_bit_cast(uint32_t, (float)r9vx_iq4_kvalue(i >> 4)) >> 16;
        lut[i] = lo | (hi << 16);
    }
}

}  // namespace r9vx

#endif
