/*
 * r9vx_x16.h -- bf16 activation rows to fp16 for the MFMA kernels: the row's
 * max |x| picks the power-of-two scale 2^e that keeps it below 2^15 (e = 0
 * for any ordinary activation; bf16 values are exact in fp16 inside that
 * range), written beside the row, and each 64-column step is stored in the
 * weight scheme's K group order (order_pos) or in natural order (PERM = 0).
 * One wave converts one row.
 */
#ifndef R9VX_X16_H
#define R9VX_X16_H

#include "r9vx_mfma.h"

namespace r9vx {

/* K offset (within a 64-step) of element i (0..7) of group q. */
template <int SCHEME>
__host__ __device__ constexpr uint32_t group_k(uint32_t q, uint32_t i) {
    if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
        return (i < 4 ? 0u : 32u) + 4 * q + (i & 3);
    } else {
        return 32 * (q >> 2) + (i < 4 ? 0u : 16u) + 4 * (q & 3) + (i & 3);
    }
}

/* Row element of elements i .. i + 3 (i = 0 or 4) of the 8-element group
 * stored at position c (a multiple of 8) of a row in order PERM: 0 natural;
 * Q4_K / IQ4_XS: each 64-column step in group_k's order; Q6_K: the two
 * 64-position steps of each 128-column span j = 0, 1 hold columns
 * 32 j + [0, 32) (group elements 0-3) and 64 + 32 j + [0, 32) (elements 4-7),
 * group q at 4 q (a Q6_K thread's half step: 16 ql bytes, whose low and
 * high nibbles are those two column ranges). */
template <int PERM>
__host__ __device__ constexpr uint32_t order_pos(uint32_t c, uint32_t i) {
    if constexpr (PERM == 0) {
        return c + i;
    } else if constexpr (PERM == R9VX_SCHEME_Q6_K) {
        return (c & ~127u) + 32 * ((c >> 6) & 1u) + 4 * ((c & 63u) >> 3) + (i ? 64u : 0u);
    } else {
        return (c & ~63u) + group_k<PERM>((c & 63u) >> 3, i);
    }
}

template <int PERM>
__device__ __forceinline__ void x16_row(const uint16_t *__restrict__ x, uint32_t k, _Float16 *__restrict__ x16,
                                        float *__restrict__ scale, uint32_t row, uint32_t lane) {
    const uint16_t *xr = x + (uint64_t)row * k;
    /* the lane's 8-value chunk at column c, in the output order */
    auto load_chunk = [&](uint32_t c, uint32_t (&w)[4]) {
        if constexpr (PERM == 0) {
            const r9vx_u32x4 v = *reinterpret_cast<const r9vx_u32x4 *>(xr + c);
            w[0] = v.x, w[1] = v.y, w[2] = v.z, w[3] = v.w;
        } else {
            const r9vx_u32x2 lo = *reinterpret_cast<const r9vx_u32x2 *>(xr + order_pos<PERM>(c, 0));
            const r9vx_u32x2 hi = *reinterpret_cast<const r9vx_u32x2 *>(xr + order_pos<PERM>(c, 4));
            w[0] = lo.x, w[1] = lo.y, w[2] = hi.x, w[3] = hi.y;
        }
    };
    _Float16 *orow = x16 + (uint64_t)row * k;
    if (k <= 64 * 8 * 8) {
        /* one pass: the lane's (at most 8) chunks stay in registers between
         * the row max and the conversion */
        uint32_t w[8][4];
        float mx = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t c = lane * 8 + 512u * i;
            if (c < k) {
                load_chunk(c, w[i]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    mx = fmaxf(mx, fabsf(__builtin_bit_cast(float, w[i][j] << 16)));
                    mx = fmaxf(mx, fabsf(__builtin_bit_cast(float, w[i][j] & 0xFFFF0000u)));
                }
            }
        }
        for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        const int e = row_shift(mx);
        const float inv = ldexpf(1.0f, -e);
        if (lane == 0) scale[row] = ldexpf(1.0f, e);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t c = lane * 8 + 512u * i;
            if (c < k) {
                uint32_t o[4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    o[j] = pack_h2(__builtin_bit_cast(float, w[i][j] << 16) * inv,
                                   __builtin_bit_cast(float, w[i][j] & 0xFFFF0000u) * inv);
                *reinterpret_cast<r9vx_u32x4 *>(orow + c) = r9vx_u32x4{o[0], o[1], o[2], o[3]};
            }
        }
        return;
    }
    float mx = 0.f;
#pragma unroll 4
    for (uint32_t c = lane * 8; c < k; c += 64 * 8) {
        r9vx_u32x4 v = *reinterpret_cast<const r9vx_u32x4 *>(xr + c);
        uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            mx = fmaxf(mx, fabsf(__builtin_bit_cast(float, w[i] << 16)));
            mx = fmaxf(mx, fabsf(__builtin_bit_cast(float, w[i] & 0xFFFF0000u)));
        }
    }
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    const int e = row_shift(mx);
    const float inv = ldexpf(1.0f, -e);
    if (lane == 0) scale[row] = ldexpf(1.0f, e);
#pragma unroll 4
    for (uint32_t c = lane * 8; c < k; c += 64 * 8) {
        uint32_t w[4];
        load_chunk(c, w);
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            o[i] = pack_h2(__builtin_bit_cast(float, w[i] << 16) * inv,
                           __builtin_bit_cast(float, w[i] & 0xFFFF0000u) * inv);
        *reinterpret_cast<r9vx_u32x4 *>(orow + c) = r9vx_u32x4{o[0], o[1], o[2], o[3]};
    }
}

/* The same with the group order chosen at run time (uniform). */
__device__ __forceinline__ void x16_row_scheme(uint32_t perm, const uint16_t *__restrict__ x, uint32_t k,
                                               _Float16 *__restrict__ x16, float *__restrict__ scale, uint32_t row,
                                               uint32_t lane) {
    if (perm == R9VX_SCHEME_Q4_K)
        x16_row<R9VX_SCHEME_Q4_K>(x, k, x16, scale, row, lane);
    else if (perm == R9VX_SCHEME_IQ4_XS)
        x16_row<R9VX_SCHEME_IQ4_XS>(x, k, x16, scale, row, lane);
    else if (perm == R9VX_SCHEME_Q6_K)
        x16_row<R9VX_SCHEME_Q6_K>(x, k, x16, scale, row, lane);
    else
        x16_row<0>(x, k, x16, scale, row, lane);
}

}  // namespace r9vx

#endif
