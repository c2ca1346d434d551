/*
 * r9vx_device.h -- shared gfx950 device helpers for the quantized-weight path.
 */
#ifndef R9VX_DEVICE_H
#define R9VX_DEVICE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "r9vx.h"
#include "r9vx_iq3s_grid.h"

#define R9VX_WAVE 64

typedef __bf16 r9vx_bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 r9vx_bf16x8 __attribute__((ext_vector_type(8)));
typedef float r9vx_f32x4 __attribute__((ext_vector_type(4)));
typedef float r9vx_f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t r9vx_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t r9vx_u32x2 __attribute__((ext_vector_type(2)));

/* GGUF block geometry (crates/r9v-format/tests/iq.rs:131-141). */
#define R9VX_Q4K_BYTES 144
#define R9VX_IQ4XS_BYTES 136
#define R9VX_Q6K_BYTES 210   /* wire block: ql 128, qh 64, scales 16, d 2 */
#define R9VX_Q6K_BODY 208    /* split-layout body: the wire block without d */
#define R9VX_Q80_BYTES 34    /* wire block: d 2, 32 int8 quants */
/* IQ3_S: 110-byte wire block (d f16 | qs 64 | qh 8 | signs 32 | scales 4);
 * the device reads the 112-byte repacked block (qs 64 | signs 32 | qh 8 |
 * scales 4 | d 2 | 0 0), in which the four sign bytes of 32-weight group g
 * form the little-endian word at 64 + 4g whose bit v signs weight v of the
 * group. */
#define R9VX_IQ3S_BYTES 110
#define R9VX_IQ3S_DEV_BYTES 112

/* The IQ3_S codebook (entry e = word e, value b in byte b). */
static __device__ const uint32_t kIq3sGrid[512] = {R9VX_IQ3S_GRID_WORDS};

/* IQ4 codebook (crates/r9v-format/src/iq_lut.rs:23-25). */
__device__ __forceinline__ int r9vx_iq4_kvalue(uint32_t q) {
    /* Two 8-entry int8 tables packed in four dwords; selected without memory. */
    const uint32_t t0 = 0xBFAD9881u; /* -127,-104,-83,-65 as bytes 0x81,0x98,0xAD,0xBF */
    const uint32_t t1 = 0xF6EADDCFu; /* -49,-35,-22,-10 */
    const uint32_t t2 = 0x26190D01u; /* 1,13,25,38 */
    const uint32_t t3 = 0x71594535u; /* 53,69,89,113 */
    uint32_t w = q < 4 ? t0 : q < 8 ? t1 : q < 12 ? t2 : t3;
    return (int)(int8_t)(w >> ((q & 3u) * 8));
}

/* f16 bits -> f32: hardware conversion is exact for every finite f16,
 * subnormals included (f16 denormals are preserved on gfx9). */
__device__ __forceinline__ float r9vx_f16_to_f32(uint16_t bits) {
    return (float)__builtin_bit_cast(_Float16, bits);
}

__device__ __forceinline__ float r9vx_bf16_to_f32(uint16_t bits) {
    return __builtin_bit_cast(float, (uint32_t)bits << 16);
}

/* f32 -> bf16 bits, round-to-nearest-even, NaN quieted
 * (crates/r9v-t0/src/dtype.rs:102-111). */
__device__ __forceinline__ uint16_t r9vx_f32_to_bf16(float v) {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    if (v != v) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

typedef _Float16 r9vx_f16x2 __attribute__((ext_vector_type(2)));
/* c + a.lo * b.lo + a.hi * b.hi, fp16 pairs, f32 accumulate (v_dot2_f32_f16). */
__device__ __forceinline__ float r9vx_dot2_f16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(r9vx_f16x2, a), __builtin_bit_cast(r9vx_f16x2, b), c, false);
}

__device__ __forceinline__ float r9vx_dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(r9vx_bf16x2, a),
                                          __builtin_bit_cast(r9vx_bf16x2, b), c, false);
}

/* 128-bit load from a 4-byte aligned global address (IQ4_XS blocks are 136 B,
 * so half of their payloads start on an 8-byte boundary; gfx9 global loads
 * accept dword alignment). */
__device__ __forceinline__ r9vx_u32x4 r9vx_ld128(const uint8_t *p) {
    typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
    return *(const u32x4a4 *)p;
}

/* Non-temporal streaming variant for weight bytes that are read once. */
__device__ __forceinline__ r9vx_u32x4 r9vx_ld128_nt(const uint8_t *p) {
    typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
    return __builtin_nontemporal_load((const u32x4a4 *)p);
}

/* Butterfly sum over aligned groups of `width` lanes (width a power of 2 <= 64). */
__device__ __forceinline__ float r9vx_group_sum(float v, int width) {
    for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, R9VX_WAVE);
    return v;
}

#endif
