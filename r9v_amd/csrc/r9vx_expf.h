/*
 * r9vx_expf.h -- f32 exp that reproduces the host glibc expf bit for bit.
 *
 * R9V's T0 router (crates/r9v-t0/src/moe_route.rs:331-346) evaluates the
 * softmax numerators with Rust f32::exp, which lowers to the platform libm
 * expf: on x86-64 Linux that is glibc's expf, whose algorithm (glibc >= 2.27)
 * is the published ARM optimized-routines method: reduce x*N/ln2 = k + r with
 * N = 32 by the 0x1.8p52 shift trick, look up 2^(k/N) in a 32-entry table,
 * evaluate a cubic in r in double precision and round once to float.  glibc
 * selects its FMA build on CPUs with FMA, in which the compiler fuses every
 * multiply that feeds an add; this restatement spells those fusions out with
 * fma() so the same double operations happen on the GPU.
 *
 * The table is 2^(i/32) correctly rounded to double, minus (i << 47) (so that
 * adding k << 47 yields 2^(k/32)); it is regenerated from that definition by
 * the CPU test.  Agreement with the host expf is checked exhaustively over
 * every float in the router's domain [-104, 0] by the CPU test suite.
 */
#ifndef R9VX_EXPF_H
#define R9VX_EXPF_H

#include <stdint.h>

#if defined(__HIPCC__)
#define R9VX_HD __host__ __device__ inline
#else
#define R9VX_HD static inline
#include <math.h>
#include <string.h>
#endif

#define R9VX_EXP2F_N 32

/* 2^(i/32) as double bits, minus (i << 47). */
#define R9VX_EXP2_TAB_INIT                                                                          \
    {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,     \
     0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,     \
     0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,     \
     0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,     \
     0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,     \
     0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,     \
     0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,     \
     0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

#if defined(__HIPCC__)
__constant__ static const uint64_t r9vx_exp2_table[32] = R9VX_EXP2_TAB_INIT;
static const uint64_t r9vx_exp2_table_host[32] = R9VX_EXP2_TAB_INIT;
__host__ __device__ inline uint64_t r9vx_exp2_tab(uint32_t i) {
#if defined(__HIP_DEVICE_COMPILE__)
    return r9vx_exp2_table[i & 31u];
#else
    return r9vx_exp2_table_host[i & 31u];
#endif
}
#else
static const uint64_t r9vx_exp2_table_host[32] = R9VX_EXP2_TAB_INIT;
static inline uint64_t r9vx_exp2_tab(uint32_t i) { return r9vx_exp2_table_host[i & 31u]; }
#endif

/* The evaluation, with TAB(i) supplying table entry i (0..31). */
#define R9VX_EXPF_BODY(TAB)                                                                       \
    const double inv_ln2_n = 0x1.71547652b82fep+0 * R9VX_EXP2F_N;                                 \
    const double shift = 0x1.8p+52;                                                               \
    /* Cubic for 2^(r/N), coefficients pre-divided by N^3, N^2, N. */                             \
    const double c0 = 0x1.c6af84b912394p-5 / R9VX_EXP2F_N / R9VX_EXP2F_N / R9VX_EXP2F_N;          \
    const double c1 = 0x1.ebfce50fac4f3p-3 / R9VX_EXP2F_N / R9VX_EXP2F_N;                         \
    const double c2 = 0x1.62e42ff0c52d6p-1 / R9VX_EXP2F_N;                                        \
    uint32_t ux;                                                                                  \
    R9VX_BITS(ux, x);                                                                             \
    uint32_t abstop = (ux >> 20) & 0x7ffu;                                                        \
    if (abstop >= 0x42bu) { /* |x| >= 88, inf or nan (top12(88.0f) = 0x42b) */                   \
        if (ux == 0xff800000u) return 0.0f;                                                       \
        if (abstop >= 0x7f8u) return x + x;                                                       \
        if (x > 0x1.62e42ep6f) return __builtin_huge_valf();                                      \
        if (x < -0x1.9fe368p6f) return 0.0f;                                                      \
    }                                                                                             \
    double xd = (double)x;                                                                        \
    double kd = fma(inv_ln2_n, xd, shift);                                                        \
    uint64_t ki;                                                                                  \
    R9VX_BITS(ki, kd);                                                                            \
    kd -= shift;                                                                                  \
    double r = fma(inv_ln2_n, xd, -kd);                                                           \
    uint64_t t = TAB((uint32_t)(ki % R9VX_EXP2F_N));                                              \
    t += ki << (52 - 5);                                                                          \
    double s;                                                                                     \
    R9VX_BITS(s, t);                                                                              \
    double z = fma(c0, r, c1);                                                                    \
    double r2 = r * r;                                                                            \
    double y = fma(c2, r, 1.0);                                                                   \
    y = fma(z, r2, y);                                                                            \
    y = y * s;                                                                                    \
    return (float)y;

#if defined(__HIPCC__)
#define R9VX_BITS(dst, src) (dst) = __builtin_bit_cast(decltype(dst), (src))
__host__ __device__ inline float r9vx_expf(float x) { R9VX_EXPF_BODY(r9vx_exp2_tab) }
/* Same function with the table in LDS (or any memory the caller filled with
 * r9vx_exp2_fill): a table lookup per call from constant memory is a global
 * load, and the special-case branches keep the compiler from batching them. */
__device__ inline float r9vx_expf_tab(float x, const uint64_t *tab) {
#define R9VX_TAB_PTR(i) tab[(i)]
    R9VX_EXPF_BODY(R9VX_TAB_PTR)
#undef R9VX_TAB_PTR
}
/* Branch-free form of r9vx_expf_tab, bit-identical to it: the main path runs
 * for every input (its table index is always in range) and the special
 * cases are applied afterwards by selects in reverse priority, so a caller's
 * loop over many inputs issues all of its table reads together. */
__device__ inline float r9vx_expf_tab_nb(float x, const uint64_t *tab) {
    const double inv_ln2_n = 0x1.71547652b82fep+0 * R9VX_EXP2F_N;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / R9VX_EXP2F_N / R9VX_EXP2F_N / R9VX_EXP2F_N;
    const double c1 = 0x1.ebfce50fac4f3p-3 / R9VX_EXP2F_N / R9VX_EXP2F_N;
    const double c2 = 0x1.62e42ff0c52d6p-1 / R9VX_EXP2F_N;
    const uint32_t ux = __builtin_bit_cast(uint32_t, x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    const double xd = (double)x;
    double kd = fma(inv_ln2_n, xd, shift);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= shift;
    const double r = fma(inv_ln2_n, xd, -kd);
    uint64_t t = tab[(uint32_t)(ki % R9VX_EXP2F_N)];
    t += ki << (52 - 5);
    const double sc = __builtin_bit_cast(double, t);
    const double z = fma(c0, r, c1);
    const double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    y = y * sc;
    const float main = (float)y;
    float sp = main; /* 88 <= |x| inside the finite range: the main path */
    sp = x < -0x1.9fe368p6f ? 0.0f : sp;
    sp = x > 0x1.62e42ep6f ? __builtin_huge_valf() : sp;
    sp = abstop >= 0x7f8u ? x + x : sp;
    sp = ux == 0xff800000u ? 0.0f : sp;
    return abstop >= 0x42bu ? sp : main;
}
__device__ inline void r9vx_exp2_fill(uint64_t *tab, uint32_t tid, uint32_t nthreads) {
    for (uint32_t i = tid; i < R9VX_EXP2F_N; i += nthreads) tab[i] = r9vx_exp2_table[i];
}
#else
#define R9VX_BITS(dst, src) memcpy(&(dst), &(src), sizeof(dst))
static inline float r9vx_expf(float x) { R9VX_EXPF_BODY(r9vx_exp2_tab) }
#endif

#endif
