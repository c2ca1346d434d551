/*
 * r9vx_internal.h -- block-header decoding shared by the kernels, and the
 * internal launchers the C-ABI layer (r9vx_api.cpp) dispatches to.
 */
#ifndef R9VX_INTERNAL_H
#define R9VX_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "r9vx.h"

#ifdef __HIPCC__
#include "r9vx_device.h"
/* Q4_K 6-bit scale/min of sub-blocks 2g and 2g+1 from the 16-byte block
 * header read as four dwords (bytes 4..15 are the packed payload):
 * crates/r9v-format/src/ggml.rs:973-995 (unpack_k4_scales). */
__device__ __forceinline__ uint32_t r9vx_q4k_payload_byte(r9vx_u32x4 h, uint32_t i) {
    uint32_t w = i < 4 ? h.y : (i < 8 ? h.z : h.w);
    return (w >> ((i & 3) * 8)) & 0xFFu;
}

__device__ __forceinline__ void r9vx_q4k_scale_pair(r9vx_u32x4 h, uint32_t g, uint32_t sc[2],
                                                    uint32_t mn[2]) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        uint32_t j = 2 * g + t;
        if (j < 4) {
            sc[t] = r9vx_q4k_payload_byte(h, j) & 63u;
            mn[t] = r9vx_q4k_payload_byte(h, j + 4) & 63u;
        } else {
            uint32_t bj4 = r9vx_q4k_payload_byte(h, j + 4);
            sc[t] = (bj4 & 0xFu) | ((r9vx_q4k_payload_byte(h, j - 4) >> 2) & 0x30u);
            mn[t] = (bj4 >> 4) | ((r9vx_q4k_payload_byte(h, j) >> 2) & 0x30u);
        }
    }
}

/* The same pair without a branch: bytes {sc(2g), sc(2g+1), mn(2g), mn(2g+1)}.
 * X gathers scale bytes 2(g&1), +1, 4+2(g&1), +1 (one v_perm of dwords 1
 * and 2), Y the same bytes of dword 3 and its nibbles shifted down; g < 2
 * keeps X's six low bits, g >= 2 combines Y's nibbles with X's top two bits
 * (the table of r9vx_q4k_scale_pair). */
__device__ __forceinline__ uint32_t r9vx_q4k_pair_bytes(r9vx_u32x4 h, uint32_t g) {
    const uint32_t sel = (g & 1u) ? 0x07060302u : 0x05040100u;
    const uint32_t x = __builtin_amdgcn_perm(h.z, h.y, sel);
    const uint32_t y = __builtin_amdgcn_perm(h.w >> 4, h.w, sel);
    return g >= 2 ? ((y & 0x0F0F0F0Fu) | ((x >> 2) & 0x30303030u)) : (x & 0x3F3F3F3Fu);
}

/* (a & m) | o in one v_and_or_b32: with both masks as literals the compiler
 * emits a v_and and a v_or (a three-operand VOP3 takes no literal here). */
__device__ __forceinline__ uint32_t r9vx_and_or(uint32_t a, uint32_t m, uint32_t o) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(o));
    return r;
}

/* IQ4_XS sub-block scale s - 32 as f32 from the 8-byte header
 * (crates/r9v-format/src/iq.rs:587-590): low nibble from scales_l, high two
 * bits from scales_h. */
__device__ __forceinline__ float r9vx_iq4xs_scale(r9vx_u32x2 h, uint32_t c) {
    uint32_t lo = (h.y >> (4 * c)) & 0xFu;
    uint32_t hi = (h.x >> (16 + 2 * c)) & 0x3u;
    return (float)(int)(lo | (hi << 4)) - 32.0f;
}
#endif

/* IQ3_S device block byte j (0..111) comes from wire byte r9vx_iq3s_wire_byte(j)
 * (j < 110; bytes 110, 111 are zero): qs (wire 2..65), signs (74..105), qh
 * (66..73), scales (106..109), d (0..1).  Used by the device repack and the
 * host-side repack of r9vx_gguf_upload. */
__host__ __device__ inline uint32_t r9vx_iq3s_wire_byte(uint32_t j) {
    return j < 64 ? 2 + j : j < 96 ? 10 + j : j < 104 ? j - 30 : j < 108 ? j + 2 : j - 108;
}

/* Internal launchers (return hipError_t as int). */
int r9vx_launch_dequant(uint32_t scheme, const uint8_t *wire, uint32_t n_rows, uint32_t k,
                        float *out, hipStream_t stream);
int r9vx_launch_validate(uint32_t scheme, const uint8_t *wire, uint32_t n_rows, uint32_t k,
                         uint32_t *bad, hipStream_t stream);
int r9vx_launch_dequant_split(uint32_t scheme, const uint8_t *wire, uint32_t n_rows, uint32_t k, float *out,
                              hipStream_t stream);
int r9vx_launch_validate_split(uint32_t scheme, const uint8_t *wire, uint32_t n_rows, uint32_t k, uint32_t *bad,
                               hipStream_t stream);
int r9vx_launch_repack(uint32_t scheme, const uint8_t *wire, uint32_t n_rows, uint32_t k, uint8_t *body,
                       uint16_t *scales, hipStream_t stream);

struct r9vx_gemv_problem {
    const uint8_t *w;
    const uint16_t *w_scales; /* Q8_0 / Q6_K: f16 d per block, row-major [n, k/block] */
    const void *x;
    const float *bias;
    const float *residual;
    void *y;
    uint32_t n, k, m;
    uint32_t scheme, x_dtype, y_dtype, epilogue;
    uint64_t w_row_stride; /* bytes between weight rows */
    uint64_t x_row_stride; /* elements between activation rows */
};
int r9vx_launch_gemv(const r9vx_gemv_problem &p, hipStream_t stream);

struct r9vx_gemm_problem {
    const uint8_t *w;
    const uint16_t *w_scales; /* Q8_0 / Q6_K: f16 d per block */
    const uint16_t *x; /* bf16 [m, k] */
    const float *bias;
    const float *residual;
    void *y;
    void *workspace; /* r9vx_gemm_workspace_bytes(m_bucket, k): fp16 x rows + row scales */
    uint32_t n, k, m;
    uint32_t m_bucket; /* the variant's bucket: the kernel is chosen from it, never from m */
    uint32_t scheme, y_dtype, epilogue;
};
size_t r9vx_gemm_workspace_bytes(uint32_t m_bucket, uint32_t k);
int r9vx_launch_gemm(const r9vx_gemm_problem &p, hipStream_t stream);
/* Compute units of the current device (cached per device; 256 if the query fails). */
uint32_t r9vx_device_cus();

struct r9vx_route_problem {
    const float *logits;
    const float *bias;
    uint32_t *ids;
    float *weights;
    uint32_t *status; /* the launch's status word; NULL = the plain-launch word of the stream */
    uint32_t t, e, k, scoring, renormalize;
    float scale;
};
/* *no_word is set when a plain launch (status NULL) finds every per-stream
 * status word of the device taken by other streams. */
int r9vx_launch_route(const r9vx_route_problem &p, hipStream_t stream, bool *no_word = nullptr);
/* Streams per device that can make plain moe_route launches. */
uint32_t r9vx_route_stream_words();

struct r9vx_route_hidden_problem {
    const uint16_t *x; /* bf16 [t, dm] */
    const float *w;    /* f32 [e, dm] */
    const float *bias;
    float *logits;     /* workspace [t, e] */
    uint32_t *counter; /* workspace word, zero between launches */
    uint32_t *status;  /* workspace word: this launch's status bits */
    uint32_t *ids;
    float *weights;
    uint32_t t, e, k, dm, scoring, renormalize;
    float scale;
};
int r9vx_launch_route_hidden(const r9vx_route_hidden_problem &p, hipStream_t stream);
int r9vx_launch_router_repack(const float *w, uint32_t e, uint32_t dm, float *out, hipStream_t stream);
int r9vx_read_route_status(uint32_t *status, hipStream_t stream);

/* Device-layout bytes of one weight row of k weights: GGUF blocks (Q4_K,
 * IQ4_XS), 112-byte IQ3_S blocks, or the body of the split layout (Q8_0 int8
 * quants, Q6_K blocks without d); and the f16 d values per row that the
 * split layout keeps in its separate scale array (0 for the others). */
__host__ __device__ inline uint64_t r9vx_row_bytes(uint32_t scheme, uint32_t k) {
    switch (scheme) {
    case R9VX_SCHEME_Q8_0: return k;
    case R9VX_SCHEME_Q6_K: return (uint64_t)(k / 256) * R9VX_Q6K_BODY;
    case R9VX_SCHEME_IQ3_S: return (uint64_t)(k / 256) * R9VX_IQ3S_DEV_BYTES;
    case R9VX_SCHEME_Q4_K: return (uint64_t)(k / 256) * R9VX_Q4K_BYTES;
    default: return (uint64_t)(k / 256) * R9VX_IQ4XS_BYTES;
    }
}
__host__ __device__ inline uint32_t r9vx_row_scales(uint32_t scheme, uint32_t k) {
    return scheme == R9VX_SCHEME_Q8_0 ? k / 32 : scheme == R9VX_SCHEME_Q6_K ? k / 256 : 0u;
}

/* Weight schemes the 256 x 256 loop of r9vx_mma3.h decodes: all five (the
 * grouped MoE GEMMs and the dense GEMM take it for every scheme and N). */
__host__ __device__ inline bool r9vx_m3_scheme(uint32_t scheme) {
    return scheme == R9VX_SCHEME_Q4_K || scheme == R9VX_SCHEME_IQ4_XS || scheme == R9VX_SCHEME_Q8_0 ||
           scheme == R9VX_SCHEME_Q6_K || scheme == R9VX_SCHEME_IQ3_S;
}
/* The K order (r9vx_x16.h order_pos) that activation rows take for a weight
 * scheme on that loop: Q4_K's and Q6_K's own; IQ4_XS's for IQ4_XS and Q8_0
 * (in both, group s of a thread's half step is elements 4s .. 4s + 3 and
 * 16 + 4s .. 16 + 4s + 3 of one 32-weight sub-block or block); 0 (natural)
 * for IQ3_S (a thread's half step is one 32-weight group in column order). */
__host__ __device__ inline uint32_t r9vx_group_order(uint32_t scheme) {
    if (scheme == R9VX_SCHEME_Q4_K || scheme == R9VX_SCHEME_Q6_K) return scheme;
    return scheme == R9VX_SCHEME_IQ4_XS || scheme == R9VX_SCHEME_Q8_0 ? (uint32_t)R9VX_SCHEME_IQ4_XS : 0u;
}

struct r9vx_moe_problem {
    const uint16_t *x; /* bf16 [t, dm] */
    const uint32_t *ids;
    const float *weights;
    const uint8_t *w_gu;
    const uint8_t *w_dn;
    const uint16_t *s_gu; /* split layout (Q8_0 / Q6_K): f16 d rows of w_gu / w_dn, else NULL */
    const uint16_t *s_dn;
    float *y;
    uint8_t *ws;
    uint32_t t, e, k, dm, dff, shared, t_bucket;
    uint32_t scheme_gu, scheme_dn;
};
size_t r9vx_moe_workspace_bytes(uint32_t t_bucket, uint32_t e, uint32_t k, uint32_t dm,
                                uint32_t dff, uint32_t shared);
int r9vx_launch_moe(const r9vx_moe_problem &p, hipStream_t stream);
int r9vx_launch_moe_sort(const r9vx_moe_problem &p, uint32_t *counts, uint32_t *offsets,
                         uint32_t *sorted, hipStream_t stream);
int r9vx_read_moe_status(const r9vx_moe_problem &p, uint32_t *status, hipStream_t stream);

#endif
