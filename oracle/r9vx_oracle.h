/*
 * r9vx_oracle.h -- CPU restatement of R9V's scalar T0 oracle for the
 * quantized-weight matrix path (GGUF Q4_K / IQ4_XS decode, Branch-D
 * matmul, moe_route, the (expert, token) permute and the sliced moe_ffn).
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links or
 * calls this code: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it, and only as the checker / CPU baseline.
 *
 * Every function cites the reference file:line it restates.  Numerics are
 * plain IEEE f32 in the reference's evaluation order; the build uses
 * -O2 -ffp-contract=off so no multiply-add is ever fused (Rust never fuses).
 *
 * Parity pinning (what checks each function, beyond restating it):
 *   rxo_f16_to_f32, rxo_f32_to_bf16 ... exhaustive/closed-form tests
 *   rxo_q4k_*  ... reference golden vectors q4k_reference.txt (6 cases)
 *   rxo_iq4xs_* ... reference golden vectors iq_a24_reference.txt (IQ4_XS)
 *   Q6_K / Q8_0 decode ... reference golden vectors gguf_a23_reference.txt
 *                  (gguf-py 0.19.0 dequantize), and a numpy restatement of
 *                  the llama.cpp row loop (dequantize_row_q6_K form)
 *   IQ3_S decode ... reference golden vectors iq_a24_reference.txt (IQ3_S,
 *                  gguf-py 0.19.0), a numpy restatement of the llama.cpp row
 *                  loop (dequantize_row_iq3_s form), and the codebook facts
 *                  of crates/r9v-format/tests/iq.rs:505-516
 *   rxo_matmul ... known answer 1408.0 (matmul_tests.rs:208-265), f64
 *                  brute force on tiny shapes, batch invariance
 *   rxo_moe_route ... equal-logit lowest-id answers (moe_route_tests.rs:107),
 *                  f64 brute force of the softmax, invariants
 *   rxo_moe_sort ... std stable sort brute force, histogram/scan invariants
 *   rxo_moe_ffn ... sliced vs full-matrix T0 equivalence on tiny E,
 *                  token-permutation invariance, duplicate slots, f64 check
 */
#ifndef R9VX_ORACLE_H
#define R9VX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Weight schemes: GGUF type codes (r9v-format ggml.rs GgmlType codes). */
#define RXO_Q4_K 12
#define RXO_IQ4_XS 23
#define RXO_Q6_K 14
#define RXO_Q8_0 8
#define RXO_IQ3_S 21

/* Element dtypes: discriminant order of r9v-ir DType (dtype.rs:15-35). */
#define RXO_F32 0
#define RXO_BF16 2

/* Error codes: 0 ok; negative = refusal before any output write. */
#define RXO_OK 0
#define RXO_ERR_SHAPE -1
#define RXO_ERR_SCALE -2
#define RXO_ERR_NONFINITE -3
#define RXO_ERR_ID -4
#define RXO_ERR_DTYPE -5
#define RXO_ERR_SCHEME -6

/* ---- scalar codecs ---------------------------------------------------- */
float rxo_f16_to_f32(uint16_t bits);
uint16_t rxo_f32_to_bf16(float v);
float rxo_bf16_to_f32(uint16_t bits);

/* ---- block decode ----------------------------------------------------- */
/* GGUF block geometry: bytes per block and weights per block. */
uint32_t rxo_block_bytes(int scheme);
uint32_t rxo_block_len(int scheme);
/* Q4_K: 12-byte packed 6-bit scales -> sc[8], mn[8]. */
void rxo_q4k_unpack_scales(const uint8_t payload[12], uint8_t sc[8], uint8_t mn[8]);
/* Decodes n_rows x k weights from GGUF wire blocks into out (row-major f32).
 * Refuses (before writing) any non-finite f16 block scale. */
int rxo_dequantize(int scheme, const uint8_t *wire, uint32_t n_rows, uint32_t k, float *out);

/* ---- Branch-D matmul -------------------------------------------------- */
/* y[m, n] = epilogue(sum_k x[m, k] * w[n, k]) with k ascending and one f32
 * accumulator; x is f32 or bf16; y is f32 or bf16 (RNE).  bias [N] f32 and
 * residual [M, N] f32 are optional (NULL = none; at most one non-NULL). */
int rxo_matmul(int scheme, const uint8_t *w, uint32_t n, uint32_t k,
               int x_dtype, const void *x, uint32_t m,
               const float *bias, const float *residual,
               int y_dtype, void *y);

/* Router logits [t, e] = bf16 x [t, dm] . f32 w [e, dm]^T in Branch D order. */
void rxo_router_logits(const uint16_t *x, const float *w, uint32_t t, uint32_t e, uint32_t dm, float *out);
/* act_mul with SiLU (crates/r9v-t0/src/act_mul.rs:86-99): y = silu(g) * u. */
void rxo_act_mul_silu(const float *g, const float *u, uint64_t n, float *y);

/* ---- MoE -------------------------------------------------------------- */
/* Reference glibc expf (the host libm the Rust T0 f32::exp resolves to). */
float rxo_expf(float x);
void rxo_expf_fill(uint32_t first_bits, uint64_t n, float *out);
/* Rows per pass of the matmul / expert dots: 4 (default) or 1 (T0's loop
 * structure).  Outputs are bit-identical either way; only speed differs. */
void rxo_set_rows_at_once(int n);
/* moe_route with softmax scoring (scoring 0) or sigmoid (scoring 1). */
int rxo_moe_route(const float *logits, const float *bias, uint32_t t, uint32_t e,
                  uint32_t k, float scale, int renormalize, int scoring,
                  uint32_t *expert_ids, float *weights);
/* Stable (expert, token, slot) ordering of the T*K routing pairs.
 * counts[e]; offsets[e] exclusive scan with offsets[E] = T*K;
 * sorted[i] = token*K + slot of the i-th pair in sorted order. */
int rxo_moe_sort(const uint32_t *expert_ids, uint32_t t, uint32_t k, uint32_t e,
                 uint32_t *counts, uint32_t *offsets, uint32_t *sorted);
/* Sliced moe_ffn: x [T, Dm] (f32 or bf16); gate/up [E+S, 2Dff, Dm] in
 * scheme_gu, down [E+S, Dm, Dff] in scheme_dn (GGUF wire blocks, expert
 * major); S shared experts follow the E routed ones and are added, weight
 * 1.0, after the routed combine.  y [T, Dm] f32.  h_bf16 != 0 rounds the
 * SwiGLU output to bf16 before the down projection. */
int rxo_moe_ffn(int x_dtype, const void *x, uint32_t t, uint32_t dm, uint32_t dff,
                uint32_t e, uint32_t s_shared, uint32_t k,
                const uint32_t *expert_ids, const float *weights,
                int scheme_gu, const uint8_t *w_gate_up,
                int scheme_dn, const uint8_t *w_down,
                int h_bf16, float *y);
/* rxo_moe_ffn with the expert FFNs over `threads` OpenMP threads;
 * bit-identical to it for every thread count. */
int rxo_moe_ffn_mt(int x_dtype, const void *x, uint32_t t, uint32_t dm, uint32_t dff,
                   uint32_t e, uint32_t s_shared, uint32_t k,
                   const uint32_t *expert_ids, const float *weights,
                   int scheme_gu, const uint8_t *w_gate_up,
                   int scheme_dn, const uint8_t *w_down,
                   int h_bf16, float *y, int threads);
/* Literal T0 form for tiny E: gate/up GEMM over the full [E*2Dff, Dm]
 * matrix, then slice (moe_ffn.rs:575-612).  Used to pin the sliced form. */
int rxo_moe_ffn_full(int x_dtype, const void *x, uint32_t t, uint32_t dm, uint32_t dff,
                     uint32_t e, uint32_t k, const uint32_t *expert_ids,
                     const float *weights, int scheme_gu, const uint8_t *w_gate_up,
                     int scheme_dn, const uint8_t *w_down, float *y);

/* Dense single-expert SwiGLU FFN over gathered rows (the shared-expert
 * graph: matmul gate, matmul up, act_mul SiLU, matmul down). */
int rxo_expert_ffn(int x_dtype, const void *x, uint32_t rows, uint32_t dm, uint32_t dff,
                   int scheme_gu, const uint8_t *w_gate_up, int scheme_dn,
                   const uint8_t *w_down, int h_bf16, float *out);

/* Multi-threaded (OpenMP over output rows) Branch-D matmul for the
 * all-cores CPU baseline; bit-identical to rxo_matmul. */
int rxo_moe_expert_mt(int x_dtype, const void *x, const uint32_t *tokens, uint32_t n_tok, uint32_t dm,
                      uint32_t dff, int scheme_gu, const uint8_t *gu, int scheme_dn, const uint8_t *dn, float *out,
                      int threads);
int rxo_matmul_mt(int scheme, const uint8_t *w, uint32_t n, uint32_t k,
                  int x_dtype, const void *x, uint32_t m, int y_dtype, void *y,
                  int threads);

#ifdef __cplusplus
}
#endif
#endif
