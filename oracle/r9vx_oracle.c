/*
 * r9vx_oracle.c -- CPU restatement of R9V's scalar T0 oracle (test
 * infrastructure only; see r9vx_oracle.h for the pinning of each part).
 *
 * Build: gcc -O2 -ffp-contract=off -fno-fast-math (oracle/Makefile).
 * All f32 arithmetic is evaluated in the reference's order, one rounding
 * per operation, exactly as the Rust source states it.
 */
#include "r9vx_oracle.h"

#include <math.h>

#include "../r9v_amd/csrc/r9vx_iq3s_grid.h"
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------
 * Scalar codecs
 * ---------------------------------------------------------------------- */

static inline uint32_t f32_bits(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    return u;
}
static inline float bits_f32(uint32_t u) {
    float v;
    memcpy(&v, &u, 4);
    return v;
}

/* crates/r9v-format/src/scales.rs:13-36 (f16_to_f32): exact widening,
 * subnormals renormalised, NaN payload kept in the top mantissa bits. */
float rxo_f16_to_f32(uint16_t bits) {
    uint32_t sign = ((uint32_t)bits & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)bits >> 10) & 0x1Fu;
    uint32_t mant = (uint32_t)bits & 0x3FFu;
    uint32_t wide;
    if (exp == 0) {
        if (mant == 0) {
            wide = sign;
        } else {
            uint32_t m = mant;
            int32_t e = 1;
            while ((m & 0x400u) == 0) {
                m <<= 1;
                e -= 1;
            }
            wide = sign | ((uint32_t)(e + 112) << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (exp == 31) {
        wide = sign | 0x7F800000u | (mant << 13);
    } else {
        wide = sign | ((exp + 112) << 23) | (mant << 13);
    }
    return bits_f32(wide);
}

/* crates/r9v-t0/src/dtype.rs:102-111 (f32_to_bf16): RNE, NaN quieted. */
uint16_t rxo_f32_to_bf16(float val) {
    uint32_t u = f32_bits(val);
    if (isnan(val)) return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t lsb = (u >> 16) & 1u;
    uint32_t rounded = u + 0x7FFFu + lsb;
    return (uint16_t)(rounded >> 16);
}

/* crates/r9v-t0/src/dtype.rs:114-116 (bf16_to_f32). */
float rxo_bf16_to_f32(uint16_t bits) { return bits_f32((uint32_t)bits << 16); }

static inline uint16_t rd_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ------------------------------------------------------------------------
 * Block decode
 * ---------------------------------------------------------------------- */

uint32_t rxo_block_bytes(int scheme) {
    /* crates/r9v-format/tests/iq.rs:131-141 and ggml.rs:336-350 block table:
     * Q4_K 144 B / 256 weights, IQ4_XS 136 B / 256, Q6_K 210 B / 256,
     * Q8_0 34 B / 32, IQ3_S 110 B / 256. */
    if (scheme == RXO_Q4_K) return 144;
    if (scheme == RXO_IQ3_S) return 110;
    if (scheme == RXO_IQ4_XS) return 136;
    if (scheme == RXO_Q6_K) return 210;
    if (scheme == RXO_Q8_0) return 34;
    return 0;
}

uint32_t rxo_block_len(int scheme) { return scheme == RXO_Q8_0 ? 32 : (rxo_block_bytes(scheme) ? 256 : 0); }

/* GGUF wire bytes of one row of k weights (k a multiple of the block). */
static uint64_t wire_row_bytes(int scheme, uint32_t k) {
    return (uint64_t)(k / rxo_block_len(scheme)) * rxo_block_bytes(scheme);
}

/* crates/r9v-format/src/ggml.rs:973-995 (unpack_k4_scales), identical to
 * records.rs:190-206 (I4KSuperblock::from_bytes). */
void rxo_q4k_unpack_scales(const uint8_t q[12], uint8_t sc[8], uint8_t mn[8]) {
    for (int j = 0; j < 4; ++j) {
        sc[j] = q[j] & 63;
        mn[j] = q[j + 4] & 63;
    }
    for (int j = 4; j < 8; ++j) {
        sc[j] = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 2) & 0x30));
        mn[j] = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 2) & 0x30));
    }
}

/* IQ4 codebook: crates/r9v-format/src/iq_lut.rs:23-25 (IQ4_KVALUES). */
static const int8_t KVALUES[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                   1,    13,   25,  38,  53,  69,  89,  113};

/* Scale validity on the GGUF wire path: crates/r9v-format/src/ggml.rs:421-445
 * (check_wire_f16) -- finite values accepted, negative included. */
static int wire_scale_ok(uint16_t bits) { return isfinite(rxo_f16_to_f32(bits)); }

/* One Q4_K block -> 256 f32.  crates/r9v-format/src/ggml.rs:744-790 (nibble
 * order: byte (j/2)*32+p of the 128-B payload holds sub-block 2g low and 2g+1
 * high) and :1131-1150 (w = (d*sc[j])*q - (dmin*mn[j]), in that order). */
static void q4k_block(const uint8_t *blk, float *out) {
    float d = rxo_f16_to_f32(rd_u16(blk));
    float dmin = rxo_f16_to_f32(rd_u16(blk + 2));
    uint8_t sc[8], mn[8];
    rxo_q4k_unpack_scales(blk + 4, sc, mn);
    const uint8_t *qs = blk + 16;
    for (int j = 0; j < 8; ++j) {
        float dl = d * (float)sc[j];
        float ml = dmin * (float)mn[j];
        for (int p = 0; p < 32; ++p) {
            uint8_t byte = qs[(j / 2) * 32 + p];
            uint32_t q = (byte >> ((j % 2) * 4)) & 0x0F;
            float prod = dl * (float)q;
            out[j * 32 + p] = prod - ml;
        }
    }
}

/* One IQ4_XS block -> 256 f32.  crates/r9v-format/src/iq.rs:578-598
 * (source_block, Iq4Xs arm): s = (lo | hi<<4) as i8 as f32 - 32, dl = d*s,
 * w = dl * KVALUES[q]; weight j of sub-block g is byte 8+16g+(j%16), low
 * nibble for j<16 (iq.rs:274-293). */
static void iq4xs_block(const uint8_t *blk, float *out) {
    float d = rxo_f16_to_f32(rd_u16(blk));
    uint16_t scales_h = rd_u16(blk + 2);
    for (int g = 0; g < 8; ++g) {
        uint8_t lo = (blk[4 + g / 2] >> ((g % 2) * 4)) & 0x0F;
        uint8_t hi = (uint8_t)((scales_h >> (2 * g)) & 0x03);
        float s = (float)(int8_t)(lo | (hi << 4)) - 32.0f;
        float dl = d * s;
        for (int j = 0; j < 32; ++j) {
            uint8_t byte = blk[8 + g * 16 + (j % 16)];
            uint8_t q = j < 16 ? (byte & 0x0F) : (byte >> 4);
            out[g * 32 + j] = dl * (float)KVALUES[q & 0x0F];
        }
    }
}

/* One Q6_K block -> 256 f32.  crates/r9v-format/src/ggml.rs:817-850
 * (block_values: value i = flat index big*32+big_p takes its low nibble from
 * byte (i/128)*64 + i%64, nibble (i%128)/64, and its high two bits from byte
 * 128 + (i/128)*32 + i%32, bit pair (i%128)/32) and :1154-1172 (dequant:
 * dl = d * (i8)scales[j] for the j-th group of 16, w = dl * (q - 32)). */
static void q6k_block(const uint8_t *blk, float *out) {
    float d = rxo_f16_to_f32(rd_u16(blk + 208));
    for (int j = 0; j < 16; ++j) {
        float dl = d * (float)(int8_t)blk[192 + j];
        for (int p = 0; p < 16; ++p) {
            int i = j * 16 + p;
            int lo = (blk[(i / 128) * 64 + i % 64] >> (4 * ((i % 128) / 64))) & 0x0F;
            int hi = (blk[128 + (i / 128) * 32 + i % 32] >> (2 * ((i % 128) / 32))) & 0x03;
            out[i] = dl * ((float)(lo | (hi << 4)) - 32.0f);
        }
    }
}

/* One Q8_0 block -> 32 f32.  crates/r9v-format/src/ggml.rs:627-640 (values
 * are the raw bytes at 2+i) and :1094-1100 (w = d * (i8)v). */
static void q80_block(const uint8_t *blk, float *out) {
    float d = rxo_f16_to_f32(rd_u16(blk));
    for (int i = 0; i < 32; ++i) out[i] = d * (float)(int8_t)blk[2 + i];
}

/* IQ3_S codebook: crates/r9v-format/src/iq_lut.rs:629-630, 512 entries of
 * four values, entry e's value b in byte b of word e. */
static const uint32_t IQ3S_GRID[512] = {R9VX_IQ3S_GRID_WORDS};

/* One IQ3_S block (d f16 | qs 64 | qh 8 | signs 32 | scales 4 = 110 B) -> 256
 * f32.  crates/r9v-format/src/iq.rs:698-722 (source_block, Iq3S arm): group g
 * of 32 has db = d * (1 + 2 s), s = nibble g%2 of scales[g/2]; index i = 8g+sg
 * takes grid entry qs[i] | (bit sg of qh[g]) << 8, and value 4 sg + b of the
 * group is (db * grid[b]) negated when bit 4 (sg%2) + b of signs[4g + sg/2]
 * is set. */
static void iq3s_block(const uint8_t *blk, float *out) {
    float d = rxo_f16_to_f32(rd_u16(blk));
    for (int g = 0; g < 8; ++g) {
        uint32_t s = (blk[106 + g / 2] >> ((g % 2) * 4)) & 0x0F;
        float db = d * (1.0f + 2.0f * (float)s);
        for (int sg = 0; sg < 8; ++sg) {
            int i = g * 8 + sg;
            uint32_t idx = blk[2 + i] | (((uint32_t)(blk[66 + g] >> sg) & 1u) << 8);
            uint8_t signs = blk[74 + g * 4 + sg / 2];
            for (int b = 0; b < 4; ++b) {
                float grid = (float)((IQ3S_GRID[idx] >> (8 * b)) & 0xFF);
                float v = db * grid;
                out[g * 32 + sg * 4 + b] = ((signs >> ((sg % 2) * 4 + b)) & 1) ? v * -1.0f : v;
            }
        }
    }
}

/* Byte offset of a block's f16 scale d that check_wire_f16 validates. */
static uint32_t d_offset(int scheme) { return scheme == RXO_Q6_K ? 208 : 0; }

static int check_scales(int scheme, const uint8_t *wire, uint64_t nblocks) {
    uint32_t bb = rxo_block_bytes(scheme);
    for (uint64_t b = 0; b < nblocks; ++b) {
        const uint8_t *blk = wire + b * bb;
        if (!wire_scale_ok(rd_u16(blk + d_offset(scheme)))) return RXO_ERR_SCALE;
        if (scheme == RXO_Q4_K && !wire_scale_ok(rd_u16(blk + 2))) return RXO_ERR_SCALE;
    }
    return RXO_OK;
}

/* Row decode shared by dequantize and the matmul oracles. */
static void decode_row(int scheme, const uint8_t *row, uint32_t k, float *out) {
    uint32_t bb = rxo_block_bytes(scheme), bl = rxo_block_len(scheme);
    for (uint32_t b = 0; b < k / bl; ++b) {
        const uint8_t *blk = row + (uint64_t)b * bb;
        float *o = out + (uint64_t)b * bl;
        if (scheme == RXO_Q4_K)
            q4k_block(blk, o);
        else if (scheme == RXO_IQ4_XS)
            iq4xs_block(blk, o);
        else if (scheme == RXO_Q6_K)
            q6k_block(blk, o);
        else if (scheme == RXO_IQ3_S)
            iq3s_block(blk, o);
        else
            q80_block(blk, o);
    }
}

/* crates/r9v-format/src/ggml.rs:1025-1066 (ggml_dequantize): validate every
 * block, then decode in ascending order. */
int rxo_dequantize(int scheme, const uint8_t *wire, uint32_t n_rows, uint32_t k, float *out) {
    if (rxo_block_bytes(scheme) == 0) return RXO_ERR_SCHEME;
    const uint32_t bl = rxo_block_len(scheme);
    if (k == 0 || k % bl != 0) return RXO_ERR_SHAPE;
    uint64_t nblocks = (uint64_t)n_rows * (k / bl);
    int rc = check_scales(scheme, wire, nblocks);
    if (rc) return rc;
    uint64_t row_bytes = (uint64_t)(k / bl) * rxo_block_bytes(scheme);
    for (uint32_t r = 0; r < n_rows; ++r)
        decode_row(scheme, wire + r * row_bytes, k, out + (uint64_t)r * k);
    return RXO_OK;
}

/* ------------------------------------------------------------------------
 * Branch-D matmul: crates/r9v-t0/src/matmul.rs:1940-2414
 *   for m { for n { acc = 0f32; for k ascending { acc += x_val * w_val } } }
 * The per-element weight formula (matmul.rs:2286-2302, s_block*q - m_block)
 * is the one q4k_block evaluates, so decoding a row once and reusing it is
 * bit-identical to T0's per-element re-decode.  Epilogue matmul.rs:2421-2446;
 * output cast via write_f32_at (dtype.rs:297-330).
 * ---------------------------------------------------------------------- */

static inline float read_x(int x_dtype, const void *x, uint64_t i) {
    if (x_dtype == RXO_BF16) return rxo_bf16_to_f32(((const uint16_t *)x)[i]);
    return ((const float *)x)[i];
}
static inline void write_y(int y_dtype, void *y, uint64_t i, float v) {
    if (y_dtype == RXO_BF16)
        ((uint16_t *)y)[i] = rxo_f32_to_bf16(v);
    else
        ((float *)y)[i] = v;
}

/* Rows per pass of dot_rows: 4 (the checker's default) or 1 (T0's own loop,
 * one row at a time; bench.py times the CPU baseline in this form). */
static int g_rows_at_once = 4;
void rxo_set_rows_at_once(int n) { g_rows_at_once = n == 1 ? 1 : 4; }

/* Branch D's dot (crates/r9v-t0/src/matmul.rs:1940-2414): per output one
 * f32 accumulator from 0, k ascending, prod = x * w rounded, then acc +=
 * prod rounded.  `rows` x rows (stride `xs` floats) against one decoded weight
 * row; four rows run as four independent chains in one pass over k, which
 * changes no row's operations or their order (only how fast they issue). */
static void dot_rows(const float *x, uint32_t rows, uint64_t xs, const float *w, uint32_t k, float *out,
                     uint64_t os) {
    uint32_t r = 0;
    for (; g_rows_at_once == 4 && r + 4 <= rows; r += 4) {
        const float *x0 = x + r * xs, *x1 = x0 + xs, *x2 = x1 + xs, *x3 = x2 + xs;
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
        for (uint32_t kk = 0; kk < k; ++kk) {
            const float wv = w[kk];
            float p0 = x0[kk] * wv, p1 = x1[kk] * wv, p2 = x2[kk] * wv, p3 = x3[kk] * wv;
            a0 += p0;
            a1 += p1;
            a2 += p2;
            a3 += p3;
        }
        out[r * os] = a0;
        out[(r + 1) * os] = a1;
        out[(r + 2) * os] = a2;
        out[(r + 3) * os] = a3;
    }
    for (; r < rows; ++r) {
        float acc = 0.0f;
        for (uint32_t kk = 0; kk < k; ++kk) {
            float prod = x[r * xs + kk] * w[kk];
            acc += prod;
        }
        out[r * os] = acc;
    }
}

/* x [m, k] in x_dtype -> f32 (bf16 -> f32 is exact), NULL on allocation failure. */
static float *x_to_f32(int x_dtype, const void *x, uint32_t m, uint32_t k) {
    float *xf = (float *)malloc(sizeof(float) * (size_t)m * k);
    if (xf)
        for (uint64_t i = 0; i < (uint64_t)m * k; ++i) xf[i] = read_x(x_dtype, x, i);
    return xf;
}

static int matmul_rows(int scheme, const uint8_t *w, uint32_t n0, uint32_t n1, uint32_t n,
                       uint32_t k, const float *xf, uint32_t m, const float *bias,
                       const float *residual, int y_dtype, void *y, float *wrow, float *acc) {
    uint64_t row_bytes = (uint64_t)(k / rxo_block_len(scheme)) * rxo_block_bytes(scheme);
    for (uint32_t col = n0; col < n1; ++col) {
        decode_row(scheme, w + col * row_bytes, k, wrow);
        dot_rows(xf, m, k, wrow, k, acc, 1);
        for (uint32_t r = 0; r < m; ++r) {
            float v = acc[r];
            if (bias) v += bias[col];
            if (residual) v += residual[(uint64_t)r * n + col];
            write_y(y_dtype, y, (uint64_t)r * n + col, v);
        }
    }
    return RXO_OK;
}

static int matmul_validate(int scheme, const uint8_t *w, uint32_t n, uint32_t k, int x_dtype,
                           uint32_t m, const float *bias, const float *residual, int y_dtype) {
    if (rxo_block_bytes(scheme) == 0) return RXO_ERR_SCHEME;
    if (n == 0 || k == 0 || m == 0 || k % 256 != 0) return RXO_ERR_SHAPE;
    if (x_dtype != RXO_F32 && x_dtype != RXO_BF16) return RXO_ERR_DTYPE;
    if (y_dtype != RXO_F32 && y_dtype != RXO_BF16) return RXO_ERR_DTYPE;
    if (bias && residual) return RXO_ERR_SHAPE;
    return check_scales(scheme, w, (uint64_t)n * (k / rxo_block_len(scheme)));
}

int rxo_matmul(int scheme, const uint8_t *w, uint32_t n, uint32_t k, int x_dtype,
               const void *x, uint32_t m, const float *bias, const float *residual,
               int y_dtype, void *y) {
    int rc = matmul_validate(scheme, w, n, k, x_dtype, m, bias, residual, y_dtype);
    if (rc) return rc;
    float *wrow = (float *)malloc(sizeof(float) * k), *acc = (float *)malloc(sizeof(float) * m);
    float *xf = x_to_f32(x_dtype, x, m, k);
    if (wrow && acc && xf) rc = matmul_rows(scheme, w, 0, n, n, k, xf, m, bias, residual, y_dtype, y, wrow, acc);
    else rc = RXO_ERR_SHAPE;
    free(wrow);
    free(acc);
    free(xf);
    return rc;
}

/* Router logits x . w^T for an f32 weight [e, dm] and bf16 x [t, dm]: Branch
 * D's loop order (crates/r9v-t0/src/matmul.rs:1940-2414 -- one f32
 * accumulator per output, k ascending, prod = x*w rounded, then acc += prod). */
void rxo_router_logits(const uint16_t *x, const float *w, uint32_t t, uint32_t e, uint32_t dm, float *out) {
    for (uint32_t r = 0; r < t; ++r)
        for (uint32_t c = 0; c < e; ++c) {
            float acc = 0.0f;
            for (uint32_t k = 0; k < dm; ++k) {
                float prod = rxo_bf16_to_f32(x[(uint64_t)r * dm + k]) * w[(uint64_t)c * dm + k];
                acc += prod;
            }
            out[(uint64_t)r * e + c] = acc;
        }
}

/* act_mul with SiLU: crates/r9v-t0/src/act_mul.rs:86-99 (y = act(g) * u, no
 * clamp) with activation.rs:135-138 (silu(x) = x / (1 + exp(-x)), f32 exp =
 * the host expf). */
void rxo_act_mul_silu(const float *g, const float *u, uint64_t n, float *y) {
    for (uint64_t i = 0; i < n; ++i) {
        float act = g[i] / (1.0f + rxo_expf(-g[i]));
        y[i] = act * u[i];
    }
}

int rxo_matmul_mt(int scheme, const uint8_t *w, uint32_t n, uint32_t k, int x_dtype,
                  const void *x, uint32_t m, int y_dtype, void *y, int threads) {
    int rc = matmul_validate(scheme, w, n, k, x_dtype, m, NULL, NULL, y_dtype);
    if (rc) return rc;
#ifdef _OPENMP
    if (threads < 1) threads = 1;
    float *xf = x_to_f32(x_dtype, x, m, k);
    if (!xf) return RXO_ERR_SHAPE;
    int failed = 0;
#pragma omp parallel num_threads(threads) reduction(| : failed)
    {
        float *wrow = (float *)malloc(sizeof(float) * k), *acc = (float *)malloc(sizeof(float) * m);
        int nt = omp_get_num_threads(), tid = omp_get_thread_num();
        uint32_t chunk = (n + nt - 1) / nt;
        uint32_t n0 = tid * chunk, n1 = n0 + chunk > n ? n : n0 + chunk;
        if (wrow && acc) {
            if (n0 < n1) matmul_rows(scheme, w, n0, n1, n, k, xf, m, NULL, NULL, y_dtype, y, wrow, acc);
        } else {
            failed = 1;
        }
        free(wrow);
        free(acc);
    }
    free(xf);
    return failed ? RXO_ERR_SHAPE : RXO_OK;
#else
    (void)threads;
    return rxo_matmul(scheme, w, n, k, x_dtype, x, m, NULL, NULL, y_dtype, y);
#endif
}

/* ------------------------------------------------------------------------
 * moe_route: crates/r9v-t0/src/moe_route.rs:312-418
 * ---------------------------------------------------------------------- */

/* Rust f32::exp lowers to the platform libm expf (glibc on x86-64 Linux). */
float rxo_expf(float x) { return expf(x); }

/* out[i] = expf of the float whose bits are first_bits + i (the host libm
 * the reference's f32::exp lowers to), for checking a device exp over a
 * range of inputs; rows split over every OpenMP thread. */
void rxo_expf_fill(uint32_t first_bits, uint64_t n, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n; ++i) {
        const uint32_t u = first_bits + (uint32_t)i;
        float x;
        memcpy(&x, &u, 4);
        out[i] = rxo_expf(x);
    }
}

/* total_cmp order (moe_route.rs:373): for finite values this is the IEEE
 * order with -0.0 < +0.0. */
static inline int32_t total_key(float v) {
    int32_t b;
    memcpy(&b, &v, 4);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

int rxo_moe_route(const float *logits, const float *bias, uint32_t t, uint32_t e, uint32_t k,
                  float scale, int renormalize, int scoring, uint32_t *expert_ids,
                  float *weights) {
    if (t == 0 || e == 0 || k == 0 || k > e) return RXO_ERR_SHAPE;
    /* Validation: non-finite logits / bias refused (moe_route.rs:270-311). */
    for (uint64_t i = 0; i < (uint64_t)t * e; ++i)
        if (!isfinite(logits[i])) return RXO_ERR_NONFINITE;
    if (bias)
        for (uint32_t c = 0; c < e; ++c)
            if (!isfinite(bias[c])) return RXO_ERR_NONFINITE;
    uint32_t *sid = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)t * k);
    float *sw = (float *)malloc(sizeof(float) * (size_t)t * k);
    float *scores = (float *)malloc(sizeof(float) * e);
    uint32_t *order = (uint32_t *)malloc(sizeof(uint32_t) * e);
    int rc = RXO_OK;
    for (uint32_t row = 0; row < t && rc == RXO_OK; ++row) {
        for (uint32_t c = 0; c < e; ++c) {
            float s = logits[(uint64_t)row * e + c];
            if (bias) s += bias[c];
            scores[c] = s;
        }
        if (scoring == 0) {
            /* moe_route.rs:331-346: max, sequential exp sum, divide. */
            float mx = scores[0];
            for (uint32_t c = 1; c < e; ++c)
                if (scores[c] > mx) mx = scores[c];
            float sum = 0.0f;
            for (uint32_t c = 0; c < e; ++c) {
                float v = rxo_expf(scores[c] - mx);
                scores[c] = v;
                sum += v;
            }
            for (uint32_t c = 0; c < e; ++c) scores[c] /= sum;
        } else {
            /* moe_route.rs:347-351: sigmoid. */
            for (uint32_t c = 0; c < e; ++c) scores[c] = 1.0f / (1.0f + rxo_expf(-scores[c]));
        }
        for (uint32_t c = 0; c < e; ++c)
            if (!isfinite(scores[c])) rc = RXO_ERR_NONFINITE;
        if (rc) break;
        /* Stable selection of the K best by (score desc total_cmp, id asc),
         * equal to the first K of the reference's full stable sort. */
        for (uint32_t c = 0; c < e; ++c) order[c] = c;
        for (uint32_t j = 0; j < k; ++j) {
            uint32_t best = j;
            for (uint32_t c = j + 1; c < e; ++c) {
                int32_t kb = total_key(scores[order[best]]), kc = total_key(scores[order[c]]);
                if (kc > kb || (kc == kb && order[c] < order[best])) best = c;
            }
            uint32_t tmp = order[j];
            order[j] = order[best];
            order[best] = tmp;
        }
        /* moe_route.rs:374-398: scale, sequential selected sum, renormalise. */
        float selected_sum = 0.0f;
        for (uint32_t j = 0; j < k; ++j) {
            uint32_t col = order[j];
            float w = scores[col] * scale;
            sid[(uint64_t)row * k + j] = col;
            sw[(uint64_t)row * k + j] = w;
            selected_sum += w;
        }
        if (renormalize) {
            if (!isfinite(selected_sum) || selected_sum == 0.0f) {
                rc = RXO_ERR_NONFINITE;
                break;
            }
            for (uint32_t j = 0; j < k; ++j) sw[(uint64_t)row * k + j] /= selected_sum;
        }
        for (uint32_t j = 0; j < k; ++j)
            if (!isfinite(sw[(uint64_t)row * k + j])) rc = RXO_ERR_NONFINITE;
    }
    if (rc == RXO_OK) {
        memcpy(expert_ids, sid, sizeof(uint32_t) * (size_t)t * k);
        memcpy(weights, sw, sizeof(float) * (size_t)t * k);
    }
    free(sid);
    free(sw);
    free(scores);
    free(order);
    return rc;
}

/* ------------------------------------------------------------------------
 * Permute: the stable (expert, token) triple sort of
 * crates/r9v-t0/src/moe_ffn.rs:477-493, as a counting sort (stable by
 * construction: pairs visited in ascending (token, slot) order).
 * ---------------------------------------------------------------------- */
int rxo_moe_sort(const uint32_t *ids, uint32_t t, uint32_t k, uint32_t e, uint32_t *counts,
                 uint32_t *offsets, uint32_t *sorted) {
    uint64_t p = (uint64_t)t * k;
    for (uint64_t i = 0; i < p; ++i)
        if (ids[i] >= e) return RXO_ERR_ID;
    memset(counts, 0, sizeof(uint32_t) * e);
    for (uint64_t i = 0; i < p; ++i) counts[ids[i]]++;
    uint32_t acc = 0;
    for (uint32_t x = 0; x < e; ++x) {
        offsets[x] = acc;
        acc += counts[x];
    }
    offsets[e] = acc;
    uint32_t *cursor = (uint32_t *)malloc(sizeof(uint32_t) * e);
    memcpy(cursor, offsets, sizeof(uint32_t) * e);
    for (uint64_t i = 0; i < p; ++i) sorted[cursor[ids[i]]++] = (uint32_t)i;
    free(cursor);
    return RXO_OK;
}

/* ------------------------------------------------------------------------
 * moe_ffn, sliced per expert: crates/r9v-t0/src/moe_ffn.rs:527-653
 * ---------------------------------------------------------------------- */

/* SiLU: crates/r9v-t0/src/activation.rs:135-138, x / (1 + exp(-x));
 * act_mul: crates/r9v-t0/src/act_mul.rs:86-99, act(g) * u. */
static inline float silu_mul(float g, float u) {
    float den = 1.0f + rxo_expf(-g);
    float a = g / den;
    return a * u;
}

/* One expert over `rows` gathered activation rows (x_rows is f32 [rows, dm]
 * holding the exact activation values).  gate/up rows [0,Dff) and [Dff,2Dff)
 * of the expert's [2Dff, Dm] block (moe_ffn.rs:51-55); Branch-D accumulation
 * for gate/up (matmul.rs:1940-2414) and down (moe_ffn.rs:1357-1456). */
static void expert_rows(const float *x_rows, uint32_t rows, uint32_t dm, uint32_t dff,
                        int scheme_gu, const uint8_t *gu, int scheme_dn, const uint8_t *dn,
                        int h_bf16, float *out, float *wrow, float *h) {
    uint64_t gu_row_bytes = wire_row_bytes(scheme_gu, dm);
    uint64_t dn_row_bytes = wire_row_bytes(scheme_dn, dff);
    float *gate = (float *)malloc(sizeof(float) * (size_t)rows * dff);
    float *up = (float *)malloc(sizeof(float) * (size_t)rows);
    for (uint32_t c = 0; c < 2 * dff; ++c) {
        decode_row(scheme_gu, gu + c * gu_row_bytes, dm, wrow);
        if (c < dff) {
            dot_rows(x_rows, rows, dm, wrow, dm, gate + c, dff);
            continue;
        }
        dot_rows(x_rows, rows, dm, wrow, dm, up, 1);
        for (uint32_t r = 0; r < rows; ++r) {
            float v = silu_mul(gate[(uint64_t)r * dff + (c - dff)], up[r]);
            if (h_bf16) v = rxo_bf16_to_f32(rxo_f32_to_bf16(v));
            h[(uint64_t)r * dff + (c - dff)] = v;
        }
    }
    free(up);
    free(gate);
    for (uint32_t d = 0; d < dm; ++d) {
        decode_row(scheme_dn, dn + d * dn_row_bytes, dff, wrow);
        dot_rows(h, rows, dff, wrow, dff, out + d, dm);
    }
}

static int ffn_validate(int x_dtype, uint32_t t, uint32_t dm, uint32_t dff, uint32_t e_all,
                        int scheme_gu, const uint8_t *gu, int scheme_dn, const uint8_t *dn) {
    if (x_dtype != RXO_F32 && x_dtype != RXO_BF16) return RXO_ERR_DTYPE;
    if (rxo_block_bytes(scheme_gu) == 0 || rxo_block_bytes(scheme_dn) == 0) return RXO_ERR_SCHEME;
    if (t == 0 || dm == 0 || dff == 0 || dm % 256 || dff % 256) return RXO_ERR_SHAPE;
    int rc = check_scales(scheme_gu, gu, (uint64_t)e_all * 2 * dff * (dm / 256));
    if (rc) return rc;
    return check_scales(scheme_dn, dn, (uint64_t)e_all * dm * (dff / 256));
}

int rxo_expert_ffn(int x_dtype, const void *x, uint32_t rows, uint32_t dm, uint32_t dff,
                   int scheme_gu, const uint8_t *gu, int scheme_dn, const uint8_t *dn,
                   int h_bf16, float *out) {
    int rc = ffn_validate(x_dtype, rows, dm, dff, 1, scheme_gu, gu, scheme_dn, dn);
    if (rc) return rc;
    float *xr = (float *)malloc(sizeof(float) * (size_t)rows * dm);
    for (uint64_t i = 0; i < (uint64_t)rows * dm; ++i) xr[i] = read_x(x_dtype, x, i);
    float *wrow = (float *)malloc(sizeof(float) * (dm > dff ? dm : dff));
    float *h = (float *)malloc(sizeof(float) * (size_t)rows * dff);
    expert_rows(xr, rows, dm, dff, scheme_gu, gu, scheme_dn, dn, h_bf16, out, wrow, h);
    free(xr);
    free(wrow);
    free(h);
    return RXO_OK;
}

/* rxo_moe_ffn with its expert FFNs spread over `threads` OpenMP threads:
 * every routed expert's unique tokens (and every token for each shared
 * expert) are cut into chunks of rows, each chunk computed independently
 * (a row's result does not depend on the rows beside it), and the combine
 * then runs serially in T0's order, so y is bit-identical for every thread
 * count. */
#define RXO_FFN_CHUNK 64u
int rxo_moe_ffn_mt(int x_dtype, const void *x, uint32_t t, uint32_t dm, uint32_t dff, uint32_t e,
                   uint32_t s_shared, uint32_t k, const uint32_t *ids, const float *weights, int scheme_gu,
                   const uint8_t *gu, int scheme_dn, const uint8_t *dn, int h_bf16, float *y, int threads) {
    int rc = ffn_validate(x_dtype, t, dm, dff, e + s_shared, scheme_gu, gu, scheme_dn, dn);
    if (rc) return rc;
    if (k == 0) return RXO_ERR_SHAPE;
    if (threads < 1) threads = 1;
    uint64_t p = (uint64_t)t * k;
    uint32_t *counts = (uint32_t *)malloc(sizeof(uint32_t) * e);
    uint32_t *offsets = (uint32_t *)malloc(sizeof(uint32_t) * (e + 1));
    uint32_t *sorted = (uint32_t *)malloc(sizeof(uint32_t) * p);
    /* rows of the unique-token runs: run of expert ex at [offsets[ex], +run_len[ex]) */
    uint32_t *run_tok = (uint32_t *)malloc(sizeof(uint32_t) * p);
    uint32_t *run_len = (uint32_t *)calloc(e, sizeof(uint32_t));
    float *o = (float *)malloc(sizeof(float) * (size_t)(p + (uint64_t)s_shared * t) * dm);
    float *ytmp = (float *)calloc((size_t)t * dm, sizeof(float));
    if (!counts || !offsets || !sorted || !run_tok || !run_len || !o || !ytmp) rc = RXO_ERR_SHAPE;
    if (!rc) rc = rxo_moe_sort(ids, t, k, e, counts, offsets, sorted);
    uint64_t n_items = 0;
    uint32_t *item_run = NULL, *item_r0 = NULL;
    if (!rc) {
        /* Unique ascending tokens of each expert's run (moe_ffn.rs:527-545). */
        for (uint32_t ex = 0; ex < e; ++ex) {
            uint32_t le = 0;
            for (uint32_t i = offsets[ex]; i < offsets[ex + 1]; ++i) {
                uint32_t tok = sorted[i] / k;
                if (le == 0 || run_tok[offsets[ex] + le - 1] != tok) run_tok[offsets[ex] + le++] = tok;
            }
            run_len[ex] = le;
            n_items += (le + RXO_FFN_CHUNK - 1) / RXO_FFN_CHUNK;
        }
        n_items += (uint64_t)s_shared * ((t + RXO_FFN_CHUNK - 1) / RXO_FFN_CHUNK);
        item_run = (uint32_t *)malloc(sizeof(uint32_t) * (n_items + 1));
        item_r0 = (uint32_t *)malloc(sizeof(uint32_t) * (n_items + 1));
        if (!item_run || !item_r0) rc = RXO_ERR_SHAPE;
    }
    if (!rc) {
        uint64_t it = 0;
        for (uint32_t ex = 0; ex < e + s_shared; ++ex) {
            const uint32_t len = ex < e ? run_len[ex] : t;
            for (uint32_t r0 = 0; r0 < len; r0 += RXO_FFN_CHUNK) item_run[it] = ex, item_r0[it++] = r0;
        }
        const uint64_t gu_expert = (uint64_t)2 * dff * wire_row_bytes(scheme_gu, dm);
        const uint64_t dn_expert = (uint64_t)dm * wire_row_bytes(scheme_dn, dff);
        int failed = 0;
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1) reduction(| : failed)
#endif
        for (int64_t i = 0; i < (int64_t)n_items; ++i) {
            const uint32_t ex = item_run[i], r0 = item_r0[i];
            const uint32_t len = ex < e ? run_len[ex] : t;
            const uint32_t rows = len - r0 < RXO_FFN_CHUNK ? len - r0 : RXO_FFN_CHUNK;
            /* output rows: routed runs at their pair offsets, shared experts after the P pair rows */
            const uint64_t orow = ex < e ? (uint64_t)offsets[ex] + r0 : p + (uint64_t)(ex - e) * t + r0;
            float *xr = (float *)malloc(sizeof(float) * (size_t)rows * dm);
            float *h = (float *)malloc(sizeof(float) * (size_t)rows * dff);
            float *wrow = (float *)malloc(sizeof(float) * (dm > dff ? dm : dff));
            if (xr && h && wrow) {
                for (uint32_t r = 0; r < rows; ++r) {
                    const uint32_t tok = ex < e ? run_tok[offsets[ex] + r0 + r] : r0 + r;
                    for (uint32_t kk = 0; kk < dm; ++kk)
                        xr[(uint64_t)r * dm + kk] = read_x(x_dtype, x, (uint64_t)tok * dm + kk);
                }
                expert_rows(xr, rows, dm, dff, scheme_gu, gu + ex * gu_expert, scheme_dn, dn + ex * dn_expert,
                            h_bf16, o + orow * dm, wrow, h);
            } else {
                failed = 1;
            }
            free(xr);
            free(h);
            free(wrow);
        }
        if (failed) rc = RXO_ERR_SHAPE;
    }
    if (!rc) {
        /* Weighted combine, experts ascending, each run in (token, slot) order
         * (moe_ffn.rs:641-653). */
        for (uint32_t ex = 0; ex < e; ++ex) {
            uint32_t r = 0;
            const uint32_t *tokens = run_tok + offsets[ex];
            const float *out = o + (uint64_t)offsets[ex] * dm;
            for (uint32_t i = offsets[ex]; i < offsets[ex + 1]; ++i) {
                uint32_t tok = sorted[i] / k, slot = sorted[i] % k;
                while (tokens[r] != tok) ++r;
                float w = weights[(uint64_t)tok * k + slot];
                for (uint32_t d = 0; d < dm; ++d) {
                    float prod = w * out[(uint64_t)r * dm + d];
                    ytmp[(uint64_t)tok * dm + d] += prod;
                }
            }
        }
        /* Shared experts: every token, weight 1.0, added after the routed
         * combine (crates/r9v-models/src/generic.rs:1458-1495 residual add). */
        for (uint32_t sidx = 0; sidx < s_shared; ++sidx) {
            const float *out = o + (p + (uint64_t)sidx * t) * dm;
            for (uint64_t i = 0; i < (uint64_t)t * dm; ++i) ytmp[i] += out[i];
        }
        memcpy(y, ytmp, sizeof(float) * (size_t)t * dm);
    }
    free(item_run);
    free(item_r0);
    free(ytmp);
    free(o);
    free(run_len);
    free(run_tok);
    free(counts);
    free(offsets);
    free(sorted);
    return rc;
}

int rxo_moe_ffn(int x_dtype, const void *x, uint32_t t, uint32_t dm, uint32_t dff, uint32_t e,
                uint32_t s_shared, uint32_t k, const uint32_t *ids, const float *weights,
                int scheme_gu, const uint8_t *gu, int scheme_dn, const uint8_t *dn, int h_bf16,
                float *y) {
    return rxo_moe_ffn_mt(x_dtype, x, t, dm, dff, e, s_shared, k, ids, weights, scheme_gu, gu, scheme_dn, dn, h_bf16,
                          y, 1);
}

/* One expert's FFN over the token rows `tokens` (the per-expert body of
 * rxo_moe_ffn: gather, gate/up, act_mul, down; moe_ffn.rs:527-639), rows
 * split over `threads` OpenMP threads (each row is independent, so the
 * result does not depend on the split).  out: [n_tok, dm].  The CPU
 * baseline of the grouped MoE GEMM times this on a subset of experts. */
int rxo_moe_expert_mt(int x_dtype, const void *x, const uint32_t *tokens, uint32_t n_tok, uint32_t dm,
                      uint32_t dff, int scheme_gu, const uint8_t *gu, int scheme_dn, const uint8_t *dn, float *out,
                      int threads) {
    if (dm == 0 || dff == 0 || dm % 256 || dff % 256) return RXO_ERR_SHAPE;
    if (threads < 1) threads = 1;
#ifdef _OPENMP
#pragma omp parallel num_threads(threads)
#endif
    {
#ifdef _OPENMP
        int nt = omp_get_num_threads(), tid = omp_get_thread_num();
#else
        int nt = 1, tid = 0;
#endif
        uint32_t chunk = (n_tok + nt - 1) / nt;
        uint32_t r0 = tid * chunk, r1 = r0 + chunk > n_tok ? n_tok : r0 + chunk;
        if (r0 < r1) {
            uint32_t rows = r1 - r0;
            float *xr = (float *)malloc(sizeof(float) * (size_t)rows * dm);
            float *wrow = (float *)malloc(sizeof(float) * (dm > dff ? dm : dff));
            float *h = (float *)malloc(sizeof(float) * (size_t)rows * dff);
            for (uint32_t r = 0; r < rows; ++r)
                for (uint32_t kk = 0; kk < dm; ++kk)
                    xr[(uint64_t)r * dm + kk] = read_x(x_dtype, x, (uint64_t)tokens[r0 + r] * dm + kk);
            expert_rows(xr, rows, dm, dff, scheme_gu, gu, scheme_dn, dn, 0, out + (uint64_t)r0 * dm, wrow, h);
            free(xr);
            free(wrow);
            free(h);
        }
    }
    return RXO_OK;
}

/* Literal T0 form: gate/up over every expert's rows, then slice the
 * expert's columns (moe_ffn.rs:575-612).  Tiny E only. */
int rxo_moe_ffn_full(int x_dtype, const void *x, uint32_t t, uint32_t dm, uint32_t dff,
                     uint32_t e, uint32_t k, const uint32_t *ids, const float *weights,
                     int scheme_gu, const uint8_t *gu, int scheme_dn, const uint8_t *dn,
                     float *y) {
    int rc = ffn_validate(x_dtype, t, dm, dff, e, scheme_gu, gu, scheme_dn, dn);
    if (rc) return rc;
    uint64_t p = (uint64_t)t * k;
    uint32_t *counts = (uint32_t *)malloc(sizeof(uint32_t) * e);
    uint32_t *offsets = (uint32_t *)malloc(sizeof(uint32_t) * (e + 1));
    uint32_t *sorted = (uint32_t *)malloc(sizeof(uint32_t) * p);
    rc = rxo_moe_sort(ids, t, k, e, counts, offsets, sorted);
    if (rc) {
        free(counts);
        free(offsets);
        free(sorted);
        return rc;
    }
    uint32_t h_width = 2 * e * dff;
    float *ytmp = (float *)calloc((size_t)t * dm, sizeof(float));
    float *xr = (float *)malloc(sizeof(float) * (size_t)t * dm);
    float *h_all = (float *)malloc(sizeof(float) * (size_t)t * h_width);
    float *h = (float *)malloc(sizeof(float) * (size_t)t * dff);
    float *out = (float *)malloc(sizeof(float) * (size_t)t * dm);
    float *wrow = (float *)malloc(sizeof(float) * (dm > dff ? dm : dff));
    uint32_t *tokens = (uint32_t *)malloc(sizeof(uint32_t) * (t + 1));
    uint64_t gu_row_bytes = wire_row_bytes(scheme_gu, dm);
    uint64_t dn_row_bytes = wire_row_bytes(scheme_dn, dff);
    for (uint32_t ex = 0; ex < e; ++ex) {
        uint32_t beg = offsets[ex], end = offsets[ex + 1];
        if (beg == end) continue;
        uint32_t le = 0;
        for (uint32_t i = beg; i < end; ++i) {
            uint32_t tok = sorted[i] / k;
            if (le == 0 || tokens[le - 1] != tok) tokens[le++] = tok;
        }
        for (uint32_t r = 0; r < le; ++r)
            for (uint32_t kk = 0; kk < dm; ++kk)
                xr[(uint64_t)r * dm + kk] = read_x(x_dtype, x, (uint64_t)tokens[r] * dm + kk);
        for (uint32_t c = 0; c < h_width; ++c) {
            decode_row(scheme_gu, gu + c * gu_row_bytes, dm, wrow);
            for (uint32_t r = 0; r < le; ++r) {
                float acc = 0.0f;
                for (uint32_t kk = 0; kk < dm; ++kk) {
                    float prod = xr[(uint64_t)r * dm + kk] * wrow[kk];
                    acc += prod;
                }
                h_all[(uint64_t)r * h_width + c] = acc;
            }
        }
        uint32_t base = ex * 2 * dff;
        for (uint32_t r = 0; r < le; ++r)
            for (uint32_t d = 0; d < dff; ++d)
                h[(uint64_t)r * dff + d] = silu_mul(h_all[(uint64_t)r * h_width + base + d],
                                                    h_all[(uint64_t)r * h_width + base + dff + d]);
        for (uint32_t d = 0; d < dm; ++d) {
            decode_row(scheme_dn, dn + ((uint64_t)ex * dm + d) * dn_row_bytes, dff, wrow);
            for (uint32_t r = 0; r < le; ++r) {
                float acc = 0.0f;
                for (uint32_t kk = 0; kk < dff; ++kk) {
                    float prod = h[(uint64_t)r * dff + kk] * wrow[kk];
                    acc += prod;
                }
                out[(uint64_t)r * dm + d] = acc;
            }
        }
        uint32_t r = 0;
        for (uint32_t i = beg; i < end; ++i) {
            uint32_t tok = sorted[i] / k, slot = sorted[i] % k;
            while (tokens[r] != tok) ++r;
            float w = weights[(uint64_t)tok * k + slot];
            for (uint32_t d = 0; d < dm; ++d) {
                float prod = w * out[(uint64_t)r * dm + d];
                ytmp[(uint64_t)tok * dm + d] += prod;
            }
        }
    }
    memcpy(y, ytmp, sizeof(float) * (size_t)t * dm);
    free(ytmp);
    free(xr);
    free(h_all);
    free(h);
    free(out);
    free(wrow);
    free(tokens);
    free(counts);
    free(offsets);
    free(sorted);
    return RXO_OK;
}
