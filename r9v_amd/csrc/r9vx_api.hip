/*
 * r9vx_api.hip -- the C ABI of include/r9vx.h: host-side validation that
 * mirrors T0's collect-all refusal (every problem is reported, nothing is
 * enqueued when any is found), variant selection by shape, and launch.
 *
 * Validation mirrors crates/r9v-t0/src/matmul.rs:60-411 (rank/dtype/scheme/
 * epilogue checks), moe_route.rs:96-311 and moe_ffn.rs:95-465, restricted to
 * what a host can see without reading device memory.
 */
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>

#include "r9vx_internal.h"
#include "r9vx_moe.h"
#include "r9vx_probe.h"

namespace {

thread_local std::string g_last_error;

struct Problems {
    std::string text;
    int code = R9VX_OK;
    void add(int c, const char *fmt, ...) {
        char buf[256];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        if (!text.empty()) text += "; ";
        text += buf;
        if (code == R9VX_OK) code = c;
    }
    int finish(const char *op) {
        if (code != R9VX_OK) g_last_error = std::string(op) + ": " + text;
        return code;
    }
};

int hip_status(const char *op, int rc) {
    if (rc != 0) {
        g_last_error = std::string(op) + ": HIP error " + std::to_string(rc) + " (" +
                       hipGetErrorString((hipError_t)rc) + ")";
    }
    return rc;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

/* Schemes read as GGUF wire blocks (every op), the ones read in the split
 * layout of r9vx_repack_launch (body + d array), and IQ3_S, read as the
 * 112-byte blocks of r9vx_repack_launch (one array). */
bool known_scheme(uint32_t s) { return s == R9VX_SCHEME_Q4_K || s == R9VX_SCHEME_IQ4_XS; }
bool split_scheme(uint32_t s) { return s == R9VX_SCHEME_Q8_0 || s == R9VX_SCHEME_Q6_K; }
bool packed_scheme(uint32_t s) { return s == R9VX_SCHEME_IQ3_S; }
bool repacked_scheme(uint32_t s) { return split_scheme(s) || packed_scheme(s); }
bool matmul_scheme(uint32_t s) { return known_scheme(s) || repacked_scheme(s); }

uint32_t block_bytes(uint32_t s) {
    switch (s) {
    case R9VX_SCHEME_Q4_K: return R9VX_Q4K_BYTES;
    case R9VX_SCHEME_IQ4_XS: return R9VX_IQ4XS_BYTES;
    case R9VX_SCHEME_Q6_K: return R9VX_Q6K_BYTES;
    case R9VX_SCHEME_Q8_0: return R9VX_Q80_BYTES;
    case R9VX_SCHEME_IQ3_S: return R9VX_IQ3S_BYTES;
    default: return 0;
    }
}
uint32_t block_len(uint32_t s) { return s == R9VX_SCHEME_Q8_0 ? 32 : 256; }

/* The weight element type and device layout each scheme is read in. */
uint32_t scheme_dtype(uint32_t s) {
    return s == R9VX_SCHEME_Q8_0 || s == R9VX_SCHEME_Q6_K ? R9VX_DTYPE_I8 : R9VX_DTYPE_I4;
}
uint32_t scheme_layout(uint32_t s) {
    if (s == R9VX_SCHEME_Q8_0 || s == R9VX_SCHEME_Q6_K) return R9VX_LAYOUT_SPLIT;
    if (s == R9VX_SCHEME_IQ3_S) return R9VX_LAYOUT_IQ3S_112;
    return R9VX_LAYOUT_GGUF_WIRE;
}
const char *layout_name(uint32_t l) {
    switch (l) {
    case R9VX_LAYOUT_CONTIGUOUS: return "contiguous";
    case R9VX_LAYOUT_L0: return "L0";
    case R9VX_LAYOUT_L1: return "L1";
    case R9VX_LAYOUT_L1S: return "L1S";
    case R9VX_LAYOUT_GGUF_WIRE: return "gguf_wire";
    case R9VX_LAYOUT_SPLIT: return "split";
    case R9VX_LAYOUT_IQ3S_112: return "iq3s_112";
    default: return "unknown";
    }
}

/* A weight's element type and layout must be the ones this path reads for
 * its scheme: the reference's native layouts (L0 row-major records, L1 / L1S
 * tiles, crates/r9v-format/src/repack.rs:274-287) are refused, not misread. */
void check_weight_keys(const char *what, uint32_t scheme, uint32_t dtype, uint32_t layout, Problems &pr) {
    if (layout != scheme_layout(scheme))
        pr.add(R9VX_ERR_UNSUPPORTED, "%s layout %u (%s): scheme %u is read in the %s layout (code %u) only", what,
               layout, layout_name(layout), scheme, layout_name(scheme_layout(scheme)), scheme_layout(scheme));
    if (dtype != scheme_dtype(scheme))
        pr.add(R9VX_ERR_UNSUPPORTED, "%s dtype %u: scheme %u weights are dtype %u", what, dtype, scheme,
               scheme_dtype(scheme));
}

/* Bytes of one weight row as the kernels read it (the split layout's body;
 * its d values add r9vx_row_scales f16 per row). */
uint64_t device_row_bytes(uint32_t s, uint32_t k) { return r9vx_row_bytes(s, k); }

}  // namespace

/* Sets the calling thread's r9vx_last_error() text (used by the other host
 * sources of the library). */
void r9vx_set_last_error(const std::string &text) { g_last_error = text; }

extern "C" {

const char *r9vx_last_error(void) { return g_last_error.c_str(); }

uint32_t r9vx_abi_version(void) { return R9VX_ABI_VERSION; }

/* ------------------------------------------------------------------ matmul */

static void check_matmul_static(const r9vx_matmul_static *st, Problems &pr) {
    if (!matmul_scheme(st->w_scheme))
        pr.add(R9VX_ERR_UNSUPPORTED, "w_scheme %u is not the SchemeId code of Q4_K (3), Q8_0 (5), Q6_K (11), IQ4_XS (15) "
               "or IQ3_S (17)", st->w_scheme);
    if (repacked_scheme(st->w_scheme) && st->in_dtype != R9VX_DTYPE_BF16)
        pr.add(R9VX_ERR_UNSUPPORTED, "w_scheme %u takes bf16 activations only", st->w_scheme);

    if (st->k == 0 || st->k % 256)
        pr.add(R9VX_ERR_INVALID, "k=%u must be a positive multiple of the 256-weight super-block", st->k);
    if (st->n == 0) pr.add(R9VX_ERR_INVALID, "n must be positive");
    if (st->in_dtype != R9VX_DTYPE_F32 && st->in_dtype != R9VX_DTYPE_BF16)
        pr.add(R9VX_ERR_UNSUPPORTED, "in_dtype %u: only f32 and bf16 activations", st->in_dtype);
    if (st->out_dtype != R9VX_DTYPE_F32 && st->out_dtype != R9VX_DTYPE_BF16)
        pr.add(R9VX_ERR_UNSUPPORTED, "out_dtype %u: only f32 and bf16 outputs", st->out_dtype);
    if (st->epilogue > R9VX_EPILOGUE_SWIGLU)
        pr.add(R9VX_ERR_UNSUPPORTED, "epilogue %u: only none/bias/residual/swiglu", st->epilogue);
    if (st->epilogue == R9VX_EPILOGUE_SWIGLU && (st->in_dtype != R9VX_DTYPE_BF16 || st->m_bucket > 8))
        pr.add(R9VX_ERR_UNSUPPORTED, "the swiglu epilogue runs the decode GEMV only: bf16 activations, m_bucket <= 8");
    if (st->epilogue == R9VX_EPILOGUE_RESIDUAL && st->residual_dtype != R9VX_DTYPE_F32)
        pr.add(R9VX_ERR_UNSUPPORTED, "residual_dtype %u: only f32 residuals", st->residual_dtype);
    if (matmul_scheme(st->w_scheme)) check_weight_keys("w", st->w_scheme, st->w_dtype, st->w_layout, pr);
    if (st->act_scheme != R9VX_ACT_SCHEME_NONE)
        pr.add(R9VX_ERR_UNSUPPORTED, "act_scheme %u: activations are not quantized on this path", st->act_scheme);
    if (st->transpose_w) pr.add(R9VX_ERR_UNSUPPORTED, "transpose_w: weights are [N, K] rows of blocks");
    if (st->interleave) pr.add(R9VX_ERR_UNSUPPORTED, "interleave is not implemented");
    if (st->sparse) pr.add(R9VX_ERR_UNSUPPORTED, "sparse (2:4) weights are not implemented");
}

/* The MFMA path (bf16 activations, m_bucket > 8) stages x as fp16 rows plus per-row
 * scales in the workspace; the GEMV path needs none. */
size_t r9vx_matmul_workspace_bytes(const r9vx_matmul_static *st) {
    if (!st || st->in_dtype != R9VX_DTYPE_BF16 || st->m_bucket <= 8) return 0;
    return r9vx_gemm_workspace_bytes(st->m_bucket, st->k);
}

uint64_t r9vx_matmul_static_bytes(const r9vx_matmul_static *st, uint32_t m) {
    if (!st || !matmul_scheme(st->w_scheme)) return 0;
    const uint64_t w_rows = st->epilogue == R9VX_EPILOGUE_SWIGLU ? 2ull * st->n : st->n;
    /* the device layout's bytes (IQ3_S: 112-byte blocks; split layouts hold the wire bytes) */
    uint64_t w = w_rows * (split_scheme(st->w_scheme) ? (st->k / block_len(st->w_scheme)) * block_bytes(st->w_scheme)
                                                       : device_row_bytes(st->w_scheme, st->k));
    uint64_t xe = st->in_dtype == R9VX_DTYPE_F32 ? 4 : 2;
    uint64_t ye = st->out_dtype == R9VX_DTYPE_F32 ? 4 : 2;
    return w + (uint64_t)m * st->k * xe + (uint64_t)m * st->n * ye;
}

uint64_t r9vx_matmul_static_flops(const r9vx_matmul_static *st, uint32_t m) {
    if (!st) return 0;
    return (st->epilogue == R9VX_EPILOGUE_SWIGLU ? 4ull : 2ull) * m * st->n * st->k;
}

int r9vx_matmul_launch(const r9vx_matmul_static *st, const r9vx_matmul_args *a,
                       r9vx_stream_t stream) {
    Problems pr;
    if (!st || !a) {
        pr.add(R9VX_ERR_NULL, "static and args must be non-NULL");
        return pr.finish("matmul");
    }
    check_matmul_static(st, pr);
    if (a->m > st->m_bucket)
        pr.add(R9VX_ERR_INVALID, "m=%u exceeds m_bucket=%u", a->m, st->m_bucket);
    if (a->m > 0) {
        if (!a->w) pr.add(R9VX_ERR_NULL, "w is NULL");
        if (!a->x) pr.add(R9VX_ERR_NULL, "x is NULL");
        if (!a->y) pr.add(R9VX_ERR_NULL, "y is NULL");
    }
    if (a->w_scales && !split_scheme(st->w_scheme))
        pr.add(R9VX_ERR_UNSUPPORTED, "w_scales must be NULL: Q4_K / IQ4_XS / IQ3_S blocks carry inline scales");
    if (split_scheme(st->w_scheme) && a->m > 0 && !a->w_scales)
        pr.add(R9VX_ERR_NULL, "w_scales (the f16 d array of the split layout) is NULL");
    if (a->w_scales && ((uintptr_t)a->w_scales & 1u)) pr.add(R9VX_ERR_ALIGN, "w_scales must be 2-byte aligned");
    if (a->w_indices) pr.add(R9VX_ERR_UNSUPPORTED, "w_indices must be NULL: no sparse weights");
    if (a->x_scale) pr.add(R9VX_ERR_UNSUPPORTED, "x_scale must be NULL: activations are not quantized");
    if (st->epilogue == R9VX_EPILOGUE_BIAS && !a->bias) pr.add(R9VX_ERR_NULL, "bias epilogue without bias");
    if (st->epilogue != R9VX_EPILOGUE_BIAS && a->bias) pr.add(R9VX_ERR_INVALID, "bias given without bias epilogue");
    if (st->epilogue == R9VX_EPILOGUE_RESIDUAL && !a->residual)
        pr.add(R9VX_ERR_NULL, "residual epilogue without residual");
    if (st->epilogue != R9VX_EPILOGUE_RESIDUAL && a->residual)
        pr.add(R9VX_ERR_INVALID, "residual given without residual epilogue");
    if ((a->w && !aligned16(a->w)) || (a->x && !aligned16(a->x)) || (a->y && !aligned16(a->y)))
        pr.add(R9VX_ERR_ALIGN, "w, x and y must be 16-byte aligned");
    if (st->in_dtype == R9VX_DTYPE_BF16 && st->m_bucket > 8 && a->m > 0) {
        if (!a->workspace)
            pr.add(R9VX_ERR_WORKSPACE, "m_bucket=%u > 8 runs the MFMA path: workspace of r9vx_matmul_workspace_bytes required",
                   st->m_bucket);
        else if ((uintptr_t)a->workspace & 255u)
            pr.add(R9VX_ERR_ALIGN, "workspace must be 256-byte aligned");
    }
    int rc = pr.finish("matmul");
    if (rc || a->m == 0) return rc;

    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const uint64_t w_row = device_row_bytes(st->w_scheme, st->k);
    /* The path is chosen by the variant's bucket, not by m: every launch of
     * one static runs the same kernels with the same per-element arithmetic,
     * so a row's outputs do not depend on the rows beside it (the
     * batch-invariance gate, crates/r9v-t0/src/harness.rs:903-948).  Buckets
     * <= 8 run the GEMV, bf16 buckets above run the MFMA GEMM. */
    const bool mfma = st->in_dtype == R9VX_DTYPE_BF16 && st->m_bucket > 8;
    if (mfma) {
        r9vx_gemm_problem g{};
        g.w = a->w;
        g.w_scales = reinterpret_cast<const uint16_t *>(a->w_scales);
        g.x = reinterpret_cast<const uint16_t *>(a->x);
        g.bias = a->bias;
        g.residual = reinterpret_cast<const float *>(a->residual);
        g.y = a->y;
        g.workspace = a->workspace;
        g.n = st->n;
        g.k = st->k;
        g.m = a->m;
        g.m_bucket = st->m_bucket;
        g.scheme = st->w_scheme;
        g.y_dtype = st->out_dtype;
        g.epilogue = st->epilogue;
        return hip_status("matmul", r9vx_launch_gemm(g, s));
    }
    /* GEMV, eight activation rows per launch. */
    const uint32_t xe = st->in_dtype == R9VX_DTYPE_F32 ? 4 : 2;
    const uint32_t ye = st->out_dtype == R9VX_DTYPE_F32 ? 4 : 2;
    for (uint32_t m0 = 0; m0 < a->m; m0 += 8) {
        r9vx_gemv_problem p{};
        p.w = a->w;
        p.w_scales = reinterpret_cast<const uint16_t *>(a->w_scales);
        p.x = reinterpret_cast<const uint8_t *>(a->x) + (uint64_t)m0 * st->k * xe;
        p.bias = a->bias;
        p.residual = a->residual ? reinterpret_cast<const float *>(a->residual) + (uint64_t)m0 * st->n : nullptr;
        p.y = reinterpret_cast<uint8_t *>(a->y) + (uint64_t)m0 * st->n * ye;
        p.n = st->n;
        p.k = st->k;
        p.m = a->m - m0 < 8 ? a->m - m0 : 8;
        p.scheme = st->w_scheme;
        p.x_dtype = st->in_dtype;
        p.y_dtype = st->out_dtype;
        p.epilogue = st->epilogue;
        p.w_row_stride = w_row;
        p.x_row_stride = st->k;
        int e = r9vx_launch_gemv(p, s);
        if (e) return hip_status("matmul", e);
    }
    return R9VX_OK;
}

/* ----------------------------------------------------------- weights/decode */

int r9vx_dequantize_launch(uint32_t scheme, const uint8_t *wire, uint32_t n_rows, uint32_t k,
                           float *out, r9vx_stream_t stream) {
    Problems pr;
    if (!matmul_scheme(scheme)) pr.add(R9VX_ERR_UNSUPPORTED, "scheme %u", scheme);
    const uint32_t bl = block_len(scheme);
    if (k == 0 || k % bl) pr.add(R9VX_ERR_INVALID, "k=%u must be a positive multiple of %u", k, bl);
    if (n_rows && (!wire || !out)) pr.add(R9VX_ERR_NULL, "wire and out must be non-NULL");
    /* Q8_0 / Q6_K / IQ3_S wire blocks are read as 16-bit words */
    const uintptr_t wmask = repacked_scheme(scheme) ? 1u : 15u;
    if ((wire && ((uintptr_t)wire & wmask)) || (out && !aligned16(out))) pr.add(R9VX_ERR_ALIGN, "wire / out alignment");
    int rc = pr.finish("dequantize");
    if (rc || n_rows == 0) return rc;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (repacked_scheme(scheme)) return hip_status("dequantize", r9vx_launch_dequant_split(scheme, wire, n_rows, k, out, s));
    return hip_status("dequantize", r9vx_launch_dequant(scheme, wire, n_rows, k, out, s));
}

int r9vx_repack_launch(uint32_t scheme, const uint8_t *wire, uint32_t n_rows, uint32_t k, uint8_t *body,
                       uint16_t *scales, r9vx_stream_t stream) {
    Problems pr;
    if (!repacked_scheme(scheme))
        pr.add(R9VX_ERR_UNSUPPORTED, "scheme %u: only Q8_0 (5), Q6_K (11) and IQ3_S (17) are repacked; Q4_K / "
               "IQ4_XS wire blocks are the device layout", scheme);
    const uint32_t bl = block_len(scheme);
    if (k == 0 || k % bl) pr.add(R9VX_ERR_INVALID, "k=%u must be a positive multiple of %u", k, bl);
    if (packed_scheme(scheme) && scales)
        pr.add(R9VX_ERR_INVALID, "scales must be NULL for IQ3_S: its 112-byte device blocks keep d inline");
    if (packed_scheme(scheme) && n_rows && (!wire || !body))
        pr.add(R9VX_ERR_NULL, "wire and body must be non-NULL");
    if (split_scheme(scheme) && n_rows && (!wire || !body || !scales))
        pr.add(R9VX_ERR_NULL, "wire, body and scales must be non-NULL");
    if ((wire && ((uintptr_t)wire & 1u)) || (body && !aligned16(body)) || (scales && ((uintptr_t)scales & 1u)))
        pr.add(R9VX_ERR_ALIGN, "wire and scales 2-byte, body 16-byte aligned");
    if (packed_scheme(scheme) && n_rows && wire && body && k % bl == 0) {
        const uint64_t nb = (uint64_t)n_rows * (k / bl);
        const uintptr_t w0 = (uintptr_t)wire, w1 = w0 + nb * block_bytes(scheme);
        const uintptr_t b0 = (uintptr_t)body, b1 = b0 + (uint64_t)n_rows * device_row_bytes(scheme, k);
        if (b0 < w1 && w0 < b1) pr.add(R9VX_ERR_INVALID, "wire and body must not overlap");
    }
    if (split_scheme(scheme) && n_rows && wire && body && scales && k % bl == 0) {
        const uint64_t nb = (uint64_t)n_rows * (k / bl);
        const uintptr_t w0 = (uintptr_t)wire, w1 = w0 + nb * block_bytes(scheme);
        const uintptr_t b0 = (uintptr_t)body, b1 = b0 + (uint64_t)n_rows * device_row_bytes(scheme, k);
        const uintptr_t s0 = (uintptr_t)scales, s1 = s0 + nb * 2;
        if ((b0 < w1 && w0 < b1) || (s0 < w1 && w0 < s1) || (s0 < b1 && b0 < s1))
            pr.add(R9VX_ERR_INVALID, "wire, body and scales must not overlap");
    }
    int rc = pr.finish("repack");
    if (rc || n_rows == 0) return rc;
    return hip_status("repack", r9vx_launch_repack(scheme, wire, n_rows, k, body, scales,
                                                   reinterpret_cast<hipStream_t>(stream)));
}

int r9vx_validate_weights_launch(uint32_t scheme, const uint8_t *wire, uint32_t n_rows, uint32_t k,
                                 uint32_t *bad_blocks, r9vx_stream_t stream) {
    Problems pr;
    if (!matmul_scheme(scheme)) pr.add(R9VX_ERR_UNSUPPORTED, "scheme %u", scheme);
    const uint32_t bl = block_len(scheme);
    if (k == 0 || k % bl) pr.add(R9VX_ERR_INVALID, "k=%u must be a positive multiple of %u", k, bl);
    if (n_rows && (!wire || !bad_blocks)) pr.add(R9VX_ERR_NULL, "wire and bad_blocks must be non-NULL");
    if (wire && ((uintptr_t)wire & (repacked_scheme(scheme) ? 1u : 3u))) pr.add(R9VX_ERR_ALIGN, "wire alignment");
    int rc = pr.finish("validate_weights");
    if (rc || n_rows == 0) return rc;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (repacked_scheme(scheme))
        return hip_status("validate_weights", r9vx_launch_validate_split(scheme, wire, n_rows, k, bad_blocks, s));
    return hip_status("validate_weights", r9vx_launch_validate(scheme, wire, n_rows, k, bad_blocks, s));
}

/* --------------------------------------------------------------- moe_route */

uint64_t r9vx_moe_route_static_bytes(const r9vx_moe_route_static *st, uint32_t t) {
    if (!st) return 0;
    return (uint64_t)t * st->e_total * 4 + (st->has_bias ? 4ull * st->e_total : 0) + (uint64_t)t * st->top_k * 8;
}

/* Per row (crates/r9v-t0/src/moe_route.rs:320-398): the bias add, the max,
 * the subtraction, exp and sum of the softmax and its divide (or sigmoid's
 * exp, add and divide), then the K scale multiplies, sum and divides. */
uint64_t r9vx_moe_route_static_flops(const r9vx_moe_route_static *st, uint32_t t) {
    if (!st) return 0;
    const uint64_t per_e = (st->has_bias ? 1u : 0u) + 4u;
    const uint64_t per_k = 1u + (st->renormalize ? 2u : 0u);
    return (uint64_t)t * (per_e * st->e_total + per_k * st->top_k);
}

static int route_launch(const char *op, const r9vx_moe_route_static *st, const r9vx_moe_route_args *a,
                        uint32_t *status, bool need_status, r9vx_stream_t stream) {
    Problems pr;
    if (!st || !a) {
        pr.add(R9VX_ERR_NULL, "static and args must be non-NULL");
        return pr.finish(op);
    }
    if (need_status && !status) pr.add(R9VX_ERR_NULL, "status word is NULL");
    if (status && ((uintptr_t)status & 3u)) pr.add(R9VX_ERR_ALIGN, "status word must be 4-byte aligned");
    float scale;
    memcpy(&scale, &st->scale_bits, 4);
    if (st->top_k == 0) pr.add(R9VX_ERR_INVALID, "top_k must be > 0");
    if (!(scale > 0.0f) || !(scale < __builtin_huge_valf()))
        pr.add(R9VX_ERR_INVALID, "scale must be finite and > 0, got %g", (double)scale);
    if (st->n_group != 0 || st->topk_group != 0)
        pr.add(R9VX_ERR_UNSUPPORTED, "grouped expert routing (n_group %u, topk_group %u) is not implemented",
               st->n_group, st->topk_group);
    if (a->t == 0 || st->e_total == 0) pr.add(R9VX_ERR_INVALID, "T=%u and E=%u must be > 0", a->t, st->e_total);
    if (st->top_k > st->e_total) pr.add(R9VX_ERR_INVALID, "top_k %u cannot exceed number of experts E=%u", st->top_k, st->e_total);
    if (st->e_total > 1024) pr.add(R9VX_ERR_UNSUPPORTED, "E=%u exceeds 1024", st->e_total);
    if (st->top_k > 32) pr.add(R9VX_ERR_UNSUPPORTED, "top_k=%u exceeds 32", st->top_k);
    if (st->scoring > R9VX_SCORING_SIGMOID) pr.add(R9VX_ERR_UNSUPPORTED, "scoring %u", st->scoring);
    if (a->t > st->t_bucket) pr.add(R9VX_ERR_INVALID, "t=%u exceeds t_bucket=%u", a->t, st->t_bucket);
    if (!a->logits || !a->expert_ids || !a->weights) pr.add(R9VX_ERR_NULL, "logits, expert_ids and weights are required");
    if (st->has_bias && !a->bias) pr.add(R9VX_ERR_NULL, "has_bias set but bias is NULL");
    if (!st->has_bias && a->bias) pr.add(R9VX_ERR_INVALID, "bias given but has_bias is 0");
    int rc = pr.finish(op);
    if (rc) return rc;
    r9vx_route_problem p{a->logits, a->bias,        a->expert_ids, a->weights,
                         status,   a->t,           st->e_total,   st->top_k,
                         st->scoring, st->renormalize ? 1u : 0u, scale};
    bool no_word = false;
    rc = r9vx_launch_route(p, reinterpret_cast<hipStream_t>(stream), &no_word);
    if (no_word) {
        pr.add(R9VX_ERR_UNSUPPORTED, "plain launches on more than %u streams of one device: use "
               "r9vx_moe_route_launch_ex with a status word of the caller's", r9vx_route_stream_words());
        return pr.finish(op);
    }
    return hip_status(op, rc);
}

int r9vx_moe_route_launch(const r9vx_moe_route_static *st, const r9vx_moe_route_args *a,
                          r9vx_stream_t stream) {
    return route_launch("moe_route", st, a, nullptr, false, stream);
}

int r9vx_moe_route_launch_ex(const r9vx_moe_route_static *st, const r9vx_moe_route_args *a, uint32_t *status,
                             r9vx_stream_t stream) {
    return route_launch("moe_route_ex", st, a, status, true, stream);
}

int r9vx_status_read(const uint32_t *word, uint32_t *status, r9vx_stream_t stream) {
    if (!word || !status) {
        g_last_error = "status_read: device word and status are required";
        return R9VX_ERR_NULL;
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    int rc = (int)hipMemcpyAsync(status, word, sizeof(uint32_t), hipMemcpyDeviceToHost, s);
    if (!rc) rc = (int)hipStreamSynchronize(s);
    return hip_status("status_read", rc);
}

static void check_route_static(const r9vx_moe_route_static *st, uint32_t t, Problems &pr, float &scale) {
    memcpy(&scale, &st->scale_bits, 4);
    if (st->top_k == 0) pr.add(R9VX_ERR_INVALID, "top_k must be > 0");
    if (!(scale > 0.0f) || !(scale < __builtin_huge_valf()))
        pr.add(R9VX_ERR_INVALID, "scale must be finite and > 0, got %g", (double)scale);
    if (st->n_group != 0 || st->topk_group != 0)
        pr.add(R9VX_ERR_UNSUPPORTED, "grouped expert routing (n_group %u, topk_group %u) is not implemented",
               st->n_group, st->topk_group);
    if (t == 0 || st->e_total == 0) pr.add(R9VX_ERR_INVALID, "T=%u and E=%u must be > 0", t, st->e_total);
    if (st->top_k > st->e_total) pr.add(R9VX_ERR_INVALID, "top_k %u cannot exceed number of experts E=%u", st->top_k, st->e_total);
    if (st->e_total > 1024) pr.add(R9VX_ERR_UNSUPPORTED, "E=%u exceeds 1024", st->e_total);
    if (st->top_k > 32) pr.add(R9VX_ERR_UNSUPPORTED, "top_k=%u exceeds 32", st->top_k);
    if (st->scoring > R9VX_SCORING_SIGMOID) pr.add(R9VX_ERR_UNSUPPORTED, "scoring %u", st->scoring);
    if (t > st->t_bucket) pr.add(R9VX_ERR_INVALID, "t=%u exceeds t_bucket=%u", t, st->t_bucket);
}

size_t r9vx_moe_route_hidden_workspace_bytes(const r9vx_moe_route_static *st) {
    if (!st) return 0;
    return (((size_t)st->t_bucket * st->e_total * 4 + 255) & ~(size_t)255) + 256;
}

int r9vx_moe_route_hidden_launch(const r9vx_moe_route_static *st, const r9vx_moe_route_hidden_args *a,
                                 r9vx_stream_t stream) {
    Problems pr;
    if (!st || !a) {
        pr.add(R9VX_ERR_NULL, "static and args must be non-NULL");
        return pr.finish("moe_route_hidden");
    }
    float scale;
    check_route_static(st, a->t, pr, scale);
    if (st->t_bucket > 8)
        pr.add(R9VX_ERR_UNSUPPORTED, "t_bucket=%u: the fused router is the decode form (t_bucket <= 8)", st->t_bucket);
    if (a->dm == 0 || a->dm % 128 || a->dm > 8192)
        pr.add(R9VX_ERR_INVALID, "dm=%u must be a positive multiple of 128, at most 8192", a->dm);
    if (!a->x || !a->w_router || !a->expert_ids || !a->weights)
        pr.add(R9VX_ERR_NULL, "x, w_router, expert_ids and weights are required");
    if (!a->workspace) pr.add(R9VX_ERR_WORKSPACE, "workspace of r9vx_moe_route_hidden_workspace_bytes required");
    if (st->has_bias && !a->bias) pr.add(R9VX_ERR_NULL, "has_bias set but bias is NULL");
    if (!st->has_bias && a->bias) pr.add(R9VX_ERR_INVALID, "bias given but has_bias is 0");
    if ((a->x && ((uintptr_t)a->x & 7u)) || (a->w_router && !aligned16(a->w_router)) ||
        (a->workspace && ((uintptr_t)a->workspace & 255u)))
        pr.add(R9VX_ERR_ALIGN, "x 8-byte, w_router 16-byte and workspace 256-byte aligned");
    int rc = pr.finish("moe_route_hidden");
    if (rc) return rc;
    const size_t logit_bytes = ((size_t)st->t_bucket * st->e_total * 4 + 255) & ~(size_t)255;
    r9vx_route_hidden_problem p{};
    p.x = reinterpret_cast<const uint16_t *>(a->x);
    p.w = a->w_router;
    p.bias = a->bias;
    p.logits = reinterpret_cast<float *>(a->workspace);
    p.counter = reinterpret_cast<uint32_t *>(a->workspace + logit_bytes);
    p.status = reinterpret_cast<uint32_t *>(a->workspace + logit_bytes + 4);
    p.ids = a->expert_ids;
    p.weights = a->weights;
    p.t = a->t;
    p.e = st->e_total;
    p.k = st->top_k;
    p.dm = a->dm;
    p.scoring = st->scoring;
    p.renormalize = st->renormalize ? 1u : 0u;
    p.scale = scale;
    return hip_status("moe_route_hidden", r9vx_launch_route_hidden(p, reinterpret_cast<hipStream_t>(stream)));
}

int r9vx_router_repack_launch(const float *w, uint32_t e, uint32_t dm, float *out, r9vx_stream_t stream) {
    Problems pr;
    if (e == 0 || dm == 0 || dm % 4) pr.add(R9VX_ERR_INVALID, "E=%u > 0 and dm=%u a positive multiple of 4", e, dm);
    if (!w || !out) pr.add(R9VX_ERR_NULL, "w and out are required");
    if ((w && !aligned16(w)) || (out && !aligned16(out))) pr.add(R9VX_ERR_ALIGN, "w and out must be 16-byte aligned");
    if (w && out) {
        const uintptr_t a0 = (uintptr_t)w, a1 = a0 + (uint64_t)e * dm * 4, b0 = (uintptr_t)out, b1 = b0 + (uint64_t)e * dm * 4;
        if (a0 < b1 && b0 < a1) pr.add(R9VX_ERR_INVALID, "w and out must not overlap");
    }
    int rc = pr.finish("router_repack");
    if (rc) return rc;
    return hip_status("router_repack", r9vx_launch_router_repack(w, e, dm, out, reinterpret_cast<hipStream_t>(stream)));
}

int r9vx_moe_route_hidden_status(const r9vx_moe_route_static *st, const uint8_t *workspace, uint32_t *status,
                                 r9vx_stream_t stream) {
    if (!st || !workspace || !status) {
        g_last_error = "moe_route_hidden_status: static, workspace and status are required";
        return R9VX_ERR_NULL;
    }
    const size_t logit_bytes = ((size_t)st->t_bucket * st->e_total * 4 + 255) & ~(size_t)255;
    const int rc = r9vx_status_read(reinterpret_cast<const uint32_t *>(workspace + logit_bytes + 4), status, stream);
    if (rc) g_last_error = "moe_route_hidden_status: " + g_last_error;
    return rc;
}

int r9vx_moe_route_status(uint32_t *status, r9vx_stream_t stream) {
    if (!status) {
        g_last_error = "moe_route_status: status is NULL";
        return R9VX_ERR_NULL;
    }
    return hip_status("moe_route_status", r9vx_read_route_status(status, reinterpret_cast<hipStream_t>(stream)));
}

/* ----------------------------------------------------------------- moe_ffn */

static void check_ffn_static(const r9vx_moe_ffn_static *st, Problems &pr) {
    if (st->e_local == 0 || st->e_local > kMoeMaxE) pr.add(R9VX_ERR_INVALID, "E=%u must be in 1..1024", st->e_local);
    if (st->k_topk == 0 || st->k_topk > kMoeMaxK) pr.add(R9VX_ERR_INVALID, "K=%u must be in 1..32", st->k_topk);
    if (st->dm == 0 || st->dm % 256) pr.add(R9VX_ERR_INVALID, "Dm=%u must be a positive multiple of 256", st->dm);
    if (st->dff == 0 || st->dff % 256) pr.add(R9VX_ERR_INVALID, "Dff=%u must be a positive multiple of 256", st->dff);
    if (!matmul_scheme(st->gate_up.scheme))
        pr.add(R9VX_ERR_UNSUPPORTED, "gate_up scheme %u: Q4_K (3), Q8_0 (5), Q6_K (11), IQ4_XS (15) or IQ3_S (17)",
               st->gate_up.scheme);
    else
        check_weight_keys("gate_up", st->gate_up.scheme, st->gate_up.dtype, st->gate_up.layout, pr);
    if (!matmul_scheme(st->down.scheme))
        pr.add(R9VX_ERR_UNSUPPORTED, "down scheme %u: Q4_K (3), Q8_0 (5), Q6_K (11), IQ4_XS (15) or IQ3_S (17)",
               st->down.scheme);
    else
        check_weight_keys("down", st->down.scheme, st->down.dtype, st->down.layout, pr);
    if (st->act_scheme != R9VX_ACT_SCHEME_NONE)
        pr.add(R9VX_ERR_UNSUPPORTED, "act_scheme %u: activations are not quantized on this path", st->act_scheme);
    if (st->placement_kind != R9VX_PLACEMENT_DEVICE)
        pr.add(R9VX_ERR_UNSUPPORTED, "placement_kind %u: device placement only", st->placement_kind);
    if (st->in_dtype != R9VX_DTYPE_BF16) pr.add(R9VX_ERR_UNSUPPORTED, "in_dtype %u: bf16 activations only", st->in_dtype);
    if (st->out_dtype != R9VX_DTYPE_F32) pr.add(R9VX_ERR_UNSUPPORTED, "out_dtype %u: f32 output only", st->out_dtype);
    if (st->act != R9VX_ACT_SILU) pr.add(R9VX_ERR_UNSUPPORTED, "act %u: SiLU only", st->act);
    if (st->shared_experts > 8) pr.add(R9VX_ERR_UNSUPPORTED, "shared_experts=%u exceeds 8", st->shared_experts);
    if (st->t_bucket == 0) pr.add(R9VX_ERR_INVALID, "t_bucket must be > 0");
    /* the grouped GEMMs address the staged activations, the h rows and one
     * expert's weights with 32-bit byte offsets */
    const uint64_t rows = (uint64_t)st->t_bucket * (st->k_topk + st->shared_experts);
    if (2ull * st->t_bucket * st->dm >= (1ull << 32) || 2ull * rows * st->dff >= (1ull << 32) ||
        2ull * st->dff * device_row_bytes(st->gate_up.scheme, st->dm) >= (1ull << 32) ||
        (uint64_t)st->dm * device_row_bytes(st->down.scheme, st->dff) >= (1ull << 32))
        pr.add(R9VX_ERR_UNSUPPORTED, "t_bucket=%u, Dm=%u, Dff=%u: staged operands or one expert exceed 4 GiB",
               st->t_bucket, st->dm, st->dff);
}

size_t r9vx_moe_ffn_workspace_bytes(const r9vx_moe_ffn_static *st) {
    if (!st) return 0;
    return (size_t)r9vx_moe_layout(st->t_bucket, st->e_local, st->k_topk, st->dm, st->dff, st->shared_experts).total;
}

uint64_t r9vx_moe_ffn_expert_bytes(const r9vx_moe_ffn_static *st) {
    if (!st) return 0;
    return 2ull * st->dff * (device_row_bytes(st->gate_up.scheme, st->dm) + 2ull * r9vx_row_scales(st->gate_up.scheme, st->dm)) +
           (uint64_t)st->dm * (device_row_bytes(st->down.scheme, st->dff) + 2ull * r9vx_row_scales(st->down.scheme, st->dff));
}

uint64_t r9vx_moe_ffn_static_bytes(const r9vx_moe_ffn_static *st, uint32_t t) {
    if (!st) return 0;
    const uint64_t pairs = (uint64_t)t * st->k_topk;
    const uint64_t experts = (pairs < st->e_local ? pairs : st->e_local) + st->shared_experts;
    return experts * r9vx_moe_ffn_expert_bytes(st) + (uint64_t)t * st->dm * 2 + pairs * 8 + (uint64_t)t * st->dm * 4;
}

uint64_t r9vx_moe_ffn_static_flops(const r9vx_moe_ffn_static *st, uint32_t t) {
    if (!st) return 0;
    uint64_t per_row = 2ull * (2ull * st->dff * st->dm) + 2ull * st->dm * st->dff;
    return per_row * ((uint64_t)t * st->k_topk + (uint64_t)t * st->shared_experts);
}

static void ffn_checks(const r9vx_moe_ffn_static *st, const uint32_t *ids, uint32_t t, Problems &pr) {
    check_ffn_static(st, pr);
    if (t == 0) pr.add(R9VX_ERR_INVALID, "t must be > 0");
    if (t > st->t_bucket) pr.add(R9VX_ERR_INVALID, "t=%u exceeds t_bucket=%u", t, st->t_bucket);
    if (!ids) pr.add(R9VX_ERR_NULL, "expert_ids is NULL");
}

/* The operand checks of a moe_ffn launch, workspace aside.  The split
 * layout (Q8_0 / Q6_K) carries its d values in the scale array of its
 * projection; the other layouts carry their scales inline. */
static void ffn_arg_checks(const r9vx_moe_ffn_static *st, const r9vx_moe_ffn_args *a, Problems &pr) {
    if (!a->x || !a->weights || !a->w_gate_up || !a->w_down || !a->y)
        pr.add(R9VX_ERR_NULL, "x, weights, w_gate_up, w_down and y are required");
    if (st) {
        const bool sg = split_scheme(st->gate_up.scheme), sd = split_scheme(st->down.scheme);
        if (sg != (a->w_gate_up_scales != nullptr))
            pr.add(sg ? R9VX_ERR_NULL : R9VX_ERR_UNSUPPORTED,
                   sg ? "w_gate_up_scales is required: scheme %u is read in the split layout (body + f16 d array)"
                      : "w_gate_up_scales must be NULL: scheme %u blocks carry their scales inline",
                   st->gate_up.scheme);
        if (sd != (a->w_down_scales != nullptr))
            pr.add(sd ? R9VX_ERR_NULL : R9VX_ERR_UNSUPPORTED,
                   sd ? "w_down_scales is required: scheme %u is read in the split layout (body + f16 d array)"
                      : "w_down_scales must be NULL: scheme %u blocks carry their scales inline",
                   st->down.scheme);
    }
    if ((a->w_gate_up_scales && ((uintptr_t)a->w_gate_up_scales & 3u)) ||
        (a->w_down_scales && ((uintptr_t)a->w_down_scales & 3u)))
        pr.add(R9VX_ERR_ALIGN, "scale arrays must be 4-byte aligned");
    if ((a->x && !aligned16(a->x)) || (a->y && !aligned16(a->y)) || (a->w_gate_up && !aligned16(a->w_gate_up)) ||
        (a->w_down && !aligned16(a->w_down)))
        pr.add(R9VX_ERR_ALIGN, "x, y and weights must be 16-byte aligned");
}

static int ffn_common(const char *op, const r9vx_moe_ffn_static *st, const uint32_t *ids, uint32_t t,
                      const uint8_t *ws, Problems &pr) {
    ffn_checks(st, ids, t, pr);
    if (!ws) pr.add(R9VX_ERR_WORKSPACE, "sort_workspace is NULL (size r9vx_moe_ffn_workspace_bytes)");
    if (ws && ((uintptr_t)ws & 255u)) pr.add(R9VX_ERR_ALIGN, "sort_workspace must be 256-byte aligned");
    return pr.finish(op);
}

static r9vx_moe_problem ffn_problem(const r9vx_moe_ffn_static *st, const r9vx_moe_ffn_args *a) {
    r9vx_moe_problem p{};
    p.x = reinterpret_cast<const uint16_t *>(a->x);
    p.ids = a->expert_ids;
    p.weights = a->weights;
    p.w_gu = reinterpret_cast<const uint8_t *>(a->w_gate_up);
    p.w_dn = reinterpret_cast<const uint8_t *>(a->w_down);
    p.s_gu = reinterpret_cast<const uint16_t *>(a->w_gate_up_scales);
    p.s_dn = reinterpret_cast<const uint16_t *>(a->w_down_scales);
    p.y = reinterpret_cast<float *>(a->y);
    p.ws = a->sort_workspace;
    p.t = a->t;
    p.e = st->e_local;
    p.k = st->k_topk;
    p.dm = st->dm;
    p.dff = st->dff;
    p.shared = st->shared_experts;
    p.t_bucket = st->t_bucket;
    p.scheme_gu = st->gate_up.scheme;
    p.scheme_dn = st->down.scheme;
    return p;
}

int r9vx_moe_ffn_launch(const r9vx_moe_ffn_static *st, const r9vx_moe_ffn_args *a,
                        r9vx_stream_t stream) {
    Problems pr;
    if (!st || !a) {
        pr.add(R9VX_ERR_NULL, "static and args must be non-NULL");
        return pr.finish("moe_ffn");
    }
    ffn_arg_checks(st, a, pr);
    int rc = ffn_common("moe_ffn", st, a->expert_ids, a->t, a->sort_workspace, pr);
    if (rc) return rc;
    r9vx_moe_problem p = ffn_problem(st, a);
    return hip_status("moe_ffn", r9vx_launch_moe(p, reinterpret_cast<hipStream_t>(stream)));
}

int r9vx_moe_ffn_status(const r9vx_moe_ffn_static *st, const uint8_t *ws, uint32_t *status,
                        r9vx_stream_t stream) {
    if (!st || !ws || !status) {
        g_last_error = "moe_ffn_status: static, workspace and status are required";
        return R9VX_ERR_NULL;
    }
    MoeLayout L = r9vx_moe_layout(st->t_bucket, st->e_local, st->k_topk, st->dm, st->dff, st->shared_experts);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    int rc = (int)hipMemcpyAsync(status, ws + L.status, sizeof(uint32_t), hipMemcpyDeviceToHost, s);
    if (!rc) rc = (int)hipStreamSynchronize(s);
    return hip_status("moe_ffn_status", rc);
}

/* ------------------------------------------------------ moe_ffn, no alloc */

}  // extern "C"

/* The sort workspace of r9vx_moe_ffn_launch_noalloc: one array on each GPU
 * the library runs on, held until the process ends.  In host code its name
 * is a host-side stand-in, never a device address: host code uses only the
 * address hipGetSymbolAddress returns for the current device (fetched once
 * per device and kept in g_scratch). */
static __device__ __align__(256) uint8_t scratch[R9VX_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
uint8_t *g_scratch[kScratchDevices];

/* Device address of the current device's scratch array, or nullptr with
 * *err set. */
uint8_t *device_scratch(hipError_t *err) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess && (dev < 0 || dev >= kScratchDevices)) e = hipErrorInvalidDevice;
    if (e != hipSuccess) {
        *err = e;
        return nullptr;
    }
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (!g_scratch[dev]) {
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            *err = e != hipSuccess ? e : hipErrorInvalidSymbol;
            return nullptr;
        }
        g_scratch[dev] = static_cast<uint8_t *>(ptr);
    }
    return g_scratch[dev];
}

__global__ void copy_status_kernel(const uint32_t *src, uint32_t *dst) { *dst = *src; }

}  // namespace

extern "C" {

int r9vx_moe_ffn_launch_noalloc(const r9vx_moe_ffn_static *st, const r9vx_moe_ffn_args *a, uint32_t *status,
                                r9vx_stream_t stream) {
    Problems pr;
    if (!st || !a) {
        pr.add(R9VX_ERR_NULL, "static and args must be non-NULL");
        return pr.finish("moe_ffn_noalloc");
    }
    ffn_arg_checks(st, a, pr);
    ffn_checks(st, a->expert_ids, a->t, pr);
    if (a->sort_workspace)
        pr.add(R9VX_ERR_INVALID, "sort_workspace must be NULL: this launch uses the library's own scratch");
    const size_t need = r9vx_moe_ffn_workspace_bytes(st);
    if (need > R9VX_NOALLOC_SCRATCH_BYTES)
        pr.add(R9VX_ERR_UNSUPPORTED,
               "the workspace of this static (%zu bytes) exceeds the no-alloc scratch (%u bytes): lower t_bucket, "
               "or call r9vx_moe_ffn_launch with a workspace",
               need, (unsigned)R9VX_NOALLOC_SCRATCH_BYTES);
    if (status && ((uintptr_t)status & 3u)) pr.add(R9VX_ERR_ALIGN, "status must be 4-byte aligned");
    int rc = pr.finish("moe_ffn_noalloc");
    if (rc) return rc;
    hipError_t err = hipSuccess;
    uint8_t *ws = device_scratch(&err);
    if (!ws) return hip_status("moe_ffn_noalloc", (int)err);
    r9vx_moe_ffn_args b = *a;
    b.sort_workspace = ws;
    const r9vx_moe_problem p = ffn_problem(st, &b);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    rc = r9vx_launch_moe(p, s);
    if (!rc && status) {
        const MoeLayout L = r9vx_moe_layout(p.t_bucket, p.e, p.k, p.dm, p.dff, p.shared);
        hipLaunchKernelGGL(copy_status_kernel, dim3(1), dim3(1), 0, s,
                           reinterpret_cast<const uint32_t *>(ws + L.status), status);
        rc = (int)hipGetLastError();
    }
    return hip_status("moe_ffn_noalloc", rc);
}

int r9vx_probe_moe_stage_launch(const r9vx_moe_ffn_static *st, const r9vx_moe_ffn_args *a, uint32_t stage,
                                r9vx_stream_t stream) {
    Problems pr;
    if (!st || !a) {
        pr.add(R9VX_ERR_NULL, "static and args must be non-NULL");
        return pr.finish("probe_moe_stage");
    }
    if (stage < 1 || stage > 3) pr.add(R9VX_ERR_INVALID, "stage %u: 1 (gate/up), 2 (down) or 3 (combine)", stage);
    if (st->t_bucket <= 8)
        pr.add(R9VX_ERR_UNSUPPORTED, "t_bucket=%u runs the decode path, which has no separate GEMM stages", st->t_bucket);
    if (!a->x || !a->weights || !a->w_gate_up || !a->w_down || !a->y)
        pr.add(R9VX_ERR_NULL, "x, weights, w_gate_up, w_down and y are required");
    int rc = ffn_common("probe_moe_stage", st, a->expert_ids, a->t, a->sort_workspace, pr);
    if (rc) return rc;
    r9vx_moe_problem p = ffn_problem(st, a);
    MoeLayout L = r9vx_moe_layout(p.t_bucket, p.e, p.k, p.dm, p.dff, p.shared);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    return hip_status("probe_moe_stage", stage == 3 ? r9vx_moe_combine_stage(p, L, s)
                                                    : r9vx_moe_grouped_part(p, L, stage, s));
}

int r9vx_moe_sort_launch(const r9vx_moe_ffn_static *st, const uint32_t *ids, uint32_t t, uint8_t *ws,
                         uint32_t *counts, uint32_t *offsets, uint32_t *sorted, r9vx_stream_t stream) {
    Problems pr;
    if (!st) {
        pr.add(R9VX_ERR_NULL, "static is NULL");
        return pr.finish("moe_sort");
    }
    if (!counts || !offsets || !sorted) pr.add(R9VX_ERR_NULL, "counts, offsets and sorted are required");
    int rc = ffn_common("moe_sort", st, ids, t, ws, pr);
    if (rc) return rc;
    r9vx_moe_ffn_args a{};
    a.expert_ids = ids;
    a.sort_workspace = ws;
    a.t = t;
    r9vx_moe_problem p = ffn_problem(st, &a);
    return hip_status("moe_sort", r9vx_launch_moe_sort(p, counts, offsets, sorted, reinterpret_cast<hipStream_t>(stream)));
}

}  // extern "C"

/* ------------------------------------------------------------------ dispatch */

int r9vx_launch_moe(const r9vx_moe_problem &p, hipStream_t s) {
    MoeLayout L = r9vx_moe_layout(p.t_bucket, p.e, p.k, p.dm, p.dff, p.shared);
    int rc = 0;
    /* Decode or grouped by the variant's t_bucket, never by t: every launch
     * of one static keeps h and o in the same precision and runs the same
     * GEMMs, so a token's output is the same bits whatever tokens share the
     * batch (crates/r9v-t0/src/harness.rs:903-948). */
    if (r9vx_moe_decode_form(p)) { /* pair-order rows: no sort; the combine checks the ids */
        rc = r9vx_moe_decode_stage(p, L, s);
    } else {
        bool x16_done = false;
        rc = r9vx_moe_sort_stage(p, L, s, &x16_done);
        if (!rc) rc = r9vx_moe_grouped_stage(p, L, s, x16_done);
    }
    if (rc) return rc;
    return r9vx_moe_combine_stage(p, L, s);
}

int r9vx_launch_moe_sort(const r9vx_moe_problem &p, uint32_t *counts, uint32_t *offsets, uint32_t *sorted,
                         hipStream_t s) {
    MoeLayout L = r9vx_moe_layout(p.t_bucket, p.e, p.k, p.dm, p.dff, p.shared);
    int rc = r9vx_moe_sort_stage(p, L, s);
    if (rc) return rc;
    uint64_t pp = (uint64_t)p.t * p.k;
    rc = (int)hipMemcpyAsync(counts, p.ws + L.counts, 4ull * p.e, hipMemcpyDeviceToDevice, s);
    if (!rc) rc = (int)hipMemcpyAsync(offsets, p.ws + L.offsets, 4ull * (p.e + 1), hipMemcpyDeviceToDevice, s);
    if (!rc) rc = (int)hipMemcpyAsync(sorted, p.ws + L.sorted, 4 * pp, hipMemcpyDeviceToDevice, s);
    return rc;
}
