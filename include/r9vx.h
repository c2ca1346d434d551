/*
 * r9vx.h -- C ABI of the MI355X (gfx950) quantized-weight matrix path.
 *
 * Drop-in for R9V's device tier of three ops: `matmul` with GGUF Q4_K /
 * IQ4_XS weights, `moe_route` and `moe_ffn`.  The argument structs are
 * byte-for-byte the kgen ABI structs of those ops
 * (crates/r9v-kgen/src/abi/per_op.rs:794-968): pointer fields first in
 * declaration order, then the u32 dynamic scalar, tail-padded to 8
 * (crates/r9v-kgen/src/abi/layout.rs:102-180).  A caller that already packs
 * `LaunchEntry.args_blob` (crates/r9v-registry/src/launch.rs:27) can pass that
 * blob's address as `args`.  The static structs carry the variant keys of
 * crates/r9v-registry/src/types.rs:727-860 that this path reads.
 *
 * Conventions (crates/r9v-kgen/src/abi/types.rs:14-19; spec-04 sec. 7):
 *  - the caller owns every buffer; workspaces are caller-allocated with the
 *    size the *_workspace_bytes query returns; nothing here allocates device
 *    memory during a launch;
 *  - device pointers should be 256-byte aligned (16-byte alignment is
 *    required and checked);
 *  - launches are stream-ordered on `stream` (NULL = the default stream);
 *  - status: 0 = launched; > 0 = a HIP error code from the runtime; < 0 = a
 *    host-side refusal (R9VX_ERR_*) before anything was enqueued.  The text of
 *    the last error on the calling thread is r9vx_last_error().
 *  - data-dependent refusals that only the device can see (non-finite router
 *    logits, expert ids >= E) follow T0's refuse-before-mutation rule: a
 *    check pass sets a status word and the compute kernels then write
 *    nothing.  Each launch owns its status word: moe_ffn's lives in its
 *    workspace, r9vx_moe_route_launch_ex takes one from the caller, and
 *    r9vx_moe_route_hidden_launch keeps one in its workspace.  The plain
 *    r9vx_moe_route_launch uses a word of the library's per stream (up to 64
 *    streams per device), so routings on different streams do not share one;
 *    launches on one stream are ordered and each overwrites it.
 */
#ifndef R9VX_H
#define R9VX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t without pulling in HIP headers. */
typedef struct ihipStream_t *r9vx_stream_t;

/* Element dtypes: discriminants of r9v-ir DType (crates/r9v-ir/src/dtype.rs:15-35). */
enum r9vx_dtype {
    R9VX_DTYPE_F32 = 0,
    R9VX_DTYPE_F16 = 1,
    R9VX_DTYPE_BF16 = 2,
    R9VX_DTYPE_I8 = 5, /* weight element type of Q8_0 / Q6_K blocks */
    R9VX_DTYPE_I4 = 6, /* weight element type of Q4_K / IQ4_XS / IQ3_S blocks */
    R9VX_DTYPE_U32 = 8
};

/* Weight layouts: LayoutId codes (crates/r9v-ir/src/layout.rs:16-38).  0-3
 * are the reference's own layouts (contiguous, row-major L0, tiled L1, tiled
 * 2:4-sparse L1S) and are refused by every entry point here: an L1 tensor in
 * `w` would otherwise be misread.  This path reads weights in the layouts
 * below, one per scheme, and a static must name the one its scheme needs. */
enum r9vx_layout {
    R9VX_LAYOUT_CONTIGUOUS = 0,
    R9VX_LAYOUT_L0 = 1,
    R9VX_LAYOUT_L1 = 2,
    R9VX_LAYOUT_L1S = 3,
    R9VX_LAYOUT_GGUF_WIRE = 0x100, /* Q4_K / IQ4_XS: the GGUF blocks as stored in the file */
    R9VX_LAYOUT_SPLIT = 0x101,     /* Q8_0 / Q6_K: body + f16 d array (r9vx_repack_launch) */
    R9VX_LAYOUT_IQ3S_112 = 0x102   /* IQ3_S: 112-byte blocks (r9vx_repack_launch) */
};

/* Activation quantization scheme (QuantScheme, crates/r9v-ir/src/quant.rs:48-62):
 * this path takes unquantized activations only. */
#define R9VX_ACT_SCHEME_NONE 0u

/* Placement (PlacementKind, crates/r9v-registry/src/types.rs:506-513): device only. */
#define R9VX_PLACEMENT_DEVICE 0u

/* Weight schemes: the reference's stable SchemeId codes
 * (SchemeId::code, crates/r9v-format/src/scheme.rs:115-138), the values a
 * MatmulStatic.w_scheme / MoeFfnProjStatic.scheme key carries
 * (QuantScheme::Scheme, crates/r9v-registry/src/types.rs:739,812).  They are
 * not GGUF ggml type ids (the reference keeps the two code spaces apart,
 * scheme.rs:78-87): every other code, GGUF ids such as 12 or 23 included, is
 * refused.  r9vx_scheme_from_ggml_type translates a GGUF tensor type. */
enum r9vx_scheme {
    R9VX_SCHEME_Q4_K = 3,    /* SchemeId::I4K: GGUF Q4_K, 144-B super-block per 256 weights */
    R9VX_SCHEME_Q8_0 = 5,    /* SchemeId::I8B32F: GGUF Q8_0, 34-B block per 32 weights; device layout split */
    R9VX_SCHEME_Q6_K = 11,   /* SchemeId::I6K: GGUF Q6_K, 210-B super-block per 256 weights; device layout split */
    R9VX_SCHEME_IQ4_XS = 15, /* SchemeId::I4Xs: GGUF IQ4_XS, 136-B super-block per 256 weights */
    R9VX_SCHEME_IQ3_S = 17   /* SchemeId::Iq3S: GGUF IQ3_S, 110-B super-block per 256 weights; device layout repacked */
};
/* The one translation from a GGUF tensor's ggml type id (crates/r9v-format/
 * src/ggml.rs:38: Q8_0 8, Q4_K 12, Q6_K 14, IQ3_S 21, IQ4_XS 23) to the
 * scheme code above; 0 for a type this path does not read.  The mapping is
 * the reference's own (GgmlType::scheme, crates/r9v-format/src/ggml.rs:253-276). */
uint32_t r9vx_scheme_from_ggml_type(uint32_t ggml_type);
/* Q4_K and IQ4_XS are read as GGUF wire blocks.  Q8_0 and Q6_K blocks (34 and
 * 210 bytes) are not 16-byte multiples, so the device reads them in a split
 * layout made at load time by r9vx_repack_launch (or r9vx_gguf_upload_split):
 *   Q8_0: body = int8 [N, K] (the 32 quants of each block, in order),
 *         w_scales = f16 [N, K/32] (each block's d);
 *   Q6_K: body = [N, K/256] blocks of 208 bytes (ql 128, qh 64, scales 16,
 *         the wire block without its trailing d), w_scales = f16 [N, K/256].
 * Bodies and scales together hold exactly the wire bytes.  A matmul on them
 * passes the body as `w` and the d array as `w_scales`.
 * IQ3_S (110-byte blocks) is repacked into one array of 112-byte blocks,
 * `scales` NULL: qs 64 | signs 32 | qh 8 | scales 4 | d 2 | two zero bytes
 * (the wire fields, in this order; crates/r9v-format/src/iq.rs:362-367 names
 * them), so the 4 sign bytes of each 32-weight group are one aligned word.
 * A matmul passes that array as `w` with `w_scales` NULL; bf16 activations. */

/* Matmul epilogues (crates/r9v-t0/src/matmul.rs:2421-2446), plus the gated
 * epilogue of the kernel generator's GEMM family ("gated (gate_up
 * interleave)", specs/spec-04-kernel-generator.md:100): with SWIGLU the
 * weights hold 2N rows, gate rows [0, N) then up rows [N, 2N) (the w_gate_up
 * convention of crates/r9v-t0/src/moe_ffn.rs:51-55), and
 * y[m, j] = silu(x[m].w[j]) * (x[m].w[N+j]) -- T0's matmul (f32 out) then
 * act_mul with SiLU (crates/r9v-t0/src/act_mul.rs:86-99,
 * crates/r9v-t0/src/activation.rs:135-138) in one launch.  bf16 activations,
 * m_bucket <= 8. */
enum r9vx_epilogue {
    R9VX_EPILOGUE_NONE = 0,
    R9VX_EPILOGUE_BIAS = 1,
    R9VX_EPILOGUE_RESIDUAL = 2,
    R9VX_EPILOGUE_SWIGLU = 3
};

/* Router scoring (crates/r9v-t0/src/moe_route.rs:329-351). */
enum r9vx_scoring { R9VX_SCORING_SOFTMAX = 0, R9VX_SCORING_SIGMOID = 1 };

/* Expert activation (crates/r9v-t0/src/activation.rs:133-138). */
enum r9vx_act { R9VX_ACT_SILU = 0 };

/* Host-side refusals. */
#define R9VX_OK 0
#define R9VX_ERR_INVALID -1     /* shape / static / argument mismatch */
#define R9VX_ERR_UNSUPPORTED -2 /* a variant key this path does not implement */
#define R9VX_ERR_NULL -3        /* a required pointer is NULL */
#define R9VX_ERR_ALIGN -4       /* a device pointer is not 16-byte aligned */
#define R9VX_ERR_WORKSPACE -5   /* workspace missing or too small */

/* Device status bits (read back by the *_status calls). */
#define R9VX_STATUS_NONFINITE 1u   /* non-finite logits / bias / scores */
#define R9VX_STATUS_DEGENERATE 2u  /* renormalise over a zero selected sum */
#define R9VX_STATUS_BAD_EXPERT 4u  /* an expert id >= E */

/* ------------------------------------------------------------------ matmul */

/* MatmulStatic (crates/r9v-registry/src/types.rs:727-770), every variant key
 * in its declaration order; bool keys are u32 0 / 1. */
typedef struct r9vx_matmul_static {
    uint32_t m_bucket;       /* M bucket; the launch's dynamic m <= m_bucket */
    uint32_t n;              /* output columns N */
    uint32_t k;              /* reduction length K, a multiple of 256 */
    uint32_t w_dtype;        /* I4 for Q4_K / IQ4_XS / IQ3_S, I8 for Q8_0 / Q6_K */
    uint32_t w_scheme;       /* enum r9vx_scheme */
    uint32_t w_layout;       /* enum r9vx_layout: GGUF_WIRE, SPLIT or IQ3S_112 as the scheme requires */
    uint32_t in_dtype;       /* F32 (GEMV, m_bucket <= 8) or BF16 */
    uint32_t act_scheme;     /* R9VX_ACT_SCHEME_NONE */
    uint32_t out_dtype;      /* F32 or BF16 (RNE) */
    uint32_t epilogue;       /* enum r9vx_epilogue */
    uint32_t residual_dtype; /* F32 when epilogue == RESIDUAL */
    uint32_t transpose_w;    /* 0: w is [N, K] */
    uint32_t interleave;     /* 0 */
    uint32_t sparse;         /* 0 */
} r9vx_matmul_static;

/* matmul ABI struct (crates/r9v-kgen/src/abi/per_op.rs:794-868). */
typedef struct r9vx_matmul_args {
    const uint8_t *w;         /* GGUF blocks (row n at n * (K/256) * block_bytes), or a split body */
    const void *w_scales;     /* Q8_0 / Q6_K: f16 d per block; NULL for Q4_K / IQ4_XS (inline) */
    const uint8_t *w_indices; /* must be NULL: no sparsity on this path */
    const void *x;            /* [m, K] in_dtype */
    const float *x_scale;     /* must be NULL: activations are not quantized */
    const float *bias;        /* [N] f32 when epilogue == BIAS */
    const void *residual;     /* [m, N] f32 when epilogue == RESIDUAL */
    void *y;                  /* [m, N] out_dtype */
    float *workspace;         /* split-K partials; may be NULL when 0 bytes are required */
    uint32_t m;               /* dynamic row count */
    uint32_t _tail_pad;
} r9vx_matmul_args;

/* Replaces: Registry::resolve + dispatch_launch for Op::Matmul
 * (crates/r9v-registry/src/resolution.rs:232, launch.rs:97) whose T0 meaning
 * is matmul_with_scales Branch D (crates/r9v-t0/src/matmul.rs:1940-2414). */
int r9vx_matmul_launch(const r9vx_matmul_static *st, const r9vx_matmul_args *args,
                       r9vx_stream_t stream);
/* Workspace slot SplitKPartials size (crates/r9v-kgen/src/abi/workspace.rs:13-40). */
size_t r9vx_matmul_workspace_bytes(const r9vx_matmul_static *st);
/* LaunchEntry.static_bytes / static_flops (crates/r9v-registry/src/launch.rs:22-25):
 * algorithmic HBM bytes (weights + x + y) and 2*m*N*K. */
uint64_t r9vx_matmul_static_bytes(const r9vx_matmul_static *st, uint32_t m);
uint64_t r9vx_matmul_static_flops(const r9vx_matmul_static *st, uint32_t m);

/* --------------------------------------------------------------- moe_route */

/* MoeRouteStatic (crates/r9v-registry/src/types.rs:774-800), every key in
 * its declaration order.  `group: Option<MoeGroup>` (MoeGroup {n_group,
 * topk_group}, crates/r9v-ir/src/op.rs:152-157) is the pair n_group /
 * topk_group, n_group = 0 meaning None; grouped routing (n_group > 0) is not
 * implemented and refused, as T0 refuses it (moe_route.rs:198-203). */
typedef struct r9vx_moe_route_static {
    uint32_t t_bucket;
    uint32_t e_total;     /* E <= 1024 */
    uint32_t top_k;       /* K <= 32, K <= E */
    uint32_t scoring;     /* enum r9vx_scoring */
    uint32_t renormalize; /* 0 / 1 */
    uint32_t n_group;     /* group: 0 (None) only */
    uint32_t topk_group;  /* group: 0 with n_group = 0 */
    uint32_t scale_bits;  /* IEEE-754 bits of the f32 route scale */
    uint32_t has_bias;    /* 0 / 1 */
} r9vx_moe_route_static;

/* moe_route ABI struct (crates/r9v-kgen/src/abi/per_op.rs:870-901). */
typedef struct r9vx_moe_route_args {
    const float *logits;  /* [t, E] f32 */
    const float *bias;    /* [E] f32 or NULL */
    uint32_t *expert_ids; /* [t, K] u32 */
    float *weights;       /* [t, K] f32 */
    uint32_t t;
    uint32_t _tail_pad;
} r9vx_moe_route_args;

/* Replaces: dispatch of Op::MoeRoute; T0 meaning moe_route
 * (crates/r9v-t0/src/moe_route.rs:89-419).  Ids are bit-exact with T0. */
int r9vx_moe_route_launch(const r9vx_moe_route_static *st, const r9vx_moe_route_args *args,
                          r9vx_stream_t stream);
/* The same launch with a caller-owned status word: `status` is a device u32
 * (4-byte aligned) that this launch overwrites with its own status bits
 * (0 when it routed every row).  Launches with distinct words may run
 * concurrently on different streams; read the word back after the stream
 * reaches the launch (r9vx_status_read).  No counterpart in the reference,
 * whose T0 refusal is a returned error: this is that error's device form. */
int r9vx_moe_route_launch_ex(const r9vx_moe_route_static *st, const r9vx_moe_route_args *args,
                             uint32_t *status, r9vx_stream_t stream);
/* Synchronises `stream`, returns the status bits of the last plain
 * r9vx_moe_route_launch on `stream` in *status (0 when none ran there) and
 * clears them.  Each stream has its own word (the library's, assigned on the
 * stream's first plain launch; a 65th stream of one device is refused with
 * R9VX_ERR_UNSUPPORTED and must use the _ex form). */
int r9vx_moe_route_status(uint32_t *status, r9vx_stream_t stream);
/* Copies a device status word (of r9vx_moe_route_launch_ex) to *status after
 * synchronising `stream`. */
int r9vx_status_read(const uint32_t *device_word, uint32_t *status, r9vx_stream_t stream);
/* LaunchEntry.static_bytes / static_flops (crates/r9v-registry/src/launch.rs:22-25):
 * logits, bias, ids and weights; and the arithmetic of scoring, the ordered
 * softmax sum and the renormalisation (about 4*E + 2*K per row). */
uint64_t r9vx_moe_route_static_bytes(const r9vx_moe_route_static *st, uint32_t t);
uint64_t r9vx_moe_route_static_flops(const r9vx_moe_route_static *st, uint32_t t);

/* Routing from hidden states (the router-logits matmul feeding moe_route,
 * fused; decode form, t_bucket <= 8).  No single op of the reference: it replaces the
 * graph's router matmul (f32 weight [E, dm], the GGUF ffn_gate_inp tensor)
 * followed by Op::MoeRoute.  Every logit is accumulated in T0's matmul order
 * (crates/r9v-t0/src/matmul.rs:1940-2414: k ascending, one f32 accumulator,
 * product rounded then added), so ids and weights equal T0's matmul +
 * moe_route (crates/r9v-t0/src/moe_route.rs:89-419) bit for bit; refusals and
 * r9vx_moe_route_status behave as for r9vx_moe_route_launch. */
typedef struct r9vx_moe_route_hidden_args {
    const void *x;          /* bf16 [t, dm] hidden states, 8-byte aligned */
    const float *w_router;  /* f32 router weight in the k4 layout of r9vx_router_repack_launch, 16-byte aligned */
    const float *bias;      /* [E] f32 or NULL (has_bias) */
    uint32_t *expert_ids;   /* [t, K] */
    float *weights;         /* [t, K] */
    uint8_t *workspace;     /* r9vx_moe_route_hidden_workspace_bytes, 256-byte aligned,
                               zero-filled once after allocation (the library leaves it so) */
    uint32_t t;
    uint32_t dm;            /* a multiple of 128, at most 8192 */
} r9vx_moe_route_hidden_args;

/* Load-time layout of the router weight for r9vx_moe_route_hidden_launch:
 * f32 [E, dm] (the GGUF ffn_gate_inp tensor, rows of dm) -> [dm/4][E][4],
 * so that a wave's load covers 4 consecutive K values of 64 consecutive
 * experts.  out may not overlap w. */
int r9vx_router_repack_launch(const float *w, uint32_t e, uint32_t dm, float *out, r9vx_stream_t stream);

int r9vx_moe_route_hidden_launch(const r9vx_moe_route_static *st, const r9vx_moe_route_hidden_args *args,
                                 r9vx_stream_t stream);
/* Workspace of r9vx_moe_route_hidden_launch: the [t_bucket, E] f32 logits, a
 * completion counter and the launch's status word. */
size_t r9vx_moe_route_hidden_workspace_bytes(const r9vx_moe_route_static *st);
/* Synchronises `stream` and returns the status bits the last
 * r9vx_moe_route_hidden_launch with this workspace left in it. */
int r9vx_moe_route_hidden_status(const r9vx_moe_route_static *st, const uint8_t *workspace, uint32_t *status,
                                 r9vx_stream_t stream);

/* ----------------------------------------------------------------- moe_ffn */

/* MoeFfnProjStatic (crates/r9v-registry/src/types.rs:801-818): one
 * projection's weight element type, scheme and layout. */
typedef struct r9vx_moe_ffn_proj {
    uint32_t dtype;  /* I4 for Q4_K / IQ4_XS / IQ3_S, I8 for Q8_0 / Q6_K */
    uint32_t scheme; /* enum r9vx_scheme (SchemeId code): Q4_K, IQ4_XS, IQ3_S, Q8_0 or Q6_K */
    uint32_t layout; /* enum r9vx_layout: GGUF_WIRE (Q4_K, IQ4_XS), IQ3S_112 (IQ3_S), SPLIT (Q8_0, Q6_K) */
} r9vx_moe_ffn_proj;

/* MoeFfnStatic (crates/r9v-registry/src/types.rs:828-860), every key in its
 * declaration order. */
typedef struct r9vx_moe_ffn_static {
    uint32_t t_bucket;
    uint32_t e_local;          /* routed experts E */
    uint32_t k_topk;           /* K */
    uint32_t dm;               /* hidden size, multiple of 256 */
    uint32_t dff;              /* expert intermediate size, multiple of 256 */
    r9vx_moe_ffn_proj gate_up; /* w_gate_up [E+S, 2Dff, Dm]: any of the five schemes */
    r9vx_moe_ffn_proj down;    /* w_down [E+S, Dm, Dff]: any of the five schemes */
    uint32_t in_dtype;         /* BF16 */
    uint32_t act_scheme;       /* R9VX_ACT_SCHEME_NONE */
    uint32_t act;              /* enum r9vx_act */
    uint32_t out_dtype;        /* F32 */
    uint32_t shared_experts;   /* S shared experts stored after the E routed ones */
    uint32_t placement_kind;   /* R9VX_PLACEMENT_DEVICE */
} r9vx_moe_ffn_static;

/* moe_ffn ABI struct (crates/r9v-kgen/src/abi/per_op.rs:903-968). */
typedef struct r9vx_moe_ffn_args {
    const void *x;                /* [t, Dm] in_dtype */
    const uint32_t *expert_ids;   /* [t, K] */
    const float *weights;         /* [t, K] */
    const void *w_gate_up;        /* expert e's gate rows [0,Dff) then up rows [Dff,2Dff), each row in
                                     the device layout of gate_up.scheme: GGUF blocks (Q4_K, IQ4_XS),
                                     112-byte blocks (IQ3_S) or the split body (Q8_0, Q6_K) */
    const void *w_gate_up_scales; /* Q8_0 / Q6_K: the split layout's f16 d per block, [E+S, 2Dff,
                                     Dm/blocklen] (blocklen 32 / 256), 4-byte aligned; NULL otherwise */
    const void *w_down;           /* [E+S, Dm, Dff] rows in the device layout of down.scheme */
    const void *w_down_scales;    /* Q8_0 / Q6_K: f16 d [E+S, Dm, Dff/blocklen]; NULL otherwise */
    void *y;                      /* [t, Dm] out_dtype */
    uint8_t *sort_workspace;      /* MoeSortBuffers, r9vx_moe_ffn_workspace_bytes */
    uint32_t t;
    uint32_t _tail_pad;
} r9vx_moe_ffn_args;

/* Replaces: dispatch of Op::MoeFfn; T0 meaning moe_ffn
 * (crates/r9v-t0/src/moe_ffn.rs:75-660) plus, when shared_experts > 0, the
 * shared-expert matmul/act_mul/residual_add graph of
 * crates/r9v-models/src/generic.rs:1458-1495, fused. */
int r9vx_moe_ffn_launch(const r9vx_moe_ffn_static *st, const r9vx_moe_ffn_args *args,
                        r9vx_stream_t stream);
size_t r9vx_moe_ffn_workspace_bytes(const r9vx_moe_ffn_static *st);
/* Synchronises `stream` and returns the status bits the last launch with
 * this workspace left in it (R9VX_STATUS_BAD_EXPERT). */
int r9vx_moe_ffn_status(const r9vx_moe_ffn_static *st, const uint8_t *sort_workspace,
                        uint32_t *status, r9vx_stream_t stream);
/* No counterpart in the reference: moe_ffn for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same checks, kernels and results as r9vx_moe_ffn_launch, but
 * the sort workspace is the library's own device array of
 * R9VX_NOALLOC_SCRATCH_BYTES on each GPU it runs on (held until the process
 * ends): args->sort_workspace must be NULL, and a static whose
 * r9vx_moe_ffn_workspace_bytes exceeds that size is refused
 * (R9VX_ERR_UNSUPPORTED).  Allocates nothing.  When `status` (a device u32)
 * is not NULL the launch's status bits are copied there on `stream`
 * (r9vx_status_read reads them).  Every call on one GPU shares that GPU's
 * array, which keeps the last call's contents: calls on one stream are
 * ordered, calls that overlap on one GPU (other streams, other threads)
 * race. */
#define R9VX_NOALLOC_SCRATCH_BYTES (16u << 20)
int r9vx_moe_ffn_launch_noalloc(const r9vx_moe_ffn_static *st, const r9vx_moe_ffn_args *args, uint32_t *status,
                                r9vx_stream_t stream);
/* LaunchEntry.static_flops (crates/r9v-registry/src/launch.rs:22-25):
 * (t*K + t*S) rows of 2*(2Dff*Dm) + 2*Dm*Dff. */
uint64_t r9vx_moe_ffn_static_flops(const r9vx_moe_ffn_static *st, uint32_t t);
/* LaunchEntry.static_bytes: an upper bound on the HBM bytes of one launch --
 * (min(E, t*K) + S) experts' gate/up and down weights, x (bf16), ids and
 * weights, y (f32).  The bytes actually read depend on how many distinct
 * experts the ids name; r9vx_moe_ffn_expert_bytes is one expert's share. */
uint64_t r9vx_moe_ffn_static_bytes(const r9vx_moe_ffn_static *st, uint32_t t);
uint64_t r9vx_moe_ffn_expert_bytes(const r9vx_moe_ffn_static *st);

/* Permute pre-pass of moe_ffn on its own: counts [E], offsets [E+1] and
 * sorted [t*K] (= token*K + slot in stable (expert, token, slot) order), the
 * counting-sort restatement of crates/r9v-t0/src/moe_ffn.rs:477-493 and the
 * MoeSortBuffers contents (crates/r9v-kgen/src/abi/workspace.rs:13-40).  Uses
 * the moe_ffn workspace for its scratch. */
int r9vx_moe_sort_launch(const r9vx_moe_ffn_static *st, const uint32_t *expert_ids, uint32_t t,
                         uint8_t *sort_workspace, uint32_t *counts, uint32_t *offsets,
                         uint32_t *sorted, r9vx_stream_t stream);

/* ------------------------------------------------------------ weights / decode */

/* `scheme` below is an enum r9vx_scheme code, as in the statics. */

/* Bit-exact decode of GGUF wire blocks to f32 [n_rows, k]: the
 * ggml_dequantize of crates/r9v-format/src/ggml.rs:1025-1150 (Q4_K; Q8_0
 * :1094-1100 and Q6_K :1154-1172 with block_values :627-640, :817-850) and
 * crates/r9v-format/src/iq.rs:578-598 (IQ4_XS).  Q8_0 / Q6_K are read in wire
 * form here. */
int r9vx_dequantize_launch(uint32_t scheme, const uint8_t *wire, uint32_t n_rows, uint32_t k,
                           float *out, r9vx_stream_t stream);
/* Load-time scale validation (check_wire_f16, crates/r9v-format/src/ggml.rs:421):
 * counts wire blocks with a non-finite d (or dmin) into *bad_blocks (device
 * u32, caller-zeroed). */
int r9vx_validate_weights_launch(uint32_t scheme, const uint8_t *wire, uint32_t n_rows,
                                 uint32_t k, uint32_t *bad_blocks, r9vx_stream_t stream);

/* Load-time repack of Q8_0 / Q6_K / IQ3_S wire blocks [n_rows, k] (device
 * memory) into the device layouts above: body and scales may not overlap the
 * wire; IQ3_S takes scales = NULL.  The counterpart of the reference's
 * load-time repack to its L1 layout (crates/r9v-format/src/repack.rs:282).
 * Q4_K and IQ4_XS need none and are refused. */
int r9vx_repack_launch(uint32_t scheme, const uint8_t *wire, uint32_t n_rows, uint32_t k,
                       uint8_t *body, uint16_t *scales, r9vx_stream_t stream);

/* ------------------------------------------------------------------ misc */

/* Text of the last refusal / HIP error on the calling thread. */
const char *r9vx_last_error(void);
/* ABI version of this header (bumped on any struct change). */
uint32_t r9vx_abi_version(void);

#define R9VX_ABI_VERSION 3u

#ifdef __cplusplus
}
#endif
#endif
