/*
 * r9vx_moe.h -- the moe_ffn workspace layout (the kgen MoeSortBuffers slot,
 * crates/r9v-kgen/src/abi/workspace.rs:13-40) and the stage launchers.
 *
 * Workspace regions (each 256-byte aligned), sized for t_bucket tokens:
 *   status  u32[16]  [0] status bits, [4] 256-row tiles
 *   counts  u32[E]   pairs per expert
 *   offsets u32[E+1] exclusive scan of counts
 *   sorted  u32[P]   pair index (token*K + slot) at each sorted position
 *   inv     u32[P]   sorted position of each pair
 *   rank    u32[P]   rank of a pair among its expert's pairs in its chunk
 *   ccount  u32[E*C] per-expert counts of each 256-pair chunk
 *   cbase   u32[E*C] exclusive scan of ccount over chunks
 *   cbad    u32[C]   1 where the chunk holds an id >= E
 *   tiles3  u32x4[...] grouped-GEMM tile schedule (expert, first position,
 *                      rows, 0), 256-row tiles (the r9vx_mma3.h kernels)
 *   h       f32[(P + S*T) * Dff]  SwiGLU rows of the decode form (t_bucket <= 8)
 *                                 in pair order, shared rows after; empty for
 *                                 the grouped form (h16 only)
 *   o       f32[(P + S*T) * Dm]   expert output rows (decode path: in pair
 *                                 order, no sort); the grouped path stores them in the
 *                                 same region as fp16 [(P + S*T) * Dm] scaled
 *                                 per (row, 64-column block), followed by the
 *                                 f32 scales [(P + S*T) * Dm/64]
 *   hexp    i32[P + S*T]          e of an h16 row's one scale 2^-e (grouped
 *                                 down GEMM past kM3MaxBlk blocks)
 *   h16     fp16[(P + S*T) * Dff] h rows scaled by a power of two, in the down
 *                                 weights' K group order (grouped GEMM)
 *   hbe     i8[(P + S*T) * NB4]   e of each (row, 128-column block)'s h16
 *                                 scale 2^-e; NB4 = Dff/128 rounded up to a
 *                                 multiple of 4 (r9vx_moe_hbe_stride)
 *   x16     fp16[T * Dm], xscale f32[T]  scaled activations in the gate/up
 *                                 weights' K group order (grouped GEMM)
 */
#ifndef R9VX_MOE_H
#define R9VX_MOE_H

#include <stddef.h>
#include <stdint.h>

#include "r9vx_internal.h"

constexpr uint32_t kMoeMaxE = 1024;
constexpr uint32_t kMoeMaxK = 32;
constexpr uint32_t kMoeTileM3 = 256; /* rows per tile of the r9vx_mma3.h grouped GEMMs */

struct MoeLayout {
    uint64_t status, counts, offsets, sorted, inv, rank, ccount, cbase, cbad, tiles3, h, o, hexp, h16, hbe, x16, xscale,
        total;
    uint32_t max_tiles3;
};

/* bytes per row of the hbe exponents: one per 128-column block of h,
 * rounded up to whole words */
__host__ __device__ inline uint32_t r9vx_moe_hbe_stride(uint32_t dff) { return (dff / 128 + 3) & ~3u; }

inline MoeLayout r9vx_moe_layout(uint32_t t_bucket, uint32_t e, uint32_t k, uint32_t dm, uint32_t dff,
                                 uint32_t shared) {
    MoeLayout L{};
    uint64_t p = (uint64_t)t_bucket * k;
    uint64_t nchunk = (p + 255) / 256;
    uint64_t rows = p + (uint64_t)shared * t_bucket;
    uint64_t off = 0;
    auto take = [&](uint64_t bytes) {
        uint64_t at = off;
        off += (bytes + 255) & ~255ull;
        return at;
    };
    L.max_tiles3 = (uint32_t)((p + (uint64_t)shared * t_bucket) / kMoeTileM3 + e + shared + 1);
    L.status = take(64);
    L.counts = take(4ull * e);
    L.offsets = take(4ull * (e + 1));
    L.sorted = take(4 * p);
    L.inv = take(4 * p);
    L.rank = take(4 * p);
    L.ccount = take(4ull * e * nchunk);
    L.cbase = take(4ull * e * nchunk);
    L.cbad = take(4 * nchunk);
    L.tiles3 = take(16ull * L.max_tiles3 + 16);
    L.h = take(t_bucket <= 8 ? 4ull * rows * dff : 0); /* the decode form (r9vx_moe_decode_form) */
    L.o = take(4ull * rows * dm);
    L.hexp = take(4ull * rows);
    L.h16 = take(2ull * rows * dff);
    L.hbe = take(rows * r9vx_moe_hbe_stride(dff));
    L.x16 = take(2ull * t_bucket * dm);
    L.xscale = take(4ull * t_bucket);
    L.total = off;
    return L;
}

struct MoeCombineArgs {
    const float *weights;
    const uint32_t *ids;
    float *y;
    uint8_t *ws;
    MoeLayout L;
    uint32_t t, k, dm, shared, p, e;
};

/* The decode form (pair-order rows, f32 h and o, GEMV kernels) serves the
 * variants with t_bucket <= 8, the grouped MFMA form every larger bucket,
 * whatever the launch's t. */
inline bool r9vx_moe_decode_form(const r9vx_moe_problem &p) { return p.t_bucket <= 8; }

/* x16_done != NULL: the sort kernels also convert the activation rows for
 * the grouped GEMMs (only on the multi-kernel path; *x16_done says whether). */
int r9vx_moe_sort_stage(const r9vx_moe_problem &p, const MoeLayout &L, hipStream_t s, bool *x16_done = nullptr);
int r9vx_moe_decode_stage(const r9vx_moe_problem &p, const MoeLayout &L, hipStream_t s);
int r9vx_moe_grouped_stage(const r9vx_moe_problem &p, const MoeLayout &L, hipStream_t s, bool x16_done = false);
int r9vx_moe_grouped_part(const r9vx_moe_problem &p, const MoeLayout &L, uint32_t part, hipStream_t s,
                          bool x16_done = false);
int r9vx_moe_combine_stage(const r9vx_moe_problem &p, const MoeLayout &L, hipStream_t s);

/* Byte offset (from L.o) of the grouped path's per-(row, 64-column) scales. */
/* silu(g) * u with the hardware exp and reciprocal (about 2 ulp each; T0's
 * f32 expf and divide, crates/r9v-t0/src/activation.rs:135-138, are matched
 * well inside the matmul tolerance). */
__device__ __forceinline__ float swiglu_fast(float g, float u) {
    return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f)) * u;
}

__host__ __device__ inline uint64_t r9vx_moe_oscale_offset(uint64_t rows, uint32_t dm) { return (2ull * rows * dm + 255) & ~255ull; }

#endif
