/*
 * moe.hip -- moe_ffn on the GPU: the (expert, token) permute, the per-expert
 * SwiGLU FFN and the weighted unpermute-sum.
 *
 * T0 meaning: crates/r9v-t0/src/moe_ffn.rs:466-660.
 *  - Permute (:477-493): a stable sort of (expert, token, slot) triples is a
 *    counting sort over the pairs in ascending (token, slot) order.  Ranks are
 *    computed per 256-pair chunk with ballot-based peer matching plus
 *    per-wave counts in LDS, chunk counts are scanned per expert, experts are
 *    scanned per chunk-total: every index depends only on the input, never on
 *    atomics ordering, so `sorted`, `counts`, `offsets` are bit-exact.
 *  - FFN per expert (:527-639): gate rows [0,Dff), up rows [Dff,2Dff) of the
 *    expert's [2Dff, Dm] block; h = silu(g)*u (activation.rs:135-138,
 *    act_mul.rs:86-99); o = h . Wd^T.  Variants with t_bucket <= 8 run
 *    dequant-fused GEMVs with the rows in pair order (token * K + slot), so
 *    they need no sort pass (h kept in f32 between them); larger buckets sort
 *    and run the grouped MFMA GEMMs of moe_gemm.hip, whatever the launch's t.
 *  - Combine (:641-653): y[t] = sum over the token's pairs in ascending
 *    (expert, slot) order of w * o, f32, then the shared experts' outputs are
 *    added (the residual_add of crates/r9v-models/src/generic.rs:1458-1495).
 *  - Refusal before mutation (:440-465): ids >= E set R9VX_STATUS_BAD_EXPERT
 *    in the workspace status word and y is not written (the grouped path's
 *    sort flags them and every later kernel returns; on the decode path the
 *    GEMVs read nothing for such a pair and the combine checks every id).
 */
#include <type_traits>

#include "r9vx_gemv_core.h"
#include "r9vx_mfma.h"
#include "r9vx_moe.h"
#include "r9vx_x16.h"

using namespace r9vx;

namespace {

/* ---------------------------------------------------------------- scans */

/* Inclusive prefix sum across a wave. */
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v, uint32_t lane) {
    for (int off = 1; off < 64; off <<= 1) {
        uint32_t o = __shfl_up(v, off, 64);
        if (lane >= (uint32_t)off) v += o;
    }
    return v;
}

/* Exclusive scan across the block (blockDim.x <= 1024); `sh` holds 16 u32. */
__device__ uint32_t block_excl_scan(uint32_t v, uint32_t *sh, uint32_t &total) {
    uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    uint32_t inc = wave_incl_scan(v, lane);
    __syncthreads();
    if (lane == 63) sh[w] = inc;
    __syncthreads();
    uint32_t base = 0, tot = 0;
    for (uint32_t i = 0; i < nw; ++i) {
        uint32_t s = sh[i];
        if (i < w) base += s;
        tot += s;
    }
    total = tot;
    return base + inc - v;
}

/* Lanes of this wave holding the same key (key < 2^bits), among `valid`. */
__device__ __forceinline__ uint64_t match_peers(uint32_t key, bool valid, int bits) {
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < bits; ++b) {
        uint32_t bit = (key >> b) & 1u;
        uint64_t ones = __ballot(valid && bit);
        peers &= bit ? ones : ~ones;
    }
    return peers;
}

__device__ __forceinline__ uint32_t rank_below(uint64_t peers, uint32_t lane) {
    uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    return (uint32_t)__popcll(peers & lt);
}

__device__ __forceinline__ int id_bits(uint32_t e) {
    int b = 1;
    while ((1u << b) < e) ++b;
    return b;
}

/* ---------------------------------------------------------------- sort: small */

struct SortArgs {
    const uint32_t *ids;
    uint8_t *ws;
    MoeLayout L;
    uint32_t p, e, k, t, shared;
    uint32_t nchunk;
    /* the grouped path's activation rows (x16_row), carried by workgroups
     * appended to the sort kernels' grids: the sort leaves most CUs idle and
     * the rows do not depend on it (x == NULL: none) */
    const uint16_t *x;
    _Float16 *x16;
    float *xscale;
    uint32_t dm, xperm;
};

/* Workgroups b >= b0 of a sort kernel convert activation rows [r0, r1), one
 * wave per row.  Returns true for them (the caller returns at once). */
__device__ __forceinline__ bool sort_x16_part(const SortArgs &a, uint32_t b0, uint32_t r0, uint32_t r1) {
    if (blockIdx.x < b0) return false;
    const uint32_t wpb = blockDim.x >> 6;
    const uint32_t row = r0 + (blockIdx.x - b0) * wpb + (threadIdx.x >> 6);
    if (row < r1) x16_row_scheme(a.xperm, a.x, a.dm, a.x16, a.xscale, row, threadIdx.x & 63);
    return true;
}

/* The grouped GEMMs' row tiles (moe_gemm.hip): expert x with n pairs from
 * sorted position `off` becomes ceil(n / 256) entries (expert, first
 * position, rows, 0) of `tiles3`, experts in ascending id, then the shared
 * experts (t rows each, after the P pair rows); status[4] = the count.
 * Thread x < E passes expert x's count and offset (blockDim.x >= E). */
__device__ void put_tile_lists(const SortArgs &a, uint32_t tot, uint32_t off, uint32_t *sh) {
    const MoeLayout &L = a.L;
    r9vx_u32x4 *t3 = reinterpret_cast<r9vx_u32x4 *>(a.ws + L.tiles3);
    const uint32_t tid = threadIdx.x;
    const bool mine = tid < a.e;
    const uint32_t n3 = mine ? (tot + kMoeTileM3 - 1) / kMoeTileM3 : 0u;
    uint32_t all3;
    const uint32_t b3 = block_excl_scan(n3, sh, all3);
    for (uint32_t j = 0; j < n3; ++j) {
        const uint32_t r = tot - j * kMoeTileM3;
        t3[b3 + j] = r9vx_u32x4{tid, off + j * kMoeTileM3, r < kMoeTileM3 ? r : kMoeTileM3, 0u};
    }
    const uint32_t s3 = (a.t + kMoeTileM3 - 1) / kMoeTileM3;
    for (uint32_t i = tid; i < a.shared * s3; i += blockDim.x) {
        const uint32_t sx = i / s3, j = i % s3, r = a.t - j * kMoeTileM3;
        t3[all3 + i] = r9vx_u32x4{a.e + sx, a.p + sx * a.t + j * kMoeTileM3, r < kMoeTileM3 ? r : kMoeTileM3, 0u};
    }
    if (tid == 0) reinterpret_cast<uint32_t *>(a.ws + L.status)[4] = all3 + a.shared * s3;
}

/* P <= 1024 pairs: everything in one workgroup of 1024 threads. */
__global__ __launch_bounds__(1024) void sort_small_kernel(SortArgs a) {
    __shared__ uint16_t cnt[16][kMoeMaxE];
    __shared__ uint32_t sh[16];
    __shared__ uint32_t bad_sh;
    const MoeLayout &L = a.L;
    uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    for (uint32_t i = tid; i < 16 * kMoeMaxE; i += blockDim.x) (&cnt[0][0])[i] = 0;
    if (tid == 0) bad_sh = 0;
    __syncthreads();
    bool in = tid < a.p;
    uint32_t id = in ? a.ids[tid] : 0u;
    bool valid = in && id < a.e;
    if (in && !valid) atomicOr(&bad_sh, R9VX_STATUS_BAD_EXPERT);
    uint64_t peers = match_peers(id, valid, id_bits(a.e));
    uint32_t rw = rank_below(peers, lane);
    if (valid && rw == 0) cnt[w][id] = (uint16_t)__popcll(peers);
    __syncthreads();
    uint32_t rank = rw;
    if (valid)
        for (uint32_t i = 0; i < w; ++i) rank += cnt[i][id];
    /* per-expert totals and their exclusive scan (thread e owns expert e) */
    uint32_t tot = 0;
    if (tid < a.e)
        for (uint32_t i = 0; i < 16; ++i) tot += cnt[i][tid];
    uint32_t all;
    uint32_t off = block_excl_scan(tid < a.e ? tot : 0u, sh, all);
    uint32_t *counts = reinterpret_cast<uint32_t *>(a.ws + L.counts);
    uint32_t *offsets = reinterpret_cast<uint32_t *>(a.ws + L.offsets);
    uint32_t *status = reinterpret_cast<uint32_t *>(a.ws + L.status);
    __shared__ uint32_t offs[kMoeMaxE];
    if (tid < a.e) {
        counts[tid] = tot;
        offsets[tid] = off;
        offs[tid] = off;
    }
    if (tid == 0) {
        offsets[a.e] = all;
        status[0] = bad_sh;
    }
    __syncthreads();
    if (valid) {
        uint32_t pos = offs[id] + rank;
        reinterpret_cast<uint32_t *>(a.ws + L.sorted)[pos] = tid;
        reinterpret_cast<uint32_t *>(a.ws + L.inv)[tid] = pos;
    }
    put_tile_lists(a, tot, off, sh);
}

/* ---------------------------------------------------------------- sort: large */

/* One 256-pair chunk per block: in-chunk ranks, per-expert chunk counts and
 * whether the chunk holds an id >= E. */
__global__ __launch_bounds__(256) void sort_count_kernel(SortArgs a, uint32_t xr0, uint32_t xr1) {
    __shared__ uint16_t cnt[4][kMoeMaxE];
    if (sort_x16_part(a, a.nchunk, xr0, xr1)) return;
    const MoeLayout &L = a.L;
    uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    uint32_t chunk = blockIdx.x, nchunk = a.nchunk;
    for (uint32_t i = tid; i < 4 * kMoeMaxE; i += 256) (&cnt[0][0])[i] = 0;
    __syncthreads();
    uint32_t pair = chunk * 256 + tid;
    bool in = pair < a.p;
    uint32_t id = in ? a.ids[pair] : 0u;
    bool valid = in && id < a.e;
    uint64_t peers = match_peers(id, valid, id_bits(a.e));
    uint32_t rw = rank_below(peers, lane);
    if (valid && rw == 0) cnt[w][id] = (uint16_t)__popcll(peers);
    const int bad = __syncthreads_or(in && !valid);
    if (tid == 0) reinterpret_cast<uint32_t *>(a.ws + L.cbad)[chunk] = bad ? 1u : 0u;
    if (valid) {
        uint32_t rank = rw;
        for (uint32_t i = 0; i < w; ++i) rank += cnt[i][id];
        reinterpret_cast<uint32_t *>(a.ws + L.rank)[pair] = rank;
    }
    uint32_t *cc = reinterpret_cast<uint32_t *>(a.ws + L.ccount);
    for (uint32_t e = tid; e < a.e; e += 256)
        cc[(uint64_t)e * nchunk + chunk] = (uint32_t)cnt[0][e] + cnt[1][e] + cnt[2][e] + cnt[3][e];
}

/* One wave per expert: exclusive scan of its chunk counts, and its total. */
__global__ __launch_bounds__(256) void sort_scan_kernel(SortArgs a, uint32_t nchunk, uint32_t xr0, uint32_t xr1) {
    if (sort_x16_part(a, (a.e + 3) / 4, xr0, xr1)) return;
    const MoeLayout &L = a.L;
    uint32_t lane = threadIdx.x & 63;
    uint32_t e = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (e >= a.e) return;
    const uint32_t *cc = reinterpret_cast<const uint32_t *>(a.ws + L.ccount) + (uint64_t)e * nchunk;
    uint32_t *cb = reinterpret_cast<uint32_t *>(a.ws + L.cbase) + (uint64_t)e * nchunk;
    /* the first 512 chunk counts are loaded before the scan starts */
    constexpr uint32_t kPre = 8;
    uint32_t pre[kPre];
#pragma unroll
    for (uint32_t i = 0; i < kPre; ++i) {
        const uint32_t c = 64 * i + lane;
        pre[i] = c < nchunk ? cc[c] : 0u;
    }
    uint32_t carry = 0;
#pragma unroll
    for (uint32_t i = 0; i < kPre; ++i) {
        if (64 * i >= nchunk) break;
        const uint32_t c = 64 * i + lane, v = pre[i];
        const uint32_t inc = wave_incl_scan(v, lane);
        if (c < nchunk) cb[c] = carry + inc - v;
        carry += __shfl(inc, 63, 64);
    }
    for (uint32_t c0 = 64 * kPre; c0 < nchunk; c0 += 64) {
        uint32_t c = c0 + lane;
        uint32_t v = c < nchunk ? cc[c] : 0u;
        uint32_t inc = wave_incl_scan(v, lane);
        if (c < nchunk) cb[c] = carry + inc - v;
        carry += __shfl(inc, 63, 64);
    }
    if (lane == 0) reinterpret_cast<uint32_t *>(a.ws + L.counts)[e] = carry;
}

/* One workgroup (blockDim.x >= E): the status word, the expert offsets (an
 * exclusive scan of the totals) and the tile lists. */
__global__ __launch_bounds__(1024) void sort_finish_kernel(SortArgs a, uint32_t nchunk, uint32_t xr0, uint32_t xr1) {
    __shared__ uint32_t sh[16];
    if (sort_x16_part(a, 1, xr0, xr1)) return;
    const MoeLayout &L = a.L;
    const uint32_t tid = threadIdx.x;
    const uint32_t *cbad = reinterpret_cast<const uint32_t *>(a.ws + L.cbad);
    uint32_t bad = 0;
    for (uint32_t c = tid; c < nchunk; c += blockDim.x) bad |= cbad[c];
    const uint32_t tot = tid < a.e ? reinterpret_cast<const uint32_t *>(a.ws + L.counts)[tid] : 0u;
    const int any_bad = __syncthreads_or(bad != 0u);
    uint32_t all;
    const uint32_t off = block_excl_scan(tot, sh, all);
    uint32_t *offsets = reinterpret_cast<uint32_t *>(a.ws + L.offsets);
    if (tid < a.e) offsets[tid] = off;
    if (tid == 0) {
        offsets[a.e] = all;
        reinterpret_cast<uint32_t *>(a.ws + L.status)[0] = any_bad ? R9VX_STATUS_BAD_EXPERT : 0u;
    }
    put_tile_lists(a, tot, off, sh);
}

__global__ __launch_bounds__(256) void sort_place_kernel(SortArgs a, uint32_t nchunk, uint32_t xr0, uint32_t xr1) {
    if (sort_x16_part(a, nchunk, xr0, xr1)) return;
    const MoeLayout &L = a.L;
    uint32_t pair = blockIdx.x * 256 + threadIdx.x;
    if (pair >= a.p) return;
    uint32_t id = a.ids[pair];
    if (id >= a.e) return;
    uint32_t chunk = pair / 256;
    const uint32_t *offsets = reinterpret_cast<const uint32_t *>(a.ws + L.offsets);
    const uint32_t *cb = reinterpret_cast<const uint32_t *>(a.ws + L.cbase);
    uint32_t pos = offsets[id] + cb[(uint64_t)id * nchunk + chunk] +
                   reinterpret_cast<const uint32_t *>(a.ws + L.rank)[pair];
    reinterpret_cast<uint32_t *>(a.ws + L.sorted)[pos] = pair;
    reinterpret_cast<uint32_t *>(a.ws + L.inv)[pair] = pos;
}

/* ---------------------------------------------------------------- decode FFN */

struct FfnArgs {
    const uint16_t *x;
    const uint32_t *ids;
    const uint8_t *w_gu;
    const uint8_t *w_dn;
    const float *weights;
    float *y;
    uint8_t *ws;
    MoeLayout L;
    const uint16_t *s_gu;  /* split layout: f16 d rows of w_gu / w_dn (NULL otherwise) */
    const uint16_t *s_dn;
    uint64_t gu_row_bytes; /* device bytes per gate/up weight row (r9vx_row_bytes) */
    uint64_t dn_row_bytes; /* device bytes per down weight row */
    uint32_t gu_srow, dn_srow; /* f16 d values per row of s_gu / s_dn */
    uint32_t t, e, k, dm, dff, shared, p;
    /* groups: row groups per sorted position; upw: units per wave */
    uint32_t gu_lpr_log2, gu_nseg, gu_groups, gu_upw;
    uint32_t dn_lpr_log2, dn_nseg, dn_groups, dn_upw;
};

/* Decode launch shape (compile-time tuning constants): gate/up row pairs
 * and down rows per lane group in one work unit, waves per workgroup. */
#ifndef R9VX_DEC_GU_PAIRS
#define R9VX_DEC_GU_PAIRS 1
#endif
#ifndef R9VX_DEC_DN_ROWS
#define R9VX_DEC_DN_ROWS 2
#endif
#ifndef R9VX_DEC_WAVES
#define R9VX_DEC_WAVES 4
#endif
constexpr int kDecPairs = R9VX_DEC_GU_PAIRS;
constexpr int kDecDnRows = R9VX_DEC_DN_ROWS;
constexpr int kDecWaves = R9VX_DEC_WAVES;

/* Token and expert of row pos: the decode path keeps the rows in pair order
 * (pos = token * K + slot, no sort pass), the shared experts' T rows each
 * after the P pairs; false for an id >= E (nothing is read for it, and the
 * combine refuses the call). */
__device__ __forceinline__ bool pos_meta(const FfnArgs &a, uint32_t pos, uint32_t &tok, uint32_t &expert) {
    if (pos >= a.p) {
        tok = (pos - a.p) % a.t;
        expert = a.e + (pos - a.p) / a.t;
        return true;
    }
    expert = a.ids[pos];
    tok = pos / a.k;
    return expert < a.e;
}

/* Steps (unit, K segment) one wave carries; all of their weight loads are
 * issued before any of them is used. */
#ifndef R9VX_DEC_STEPS
#define R9VX_DEC_STEPS 2
#endif
constexpr uint32_t kDecSteps = R9VX_DEC_STEPS;

/* A wave's units: [u0, u0 + n), n <= upw, in sorted-position order, so that
 * they walk consecutive weight rows; the host caps upw at the row groups per
 * position, so a wave's units share at most two positions (expert,
 * activation row).  A wave with more than kDecSteps steps takes them
 * kDecSteps at a time. */
__device__ __forceinline__ bool wave_units(uint32_t units, uint32_t upw, uint32_t &u0, uint32_t &n) {
    const uint32_t gw = __builtin_amdgcn_readfirstlane(blockIdx.x * kDecWaves + (threadIdx.x >> 6));
    u0 = gw * upw;
    if (u0 >= units) return false;
    n = units - u0 < upw ? units - u0 : upw;
    return true;
}

/* (position, row group, K segment) of a step, advanced without division */
struct Cur {
    uint32_t pos, g, seg;
};
__device__ __forceinline__ void advance(Cur &c, uint32_t nseg, uint32_t groups) {
    if (++c.seg == nseg) {
        c.seg = 0;
        if (++c.g == groups) {
            c.g = 0;
            ++c.pos;
        }
    }
}

/* Weight registers of one gate/up step: chunk ci of kPairs (gate, up) row
 * pairs. */
template <int GU>
struct GuRegs {
    static constexpr bool kIq3 = GU == R9VX_SCHEME_IQ3_S;
    static constexpr bool kSplit = GU == R9VX_SCHEME_Q8_0 || GU == R9VX_SCHEME_Q6_K;
    using Pay = typename std::conditional<kIq3 || kSplit, Payload2, r9vx_u32x4>::type;
    Pay qg[kDecPairs], qu[kDecPairs];
    Hdr hg[kDecPairs], hu[kDecPairs];
};

/* Loads of a gate/up step: rows (g * kPairs + r) * rpi + slot of the
 * expert's gate half and the same rows of its up half (clamped to Dff - 1;
 * the rows past Dff are never stored). */
template <int GU>
__device__ __forceinline__ void gu_load(const FfnArgs &a, uint32_t expert, uint32_t g, uint32_t ci, uint32_t rpi,
                                        uint32_t slot, GuRegs<GU> &w) {
    const uint8_t *wexp = a.w_gu + (uint64_t)expert * 2 * a.dff * a.gu_row_bytes;
    const uint16_t *sexp = GuRegs<GU>::kSplit ? a.s_gu + (uint64_t)expert * 2 * a.dff * a.gu_srow : nullptr;
#pragma unroll
    for (int r = 0; r < kDecPairs; ++r) {
        const uint32_t row = (g * kDecPairs + r) * rpi + slot;
        const uint32_t rr = row < a.dff ? row : a.dff - 1;
        if constexpr (GuRegs<GU>::kSplit) {
            load_chunk_split<GU>(wexp + (uint64_t)rr * a.gu_row_bytes, sexp + (uint64_t)rr * a.gu_srow, ci, w.qg[r],
                                 w.hg[r]);
            load_chunk_split<GU>(wexp + (uint64_t)(a.dff + rr) * a.gu_row_bytes,
                                 sexp + (uint64_t)(a.dff + rr) * a.gu_srow, ci, w.qu[r], w.hu[r]);
        } else if constexpr (GuRegs<GU>::kIq3) {
            load_chunk_iq3s(wexp + (uint64_t)rr * a.gu_row_bytes, ci, w.qg[r], w.hg[r]);
            load_chunk_iq3s(wexp + (uint64_t)(a.dff + rr) * a.gu_row_bytes, ci, w.qu[r], w.hu[r]);
        } else {
            load_chunk<GU>(wexp + (uint64_t)rr * a.gu_row_bytes, ci, w.qg[r], w.hg[r]);
            load_chunk<GU>(wexp + (uint64_t)(a.dff + rr) * a.gu_row_bytes, ci, w.qu[r], w.hu[r]);
        }
    }
}

template <int GU>
__device__ __forceinline__ void gu_dot(const GuRegs<GU> &w, uint32_t ci, const XChunk<GU, false> (&xc)[1],
                                       float (&ag)[kDecPairs][1], float (&au)[kDecPairs][1], const uint32_t *lut) {
#pragma unroll
    for (int r = 0; r < kDecPairs; ++r) {
        if constexpr (GuRegs<GU>::kSplit) {
            chunk_dot_split<GU, 1>(w.qg[r], w.hg[r], ci & 7, xc, ag[r]);
            chunk_dot_split<GU, 1>(w.qu[r], w.hu[r], ci & 7, xc, au[r]);
        } else if constexpr (GuRegs<GU>::kIq3) {
            chunk_dot_iq3s<1>(w.qg[r], w.hg[r], ci & 7, xc, ag[r], lut);
            chunk_dot_iq3s<1>(w.qu[r], w.hu[r], ci & 7, xc, au[r], lut);
        } else {
            chunk_dot<GU, false, 1>(w.qg[r], w.hg[r], ci & 7, xc, ag[r], lut);
            chunk_dot<GU, false, 1>(w.qu[r], w.hu[r], ci & 7, xc, au[r], lut);
        }
    }
}

/* Weight registers of one down step: chunk ci of kDnRows rows. */
template <int DN>
struct DnRegs {
    static constexpr bool kIq3 = DN == R9VX_SCHEME_IQ3_S;
    static constexpr bool kSplit = DN == R9VX_SCHEME_Q8_0 || DN == R9VX_SCHEME_Q6_K;
    static constexpr bool kF32x = kIq3 || kSplit; /* chunk_dot_f32x against the f32 h rows */
    static constexpr bool kF16 = DN == R9VX_SCHEME_Q4_K;
    using Pay = typename std::conditional<kF32x, Payload2, r9vx_u32x4>::type;
    Pay q[kDecDnRows];
    Hdr hd[kDecDnRows];
};

template <int DN>
__device__ __forceinline__ void dn_load(const FfnArgs &a, uint32_t expert, uint32_t g, uint32_t ci, uint32_t rpi,
                                        uint32_t slot, DnRegs<DN> &w) {
    const uint8_t *wexp = a.w_dn + (uint64_t)expert * a.dm * a.dn_row_bytes;
    const uint16_t *sexp = DnRegs<DN>::kSplit ? a.s_dn + (uint64_t)expert * a.dm * a.dn_srow : nullptr;
#pragma unroll
    for (int r = 0; r < kDecDnRows; ++r) {
        const uint32_t row = (g * kDecDnRows + r) * rpi + slot;
        const uint32_t rr = row < a.dm ? row : a.dm - 1;
        if constexpr (DnRegs<DN>::kSplit)
            load_chunk_split<DN>(wexp + (uint64_t)rr * a.dn_row_bytes, sexp + (uint64_t)rr * a.dn_srow, ci, w.q[r],
                                 w.hd[r]);
        else if constexpr (DnRegs<DN>::kIq3)
            load_chunk_iq3s(wexp + (uint64_t)rr * a.dn_row_bytes, ci, w.q[r], w.hd[r]);
        else
            load_chunk<DN>(wexp + (uint64_t)rr * a.dn_row_bytes, ci, w.q[r], w.hd[r]);
    }
}

/* The h chunk of one (position, K segment) arranged for the down dots.
 * Q4_K: the chunk's 32 h values scaled by 2^-e (e from the chunk's max|h|,
 * so |h| 2^-e < 2^15; e = 0 unless max|h| >= 2^15) and rounded once to
 * fp16, paired like the weights; weights as fp16 1024 + q, so one
 * v_dot2_f32_f16 does two products exactly in f32, and the 1024 offset
 * comes off with the sums of the same rounded values.  IQ4_XS: the f32 path
 * of the dense GEMV. */
template <int DN>
struct DnX {
    XChunk<DN, true> xc[1];
    uint32_t hp[16];
    float hsc, slo, shi;
};

template <int DN>
__device__ __forceinline__ void dn_arrange(const XRaw<true> &xr, DnX<DN> &d) {
    if constexpr (DnRegs<DN>::kF16) {
        float mx = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(xr.v[i].x), fabsf(xr.v[i].y)), fmaxf(fabsf(xr.v[i].z), fabsf(xr.v[i].w))));
        d.hsc = ldexpf(1.0f, row_shift(mx));
        const float inv = 1.0f / d.hsc; /* a power of two: exact */
        float lo[16], hi[16];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                lo[4 * i + j] = xr.v[i][j] * inv;
                hi[4 * i + j] = xr.v[4 + i][j] * inv;
            }
        /* dword dw of the payload holds bytes 4dw..4dw+3: pairs
         * {lo(4dw), lo(4dw+2)}, {lo(4dw+1), lo(4dw+3)}, {hi(4dw), hi(4dw+2)},
         * {hi(4dw+1), hi(4dw+3)} */
#pragma unroll
        for (int dw = 0; dw < 4; ++dw) {
            d.hp[4 * dw + 0] = pack_h2(lo[4 * dw], lo[4 * dw + 2]);
            d.hp[4 * dw + 1] = pack_h2(lo[4 * dw + 1], lo[4 * dw + 3]);
            d.hp[4 * dw + 2] = pack_h2(hi[4 * dw], hi[4 * dw + 2]);
            d.hp[4 * dw + 3] = pack_h2(hi[4 * dw + 1], hi[4 * dw + 3]);
        }
        const uint32_t one2 = 0x3C003C00u; /* fp16 {1, 1} */
        float slo = 0.f, shi = 0.f;
#pragma unroll
        for (int dw = 0; dw < 4; ++dw) {
            slo = r9vx_dot2_f16(d.hp[4 * dw + 0], one2, slo);
            slo = r9vx_dot2_f16(d.hp[4 * dw + 1], one2, slo);
            shi = r9vx_dot2_f16(d.hp[4 * dw + 2], one2, shi);
            shi = r9vx_dot2_f16(d.hp[4 * dw + 3], one2, shi);
        }
        d.slo = slo;
        d.shi = shi;
    } else {
        arrange_x<DN, true>(xr, d.xc[0]);
    }
}

template <int DN>
__device__ __forceinline__ void dn_dot(const DnRegs<DN> &w, uint32_t ci, const DnX<DN> &d,
                                       float (&acc)[kDecDnRows][1], const uint32_t *lut) {
#pragma unroll
    for (int r = 0; r < kDecDnRows; ++r) {
        if constexpr (DnRegs<DN>::kF32x) {
            acc[r][0] += chunk_dot_f32x<DN>(w.q[r], w.hd[r], ci & 7, d.xc[0], lut);
        } else if constexpr (DnRegs<DN>::kF16) {
            const uint32_t qw[4] = {w.q[r].x, w.q[r].y, w.q[r].z, w.q[r].w};
            const Hdr &hh = w.hd[r];
            const float dd = r9vx_f16_to_f32((uint16_t)(hh.v.x & 0xFFFF));
            const float dmin = r9vx_f16_to_f32((uint16_t)(hh.v.x >> 16));
            const uint32_t sm = r9vx_q4k_pair_bytes(hh.v, (ci & 7) >> 1);
            const float dl0 = dd * (float)(sm & 0xFFu), dl1 = dd * (float)((sm >> 8) & 0xFFu);
            const float off0 = fmaf(1024.f, dl0, dmin * (float)((sm >> 16) & 0xFFu));
            const float off1 = fmaf(1024.f, dl1, dmin * (float)(sm >> 24));
            float dlo = 0.f, dhi = 0.f;
#pragma unroll
            for (int dw = 0; dw < 4; ++dw) {
                dlo = r9vx_dot2_f16(r9vx_and_or(qw[dw], 0x000F000Fu, 0x64006400u), d.hp[4 * dw + 0], dlo);
                dlo = r9vx_dot2_f16(r9vx_and_or(qw[dw] >> 8, 0x000F000Fu, 0x64006400u), d.hp[4 * dw + 1], dlo);
                dhi = r9vx_dot2_f16(r9vx_and_or(qw[dw] >> 4, 0x000F000Fu, 0x64006400u), d.hp[4 * dw + 2], dhi);
                dhi = r9vx_dot2_f16(r9vx_and_or(qw[dw] >> 12, 0x000F000Fu, 0x64006400u), d.hp[4 * dw + 3], dhi);
            }
            acc[r][0] += d.hsc * (dl0 * dlo + dl1 * dhi - (off0 * d.slo + off1 * d.shi));
        } else {
            chunk_dot<DN, true, 1>(w.q[r], w.hd[r], ci & 7, d.xc, acc[r], lut);
        }
    }
}

/* gate/up GEMV + SwiGLU.  A unit is kPairs * (64 / LPR) (gate, up) row
 * pairs of one sorted position. */
template <int GU>
__global__ __launch_bounds__(kDecWaves * 64) void moe_gu_kernel(FfnArgs a) {
    constexpr bool kIq3 = GU == R9VX_SCHEME_IQ3_S;
    __shared__ __attribute__((aligned(16))) uint32_t lut[kIq3 ? 1024 : 256];
    if constexpr (GU == R9VX_SCHEME_IQ4_XS) init_iq4_lut(lut, threadIdx.x, blockDim.x);
    if constexpr (kIq3) build_iq3s_lut(lut, threadIdx.x, blockDim.x);
    __syncthreads(); /* the last barrier: waves run independently from here */
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t lpr = 1u << a.gu_lpr_log2, rpi = 64u >> a.gu_lpr_log2;
    const uint32_t lir = lane & (lpr - 1), slot = lane >> a.gu_lpr_log2;
    const uint32_t nseg = a.gu_nseg, groups = a.gu_groups;
    uint32_t u0, n;
    if (!wave_units((a.p + a.shared * a.t) * groups, a.gu_upw, u0, n)) return;
    const uint32_t nsteps = n * nseg;
    /* the (at most two) positions of the wave's units */
    uint32_t tok[2], expert[2];
    const uint32_t pos0 = u0 / groups, pos1 = (u0 + n - 1) / groups;
    const bool ok0 = pos_meta(a, pos0, tok[0], expert[0]), ok1 = pos_meta(a, pos1, tok[1], expert[1]);
    if (!ok0 || !ok1) return; /* refused: nothing is read or written */
    float *h = reinterpret_cast<float *>(a.ws + a.L.h);

    XChunk<GU, false> xc[1];
    uint32_t xpos = ~0u, xseg = ~0u;
    float ag[kDecPairs][1], au[kDecPairs][1];
    Cur lc{pos0, u0 % groups, 0u}, c = lc; /* load and compute cursors */
    GuRegs<GU> wr[kDecSteps];
    for (uint32_t base = 0; base < nsteps; base += kDecSteps) {
        /* 1. every weight load of the batch's steps (steps past the last repeat it) */
#pragma unroll
        for (uint32_t s = 0; s < kDecSteps; ++s) {
            gu_load<GU>(a, expert[lc.pos == pos0 ? 0 : 1], lc.g, lc.seg * lpr + lir, rpi, slot, wr[s]);
            if (base + s + 1 < nsteps) advance(lc, nseg, groups);
        }

        /* 2. the steps in order; the arranged activation chunk is reused while
         * (position, segment) stays the same */
#pragma unroll
        for (uint32_t s = 0; s < kDecSteps; ++s) {
            if (base + s >= nsteps) break;
            const uint32_t ci = c.seg * lpr + lir;
            if (c.pos != xpos || c.seg != xseg) {
                uint32_t klo, khi;
                chunk_k<GU>(ci, klo, khi);
                XRaw<false> xr;
                load_x_raw<false>(a.x + (uint64_t)tok[c.pos == pos0 ? 0 : 1] * a.dm, klo, khi, xr);
                arrange_x<GU, false>(xr, xc[0]);
                xpos = c.pos;
                xseg = c.seg;
            }
            if (c.seg == 0)
#pragma unroll
                for (int r = 0; r < kDecPairs; ++r) ag[r][0] = au[r][0] = 0.f;
            gu_dot<GU>(wr[s], ci, xc, ag, au, lut);
            if (c.seg + 1 == nseg) {
                float gu[2][kDecPairs];
#pragma unroll
                for (int r = 0; r < kDecPairs; ++r) {
                    gu[0][r] = ag[r][0];
                    gu[1][r] = au[r][0];
                }
                const uint32_t pos = c.pos, g = c.g;
                lane_reduce_w<kDecPairs, 2>(gu, lane, a.gu_lpr_log2, [&](int r, const float (&val)[2]) {
                    const uint32_t row = (g * kDecPairs + r) * rpi + slot;
                    if (row >= a.dff) return;
                    h[(uint64_t)pos * a.dff + row] = swiglu_fast(val[0], val[1]);
                });
            }
            advance(c, nseg, groups);
        }
    }
}

/* down GEMV: o[pos, d] = h[pos, :] . Wd[d, :]; a unit is kDecDnRows * (64 /
 * LPR) rows of one sorted position. */
template <int DN>
__global__ __launch_bounds__(kDecWaves * 64) void moe_down_kernel(FfnArgs a) {
    constexpr bool kIq3 = DN == R9VX_SCHEME_IQ3_S;
    __shared__ __attribute__((aligned(16))) uint32_t lut[kIq3 ? 1024 : 256];
    if constexpr (DN == R9VX_SCHEME_IQ4_XS) init_iq4_lut(lut, threadIdx.x, blockDim.x);
    if constexpr (kIq3) build_iq3s_lut(lut, threadIdx.x, blockDim.x);
    __syncthreads(); /* the last barrier: waves run independently from here */
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t lpr = 1u << a.dn_lpr_log2, rpi = 64u >> a.dn_lpr_log2;
    const uint32_t lir = lane & (lpr - 1), slot = lane >> a.dn_lpr_log2;
    const uint32_t nseg = a.dn_nseg, groups = a.dn_groups;
    uint32_t u0, n;
    if (!wave_units((a.p + a.shared * a.t) * groups, a.dn_upw, u0, n)) return;
    const uint32_t nsteps = n * nseg;
    uint32_t tok[2], expert[2];
    const uint32_t pos0 = u0 / groups, pos1 = (u0 + n - 1) / groups;
    const bool ok0 = pos_meta(a, pos0, tok[0], expert[0]), ok1 = pos_meta(a, pos1, tok[1], expert[1]);
    if (!ok0 || !ok1) return;
    const float *h = reinterpret_cast<const float *>(a.ws + a.L.h);
    float *o = reinterpret_cast<float *>(a.ws + a.L.o);

    /* the h chunk of (position, segment), arranged once and reused while it
     * stays the same */
    DnX<DN> hx;
    uint32_t xpos = ~0u, xseg = ~0u;
    float acc[kDecDnRows][1];
    Cur lc{pos0, u0 % groups, 0u}, c = lc; /* load and compute cursors */
    DnRegs<DN> wr[kDecSteps];
    for (uint32_t base = 0; base < nsteps; base += kDecSteps) {
        /* every weight load of the batch's steps (steps past the last repeat it) */
#pragma unroll
        for (uint32_t s = 0; s < kDecSteps; ++s) {
            dn_load<DN>(a, expert[lc.pos == pos0 ? 0 : 1], lc.g, lc.seg * lpr + lir, rpi, slot, wr[s]);
            if (base + s + 1 < nsteps) advance(lc, nseg, groups);
        }
#pragma unroll
        for (uint32_t s = 0; s < kDecSteps; ++s) {
            if (base + s >= nsteps) break;
            const uint32_t ci = c.seg * lpr + lir;
            if (c.pos != xpos || c.seg != xseg) {
                uint32_t klo, khi;
                chunk_k<DN>(ci, klo, khi);
                XRaw<true> xr;
                load_x_raw<true>(h + (uint64_t)c.pos * a.dff, klo, khi, xr);
                dn_arrange<DN>(xr, hx);
                xpos = c.pos;
                xseg = c.seg;
            }
            if (c.seg == 0)
#pragma unroll
                for (int r = 0; r < kDecDnRows; ++r) acc[r][0] = 0.f;
            dn_dot<DN>(wr[s], ci, hx, acc, lut);
            if (c.seg + 1 == nseg) {
                float v[1][kDecDnRows];
#pragma unroll
                for (int r = 0; r < kDecDnRows; ++r) v[0][r] = acc[r][0];
                const uint32_t pos = c.pos, g = c.g;
                lane_reduce_w<kDecDnRows, 1>(v, lane, a.dn_lpr_log2, [&](int r, const float (&val)[1]) {
                    const uint32_t row = (g * kDecDnRows + r) * rpi + slot;
                    if (row >= a.dm) return;
                    o[(uint64_t)pos * a.dm + row] = val[0];
                });
            }
            advance(c, nseg, groups);
        }
    }
}

/* Pipelined forms for rows of one K segment (nseg == 1, K <= 2048): a wave
 * walks its units (row groups of one position: the host makes the units per
 * wave divide the row groups per position) in batches of kDecSteps and
 * issues the weight loads of batch b + 1 before it computes batch b, so a
 * batch's loads are in flight while the previous batch computes.  Every
 * load of the loop is issued unconditionally (steps past the wave's last
 * repeat its addresses): a load issued on one path only would make the next
 * wait a wait for everything.  The step outputs wait in LDS and are stored
 * after the wave's last load, because a store issued between two loads
 * turns the wait for the older load into a wait for every outstanding
 * memory operation; the gate/up kernel applies SiLU(g) * u there (the
 * hardware exp and reciprocal, as the grouped GEMMs), one row per lane.  A
 * lane's K chunk is the same in every step, so its activation chunk is
 * loaded and arranged once.  The arithmetic per step is that of
 * moe_gu_kernel / moe_down_kernel. */
#ifndef R9VX_GU_PIPE_STEPS
#define R9VX_GU_PIPE_STEPS 1
#endif
#ifndef R9VX_GU_PIPE_UPW
#define R9VX_GU_PIPE_UPW 2
#endif
#ifndef R9VX_DN_PIPE_STEPS
#define R9VX_DN_PIPE_STEPS 1
#endif
#ifndef R9VX_DN_PIPE_UPW
#define R9VX_DN_PIPE_UPW 8
#endif
/* steps per batch and units per wave (at most) of the two kernels */
constexpr uint32_t kGuPipeSteps = R9VX_GU_PIPE_STEPS, kGuPipeUpw = R9VX_GU_PIPE_UPW;
constexpr uint32_t kDnPipeSteps = R9VX_DN_PIPE_STEPS, kDnPipeUpw = R9VX_DN_PIPE_UPW;
static_assert((kDecPairs & (kDecPairs - 1)) == 0 && (kDecDnRows & (kDecDnRows - 1)) == 0,
              "rows per step must be a power of two");

/* The LDS tables of a decode kernel (IQ4_XS codebook pairs, IQ3_S grid),
 * loaded to registers as the kernel's first memory operations and written
 * to LDS after the first weight loads are issued: loads complete in order,
 * so the LDS writes wait for the table words only, and the tables' latency
 * overlaps the weights'. */
template <int S>
struct DecTables {
    r9vx_u32x4 iq4;
    uint32_t g[2];
    __device__ __forceinline__ void load(uint32_t tid) {
        if constexpr (S == R9VX_SCHEME_IQ4_XS)
            if (tid < 64) iq4 = reinterpret_cast<const r9vx_u32x4 *>(kIq4PairLut.v)[tid];
        if constexpr (S == R9VX_SCHEME_IQ3_S) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
                if (tid + 256 * i < 512) g[i] = kIq3sGrid[tid + 256 * i];
        }
    }
    __device__ __forceinline__ void store(uint32_t *lut, uint32_t tid) const {
        if constexpr (S == R9VX_SCHEME_IQ4_XS)
            if (tid < 64) reinterpret_cast<r9vx_u32x4 *>(lut)[tid] = iq4;
        if constexpr (S == R9VX_SCHEME_IQ3_S) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint32_t e = tid + 256 * i;
                if (e >= 512) continue;
                uint32_t h[4];
#pragma unroll
                for (int b = 0; b < 4; ++b) h[b] = __builtin_bit_cast(uint32_t, (float)((g[i] >> (8 * b)) & 0xFF)) >> 16;
                lut[2 * e] = h[0] | (h[1] << 16);
                lut[2 * e + 1] = h[2] | (h[3] << 16);
            }
        }
    }
};

/* Workgroup barrier over LDS only: the weight loads in flight are not
 * waited for. */
__device__ __forceinline__ void lds_only_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

/* The wave's position and first row group; a wave without units, or with a
 * refused id, gets expert 0's rows of position 0 (in bounds, never used) so
 * that every path issues the same loads and the waits after them stay
 * counted.  Returns whether the wave computes. */
__device__ __forceinline__ bool pipe_wave(const FfnArgs &a, uint32_t groups, uint32_t upw, uint32_t &u0, uint32_t &n,
                                          uint32_t &pos, uint32_t &g0, uint32_t &tok, uint32_t &expert) {
    n = 0;
    bool ok = wave_units((a.p + a.shared * a.t) * groups, upw, u0, n);
    pos = ok ? u0 / groups : 0u;
    ok = pos_meta(a, pos, tok, expert) && ok; /* refused: nothing is read or written */
    if (!ok) pos = tok = expert = 0;
    g0 = ok ? u0 - pos * groups : 0u;
    return ok;
}

template <int GU>
__global__ __launch_bounds__(kDecWaves * 64) void moe_gu_pipe_kernel(FfnArgs a) {
    constexpr bool kIq3 = GU == R9VX_SCHEME_IQ3_S;
    constexpr uint32_t kObuf = kGuPipeUpw * kDecPairs * 8; /* rows per wave, at most */
    __shared__ __attribute__((aligned(16))) uint32_t lut[kIq3 ? 1024 : 256];
    __shared__ float2 obuf[kDecWaves][kObuf]; /* (gate, up) dot of each row */
    DecTables<GU> tb;
    tb.load(threadIdx.x);
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t rpi = 64u >> a.gu_lpr_log2, rps = kDecPairs * rpi;
    const uint32_t ci = lane & ((1u << a.gu_lpr_log2) - 1), slot = lane >> a.gu_lpr_log2;
    uint32_t u0, n, pos, g0, tok, expert;
    const bool ok = pipe_wave(a, a.gu_groups, a.gu_upw, u0, n, pos, g0, tok, expert);
    float2 *ob = obuf[threadIdx.x >> 6];

    uint32_t klo, khi;
    chunk_k<GU>(ci, klo, khi);
    XRaw<false> xr;
    load_x_raw<false>(a.x + (uint64_t)tok * a.dm, klo, khi, xr);
    uint32_t li = 0, cs = 0; /* step indices of the next load and the next compute */
    auto issue = [&](GuRegs<GU> (&w)[kGuPipeSteps]) {
#pragma unroll
        for (uint32_t s = 0; s < kGuPipeSteps; ++s) {
            gu_load<GU>(a, expert, g0 + li, ci, rpi, slot, w[s]);
            if (li + 1 < n) ++li;
        }
    };
    XChunk<GU, false> xc[1];
    auto compute = [&](const GuRegs<GU> (&w)[kGuPipeSteps]) {
#pragma unroll
        for (uint32_t s = 0; s < kGuPipeSteps; ++s) {
            if (cs >= n) break;
            float ag[kDecPairs][1], au[kDecPairs][1];
#pragma unroll
            for (int r = 0; r < kDecPairs; ++r) ag[r][0] = au[r][0] = 0.f;
            gu_dot<GU>(w[s], ci, xc, ag, au, lut);
            float gu[2][kDecPairs];
#pragma unroll
            for (int r = 0; r < kDecPairs; ++r) {
                gu[0][r] = ag[r][0];
                gu[1][r] = au[r][0];
            }
            float2 *os = ob + cs * rps;
            lane_reduce_w<kDecPairs, 2>(gu, lane, a.gu_lpr_log2, [&](int r, const float (&val)[2]) {
                os[r * rpi + slot] = float2{val[0], val[1]};
            });
            ++cs;
        }
    };
    GuRegs<GU> wa[kGuPipeSteps], wb[kGuPipeSteps];
    issue(wa);
    tb.store(lut, threadIdx.x);
    lds_only_barrier(); /* the last barrier: waves run independently from here */
    if (!ok) return;
    arrange_x<GU, false>(xr, xc[0]);
    const uint32_t nb = (n + kGuPipeSteps - 1) / kGuPipeSteps;
    for (uint32_t b = 0;; b += 2) {
        issue(wb);
        compute(wa);
        if (b + 2 >= nb) {
            compute(wb);
            break;
        }
        issue(wa);
        compute(wb);
    }
    /* h rows g0 * rps + j, j < n * rps: one row per lane */
    wave_lds_sync();
    float *h = reinterpret_cast<float *>(a.ws + a.L.h) + (uint64_t)pos * a.dff + g0 * rps;
    const uint32_t nrows = min(n * rps, a.dff - g0 * rps);
    for (uint32_t j = lane; j < nrows; j += 64) {
        const float2 v = ob[j];
        h[j] = swiglu_fast(v.x, v.y);
    }
}

template <int DN>
__global__ __launch_bounds__(kDecWaves * 64) void moe_down_pipe_kernel(FfnArgs a) {
    constexpr bool kIq3 = DN == R9VX_SCHEME_IQ3_S;
    constexpr uint32_t kObuf = kDnPipeUpw * kDecDnRows * 8;
    __shared__ __attribute__((aligned(16))) uint32_t lut[kIq3 ? 1024 : 256];
    __shared__ float obuf[kDecWaves][kObuf];
    DecTables<DN> tb;
    tb.load(threadIdx.x);
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t rpi = 64u >> a.dn_lpr_log2, rps = kDecDnRows * rpi;
    const uint32_t ci = lane & ((1u << a.dn_lpr_log2) - 1), slot = lane >> a.dn_lpr_log2;
    uint32_t u0, n, pos, g0, tok, expert;
    const bool ok = pipe_wave(a, a.dn_groups, a.dn_upw, u0, n, pos, g0, tok, expert);
    float *ob = obuf[threadIdx.x >> 6];

    uint32_t klo, khi;
    chunk_k<DN>(ci, klo, khi);
    XRaw<true> xr;
    load_x_raw<true>(reinterpret_cast<const float *>(a.ws + a.L.h) + (uint64_t)pos * a.dff, klo, khi, xr);
    uint32_t li = 0, cs = 0;
    auto issue = [&](DnRegs<DN> (&w)[kDnPipeSteps]) {
#pragma unroll
        for (uint32_t s = 0; s < kDnPipeSteps; ++s) {
            dn_load<DN>(a, expert, g0 + li, ci, rpi, slot, w[s]);
            if (li + 1 < n) ++li;
        }
    };
    DnX<DN> hx;
    auto compute = [&](const DnRegs<DN> (&w)[kDnPipeSteps]) {
#pragma unroll
        for (uint32_t s = 0; s < kDnPipeSteps; ++s) {
            if (cs >= n) break;
            float acc[kDecDnRows][1];
#pragma unroll
            for (int r = 0; r < kDecDnRows; ++r) acc[r][0] = 0.f;
            dn_dot<DN>(w[s], ci, hx, acc, lut);
            float v[1][kDecDnRows];
#pragma unroll
            for (int r = 0; r < kDecDnRows; ++r) v[0][r] = acc[r][0];
            float *os = ob + cs * rps;
            lane_reduce_w<kDecDnRows, 1>(v, lane, a.dn_lpr_log2,
                                         [&](int r, const float (&val)[1]) { os[r * rpi + slot] = val[0]; });
            ++cs;
        }
    };
    DnRegs<DN> wa[kDnPipeSteps], wb[kDnPipeSteps];
    issue(wa);
    tb.store(lut, threadIdx.x);
    lds_only_barrier(); /* the last barrier: waves run independently from here */
    if (!ok) return;
    dn_arrange<DN>(xr, hx);
    const uint32_t nb = (n + kDnPipeSteps - 1) / kDnPipeSteps;
    for (uint32_t b = 0;; b += 2) {
        issue(wb);
        compute(wa);
        if (b + 2 >= nb) {
            compute(wb);
            break;
        }
        issue(wa);
        compute(wb);
    }
    wave_lds_sync();
    float *o = reinterpret_cast<float *>(a.ws + a.L.o) + (uint64_t)pos * a.dm + g0 * rps;
    const uint32_t nrows = min(n * rps, a.dm - g0 * rps);
    for (uint32_t j = lane; j < nrows; j += 64) o[j] = ob[j];
}

}  // namespace

/* ---------------------------------------------------------------- combine */

/* y[t, d] = sum over the token's pairs in ascending sorted position (=
 * ascending expert, then slot) of w * o, then + each shared expert's o.
 * Every wave works alone: it loads all ids of the batch (the refusal below)
 * and the token's K ids and weights in one round of loads, ranks the K
 * slots by (expert, slot) across its lanes, and then issues the token's row
 * loads in rank order (the order is the same in every lane) before the
 * ordered f32 sum. */
__global__ __launch_bounds__(256) void r9vx_moe_combine_kernel(MoeCombineArgs a) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t t = blockIdx.y, kk = a.k;
    /* the refusal of moe_ffn.rs:440-465 for the whole batch (the decode path
     * has no sort pass): every wave checks every id (p = t * K <= 8 * 32,
     * four per lane) before writing y, and block (0, 0) leaves the call's
     * status word */
    uint32_t badl = 0;
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
        const uint32_t i = lane + 64 * j;
        if (i < a.p && a.ids[i] >= a.e) badl = 1u;
    }
    uint32_t key = ~0u;
    float wt = 0.f;
    if (lane < kk) {
        key = (a.ids[(uint64_t)t * kk + lane] << 8) | lane;
        wt = a.weights[(uint64_t)t * kk + lane];
    }
    const bool bad = __ballot(badl) != 0ull;
    if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0)
        reinterpret_cast<uint32_t *>(a.ws + a.L.status)[0] = bad ? R9VX_STATUS_BAD_EXPERT : 0u;
    if (bad) return;
    /* rank of the lane's slot by key (keys are distinct; lanes >= K rank K) */
    uint32_t rank = 0;
    for (uint32_t i = 0; i < kk; ++i) rank += (uint32_t)__builtin_amdgcn_readlane((int)key, (int)i) < key ? 1u : 0u;
    const uint32_t d0 = (blockIdx.x * 256 + threadIdx.x) * 4;
    const bool live = d0 < a.dm;
    const float *o = reinterpret_cast<const float *>(a.ws + a.L.o);
    r9vx_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    /* Eight rows in flight at a time; rows[] is indexed by constants only so
     * it stays in registers. */
    for (uint32_t jb = 0; jb < kk; jb += 8) {
        r9vx_f32x4 rows[8];
        float w[8];
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j) {
            if (jb + j >= kk) break;
            const uint32_t slot = (uint32_t)__builtin_ctzll(__ballot(rank == jb + j));
            w[j] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wt), (int)slot));
            if (live) rows[j] = *reinterpret_cast<const r9vx_f32x4 *>(o + ((uint64_t)t * kk + slot) * a.dm + d0);
        }
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j) {
            if (jb + j >= kk) break;
            acc.x = acc.x + w[j] * rows[j].x;
            acc.y = acc.y + w[j] * rows[j].y;
            acc.z = acc.z + w[j] * rows[j].z;
            acc.w = acc.w + w[j] * rows[j].w;
        }
    }
    if (!live) return;
    for (uint32_t s = 0; s < a.shared; ++s) {
        r9vx_f32x4 v = *reinterpret_cast<const r9vx_f32x4 *>(o + (uint64_t)(a.p + s * a.t + t) * a.dm + d0);
        acc.x = acc.x + v.x;
        acc.y = acc.y + v.y;
        acc.z = acc.z + v.z;
        acc.w = acc.w + v.w;
    }
    *reinterpret_cast<r9vx_f32x4 *>(a.y + (uint64_t)t * a.dm + d0) = acc;
}

/* The same combine over the grouped path's fp16 rows: row value = o16 *
 * oscale[row, d / 64] (exact: the scale is a power of two), summed in the
 * same order.  The o rows are read once and y is written once, both with
 * non-temporal accesses so the stream does not evict what the GEMMs keep in
 * the caches (configs[4]: 79 -> 69 us). */
__global__ __launch_bounds__(256) void r9vx_moe_combine16_kernel(MoeCombineArgs a) {
    __shared__ uint32_t spos[kMoeMaxK], opos[kMoeMaxK];
    __shared__ float sw[kMoeMaxK], ow[kMoeMaxK];
    const uint32_t *status = reinterpret_cast<const uint32_t *>(a.ws + a.L.status);
    const uint32_t t = blockIdx.y;
    const uint32_t kk = a.k;
    const uint32_t *inv = reinterpret_cast<const uint32_t *>(a.ws + a.L.inv);
    /* the status word, the token's positions and weights in one round of
     * loads (all inside the workspace and the weights array) */
    const uint32_t st = status[0];
    uint32_t ps = 0;
    float wv = 0.f;
    if (threadIdx.x < kk) {
        ps = inv[(uint64_t)t * kk + threadIdx.x];
        wv = a.weights[(uint64_t)t * kk + threadIdx.x];
    }
    if (st != 0u) return; /* uniform: a refused call writes no y */
    if (threadIdx.x < kk) {
        spos[threadIdx.x] = ps;
        sw[threadIdx.x] = wv;
    }
    __syncthreads();
    if (threadIdx.x < kk) {
        const uint32_t p = spos[threadIdx.x];
        uint32_t rank = 0;
        for (uint32_t j = 0; j < kk; ++j) rank += spos[j] < p ? 1u : 0u;
        opos[rank] = p;
        ow[rank] = sw[threadIdx.x];
    }
    __syncthreads();
    const uint32_t d0 = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (d0 >= a.dm) return;
    const uint64_t nrows = (uint64_t)a.p + (uint64_t)a.shared * a.t;
    const _Float16 *o16 = reinterpret_cast<const _Float16 *>(a.ws + a.L.o);
    const float *oscale = reinterpret_cast<const float *>(a.ws + a.L.o + r9vx_moe_oscale_offset(nrows, a.dm));
    const uint32_t nblk = a.dm / 64, blk = d0 / 64;
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    r9vx_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t jb = 0; jb < kk; jb += 8) {
        h4 rows[8];
        float scs[8];
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j)
            if (jb + j < kk) {
                const uint64_t row = opos[jb + j];
                rows[j] = __builtin_nontemporal_load(reinterpret_cast<const h4 *>(o16 + row * a.dm + d0));
                scs[j] = oscale[row * nblk + blk];
            }
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j) {
            if (jb + j < kk) {
                const float w = ow[jb + j], sc = scs[j];
                acc.x = acc.x + w * ((float)rows[j].x * sc);
                acc.y = acc.y + w * ((float)rows[j].y * sc);
                acc.z = acc.z + w * ((float)rows[j].z * sc);
                acc.w = acc.w + w * ((float)rows[j].w * sc);
            }
        }
    }
    for (uint32_t s = 0; s < a.shared; ++s) {
        const uint64_t row = (uint64_t)a.p + s * a.t + t;
        const h4 v = *reinterpret_cast<const h4 *>(o16 + row * a.dm + d0);
        const float sc = oscale[row * nblk + blk];
        acc.x = acc.x + (float)v.x * sc;
        acc.y = acc.y + (float)v.y * sc;
        acc.z = acc.z + (float)v.z * sc;
        acc.w = acc.w + (float)v.w * sc;
    }
    __builtin_nontemporal_store(acc, reinterpret_cast<r9vx_f32x4 *>(a.y + (uint64_t)t * a.dm + d0));
}

/* ---------------------------------------------------------------- host side */

static uint32_t lpr_for(uint32_t k, uint32_t &nseg) {
    uint32_t cpr = k / 32, lpr = 64;
    while (lpr > 8 && cpr % lpr) lpr >>= 1;
    if (cpr < lpr) lpr = cpr;
    nseg = cpr / lpr;
    uint32_t l2 = 0;
    while ((1u << l2) < lpr) ++l2;
    return l2;
}

int r9vx_moe_sort_stage(const r9vx_moe_problem &p, const MoeLayout &L, hipStream_t s, bool *x16_done) {
    SortArgs a{p.ids, p.ws, L, p.t * p.k, p.e, p.k, p.t, p.shared};
    if (x16_done) *x16_done = false;
    if (a.p <= 1024) {
        hipLaunchKernelGGL(sort_small_kernel, dim3(1), dim3(1024), 0, s, a);
        return (int)hipGetLastError();
    }
    const uint32_t nchunk = (a.p + 255) / 256;
    a.nchunk = nchunk;
    /* x16_done: the activation rows go with the four kernels, 20 / 20 / 40
     * / 20 % of them (the one-workgroup finish kernel leaves the most CUs
     * idle), four rows per 256-thread workgroup, sixteen per 1024 */
    uint32_t xr[5] = {0, 0, 0, 0, 0};
    if (x16_done) {
        a.x = p.x;
        a.x16 = reinterpret_cast<_Float16 *>(p.ws + L.x16);
        a.xscale = reinterpret_cast<float *>(p.ws + L.xscale);
        a.dm = p.dm;
        a.xperm = r9vx_group_order(p.scheme_gu);
        constexpr uint32_t kCum[5] = {0, 20, 40, 80, 100};
        for (int i = 1; i <= 4; ++i) xr[i] = (uint32_t)((uint64_t)p.t * kCum[i] / 100);
        *x16_done = true;
    }
    auto xblocks = [&](int i, uint32_t rows_per_block) { return (xr[i + 1] - xr[i] + rows_per_block - 1) / rows_per_block; };
    hipLaunchKernelGGL(sort_count_kernel, dim3(nchunk + xblocks(0, 4)), dim3(256), 0, s, a, xr[0], xr[1]);
    hipLaunchKernelGGL(sort_scan_kernel, dim3((p.e + 3) / 4 + xblocks(1, 4)), dim3(256), 0, s, a, nchunk, xr[1], xr[2]);
    hipLaunchKernelGGL(sort_finish_kernel, dim3(1 + xblocks(2, 16)), dim3(1024), 0, s, a, nchunk, xr[2], xr[3]);
    hipLaunchKernelGGL(sort_place_kernel, dim3(nchunk + xblocks(3, 4)), dim3(256), 0, s, a, nchunk, xr[3], xr[4]);
    return (int)hipGetLastError();
}

int r9vx_moe_decode_stage(const r9vx_moe_problem &p, const MoeLayout &L, hipStream_t s) {
    FfnArgs f{};
    f.x = p.x;
    f.ids = p.ids;
    f.w_gu = p.w_gu;
    f.w_dn = p.w_dn;
    f.weights = p.weights;
    f.y = p.y;
    f.ws = p.ws;
    f.L = L;
    f.s_gu = p.s_gu;
    f.s_dn = p.s_dn;
    f.gu_row_bytes = r9vx_row_bytes(p.scheme_gu, p.dm);
    f.dn_row_bytes = r9vx_row_bytes(p.scheme_dn, p.dff);
    f.gu_srow = r9vx_row_scales(p.scheme_gu, p.dm);
    f.dn_srow = r9vx_row_scales(p.scheme_dn, p.dff);
    f.t = p.t;
    f.e = p.e;
    f.k = p.k;
    f.dm = p.dm;
    f.dff = p.dff;
    f.shared = p.shared;
    f.p = p.t * p.k;
    f.gu_lpr_log2 = lpr_for(p.dm, f.gu_nseg);
    f.dn_lpr_log2 = lpr_for(p.dff, f.dn_nseg);
    const uint32_t gu_rows = kDecPairs * (64u >> f.gu_lpr_log2), dn_rows = kDecDnRows * (64u >> f.dn_lpr_log2);
    f.gu_groups = (p.dff + gu_rows - 1) / gu_rows;
    f.dn_groups = (p.dm + dn_rows - 1) / dn_rows;
    /* one wave per upw units of (position, row group); a unit is nseg steps */
    const uint32_t npos = f.p + p.shared * p.t;
    auto upw_for = [](uint32_t groups, uint32_t nseg) {
        uint32_t upw = kDecSteps / nseg;
        if (upw < 1) upw = 1;
        return upw < groups ? upw : groups;
    };
    f.gu_upw = upw_for(f.gu_groups, f.gu_nseg);
    f.dn_upw = upw_for(f.dn_groups, f.dn_nseg);
    /* rows of one K segment take the pipelined kernels: the largest units
     * per wave <= kPipeUpw that divides the row groups per position, so a
     * wave's units lie in one position */
    auto pipe_upw = [](uint32_t groups, uint32_t most) {
        uint32_t u = most;
        while (groups % u) --u;
        return u;
    };
    const bool gu_pipe = f.gu_nseg == 1, dn_pipe = f.dn_nseg == 1;
    if (gu_pipe) f.gu_upw = pipe_upw(f.gu_groups, kGuPipeUpw);
    if (dn_pipe) f.dn_upw = pipe_upw(f.dn_groups, kDnPipeUpw);
    auto grid_for = [&](uint32_t groups, uint32_t upw) {
        const uint32_t units = npos * groups;
        const uint32_t waves = (units + upw - 1) / upw;
        return dim3((waves + kDecWaves - 1) / kDecWaves);
    };
    const dim3 block(kDecWaves * 64);
    const dim3 ggu = grid_for(f.gu_groups, f.gu_upw), gdn = grid_for(f.dn_groups, f.dn_upw);
#define R9VX_GU(S) (gu_pipe ? moe_gu_pipe_kernel<S> : moe_gu_kernel<S>)
#define R9VX_DN(S) (dn_pipe ? moe_down_pipe_kernel<S> : moe_down_kernel<S>)
    switch (p.scheme_gu) {
    case R9VX_SCHEME_IQ3_S: hipLaunchKernelGGL(R9VX_GU(R9VX_SCHEME_IQ3_S), ggu, block, 0, s, f); break;
    case R9VX_SCHEME_IQ4_XS: hipLaunchKernelGGL(R9VX_GU(R9VX_SCHEME_IQ4_XS), ggu, block, 0, s, f); break;
    case R9VX_SCHEME_Q8_0: hipLaunchKernelGGL(R9VX_GU(R9VX_SCHEME_Q8_0), ggu, block, 0, s, f); break;
    case R9VX_SCHEME_Q6_K: hipLaunchKernelGGL(R9VX_GU(R9VX_SCHEME_Q6_K), ggu, block, 0, s, f); break;
    default: hipLaunchKernelGGL(R9VX_GU(R9VX_SCHEME_Q4_K), ggu, block, 0, s, f); break;
    }
    switch (p.scheme_dn) {
    case R9VX_SCHEME_IQ3_S: hipLaunchKernelGGL(R9VX_DN(R9VX_SCHEME_IQ3_S), gdn, block, 0, s, f); break;
    case R9VX_SCHEME_IQ4_XS: hipLaunchKernelGGL(R9VX_DN(R9VX_SCHEME_IQ4_XS), gdn, block, 0, s, f); break;
    case R9VX_SCHEME_Q8_0: hipLaunchKernelGGL(R9VX_DN(R9VX_SCHEME_Q8_0), gdn, block, 0, s, f); break;
    case R9VX_SCHEME_Q6_K: hipLaunchKernelGGL(R9VX_DN(R9VX_SCHEME_Q6_K), gdn, block, 0, s, f); break;
    default: hipLaunchKernelGGL(R9VX_DN(R9VX_SCHEME_Q4_K), gdn, block, 0, s, f); break;
    }
#undef R9VX_GU
#undef R9VX_DN
    return (int)hipGetLastError();
}

int r9vx_moe_combine_stage(const r9vx_moe_problem &p, const MoeLayout &L, hipStream_t s) {
    MoeCombineArgs c{p.weights, p.ids, p.y, p.ws, L, p.t, p.k, p.dm, p.shared, p.t * p.k, p.e};
    dim3 grid((p.dm / 4 + 255) / 256, p.t);
    if (r9vx_moe_decode_form(p))
        hipLaunchKernelGGL(r9vx_moe_combine_kernel, grid, dim3(256), 0, s, c);
    else /* the grouped path's fp16 rows */
        hipLaunchKernelGGL(r9vx_moe_combine16_kernel, grid, dim3(256), 0, s, c);
    return (int)hipGetLastError();
}
