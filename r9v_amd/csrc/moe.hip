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
 *    act_mul.rs:86-99); o = h . Wd^T.  Decode (t <= 8) runs dequant-fused
 *    GEMVs over the active experts' rows (h kept in f32 between them); larger
 *    t runs the grouped MFMA GEMM of moe_gemm.hip.
 *  - Combine (:641-653): y[t] = sum over the token's pairs in ascending
 *    (expert, slot) order of w * o, f32, then the shared experts' outputs are
 *    added (the residual_add of crates/r9v-models/src/generic.rs:1458-1495).
 *  - Refusal before mutation (:440-465): ids >= E set R9VX_STATUS_BAD_EXPERT
 *    in the workspace status word and every kernel that writes y or
 *    intermediate rows returns without writing.
 */
#include "r9vx_expf.h"
#include "r9vx_gemv_core.h"
#include "r9vx_moe.h"

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

/* Work-list entry of one expert: (expert, first sorted position, pair count). */
__device__ __forceinline__ void put_work(const MoeLayout &L, uint8_t *ws, uint32_t idx, uint32_t e,
                                         uint32_t beg, uint32_t m) {
    r9vx_u32x4 *work = reinterpret_cast<r9vx_u32x4 *>(ws + L.work);
    work[idx] = r9vx_u32x4{e, beg, m, 0u};
}

/* ---------------------------------------------------------------- sort: small */

struct SortArgs {
    const uint32_t *ids;
    uint8_t *ws;
    MoeLayout L;
    uint32_t p, e, k, t, shared;
};

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
    if (tid == 0) offsets[a.e] = all;
    __syncthreads();
    if (valid) {
        uint32_t pos = offs[id] + rank;
        reinterpret_cast<uint32_t *>(a.ws + L.sorted)[pos] = tid;
        reinterpret_cast<uint32_t *>(a.ws + L.inv)[tid] = pos;
    }
    /* compact work list of active experts, ascending id, then shared experts */
    uint32_t act = (tid < a.e && tot > 0) ? 1u : 0u;
    uint32_t n_act;
    uint32_t idx = block_excl_scan(act, sh, n_act);
    if (act) put_work(L, a.ws, idx, tid, off, tot);
    if (tid < a.shared) put_work(L, a.ws, n_act + tid, a.e + tid, a.p + tid * a.t, a.t);
    if (tid == 0) {
        status[0] = bad_sh;
        status[2] = n_act + a.shared;
    }
}

/* ---------------------------------------------------------------- sort: large */

__global__ void sort_prep_kernel(uint8_t *ws, MoeLayout L) {
    uint32_t *status = reinterpret_cast<uint32_t *>(ws + L.status);
    status[0] = 0u; /* status bits */
    status[1] = 0u; /* finished-expert counter */
    status[2] = 0u; /* work items */
}

/* One 256-pair chunk per block: in-chunk ranks and per-expert chunk counts. */
__global__ __launch_bounds__(256) void sort_count_kernel(SortArgs a) {
    __shared__ uint16_t cnt[4][kMoeMaxE];
    const MoeLayout &L = a.L;
    uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    uint32_t chunk = blockIdx.x, nchunk = gridDim.x;
    for (uint32_t i = tid; i < 4 * kMoeMaxE; i += 256) (&cnt[0][0])[i] = 0;
    __syncthreads();
    uint32_t pair = chunk * 256 + tid;
    bool in = pair < a.p;
    uint32_t id = in ? a.ids[pair] : 0u;
    bool valid = in && id < a.e;
    if (in && !valid) atomicOr(reinterpret_cast<uint32_t *>(a.ws + L.status), R9VX_STATUS_BAD_EXPERT);
    uint64_t peers = match_peers(id, valid, id_bits(a.e));
    uint32_t rw = rank_below(peers, lane);
    if (valid && rw == 0) cnt[w][id] = (uint16_t)__popcll(peers);
    __syncthreads();
    if (valid) {
        uint32_t rank = rw;
        for (uint32_t i = 0; i < w; ++i) rank += cnt[i][id];
        reinterpret_cast<uint32_t *>(a.ws + L.rank)[pair] = rank;
    }
    uint32_t *cc = reinterpret_cast<uint32_t *>(a.ws + L.ccount);
    for (uint32_t e = tid; e < a.e; e += 256)
        cc[(uint64_t)e * nchunk + chunk] = (uint32_t)cnt[0][e] + cnt[1][e] + cnt[2][e] + cnt[3][e];
}

/* One wave per expert: exclusive scan of its chunk counts.  The last wave to
 * finish scans the expert totals into offsets and writes the work list. */
__global__ __launch_bounds__(256) void sort_scan_kernel(SortArgs a, uint32_t nchunk) {
    const MoeLayout &L = a.L;
    uint32_t lane = threadIdx.x & 63;
    uint32_t e = blockIdx.x * 4 + (threadIdx.x >> 6);
    uint32_t *status = reinterpret_cast<uint32_t *>(a.ws + L.status);
    uint32_t *counts = reinterpret_cast<uint32_t *>(a.ws + L.counts);
    if (e < a.e) {
        const uint32_t *cc = reinterpret_cast<const uint32_t *>(a.ws + L.ccount) + (uint64_t)e * nchunk;
        uint32_t *cb = reinterpret_cast<uint32_t *>(a.ws + L.cbase) + (uint64_t)e * nchunk;
        uint32_t carry = 0;
        for (uint32_t c0 = 0; c0 < nchunk; c0 += 64) {
            uint32_t c = c0 + lane;
            uint32_t v = c < nchunk ? cc[c] : 0u;
            uint32_t inc = wave_incl_scan(v, lane);
            if (c < nchunk) cb[c] = carry + inc - v;
            carry += __shfl(inc, 63, 64);
        }
        if (lane == 0) counts[e] = carry;
        __threadfence();
        uint32_t prev = 0;
        if (lane == 0) prev = atomicAdd(&status[1], 1u);
        prev = __shfl(prev, 0, 64);
        if (prev != a.e - 1) return;
        __threadfence();
        /* last expert finished: scan the totals (this wave only) */
        uint32_t *offsets = reinterpret_cast<uint32_t *>(a.ws + L.offsets);
        uint32_t base = 0, nact = 0;
        for (uint32_t e0 = 0; e0 < a.e; e0 += 64) {
            uint32_t ee = e0 + lane;
            uint32_t v = ee < a.e ? __hip_atomic_load(&counts[ee], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
            uint32_t inc = wave_incl_scan(v, lane);
            uint32_t act = v > 0 ? 1u : 0u;
            uint32_t ainc = wave_incl_scan(act, lane);
            if (ee < a.e) {
                offsets[ee] = base + inc - v;
                if (act) put_work(L, a.ws, nact + ainc - 1, ee, base + inc - v, v);
            }
            base += __shfl(inc, 63, 64);
            nact += __shfl(ainc, 63, 64);
        }
        if (lane == 0) offsets[a.e] = base;
        for (uint32_t s = lane; s < a.shared; s += 64) put_work(L, a.ws, nact + s, a.e + s, a.p + s * a.t, a.t);
        if (lane == 0) status[2] = nact + a.shared;
    }
}

__global__ __launch_bounds__(256) void sort_place_kernel(SortArgs a, uint32_t nchunk) {
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
    const uint8_t *w_gu;
    const uint8_t *w_dn;
    const float *weights;
    float *y;
    uint8_t *ws;
    MoeLayout L;
    uint64_t gu_row_bytes; /* bytes per gate/up weight row (Dm/256 blocks) */
    uint64_t dn_row_bytes; /* bytes per down weight row (Dff/256 blocks) */
    uint32_t t, e, k, dm, dff, shared, p;
    uint32_t gu_lpr_log2, gu_nseg;
    uint32_t dn_lpr_log2, dn_nseg;
};

/* Decode launch shape (compile-time tuning constants): activation rows per
 * pass, gate/up row pairs and down rows per lane group per wave, waves per
 * workgroup. */
#ifndef R9VX_DEC_MT
#define R9VX_DEC_MT 1
#endif
#ifndef R9VX_DEC_GU_PAIRS
#define R9VX_DEC_GU_PAIRS 1
#endif
#ifndef R9VX_DEC_DN_ROWS
#define R9VX_DEC_DN_ROWS 2
#endif
#ifndef R9VX_DEC_WAVES
#define R9VX_DEC_WAVES 2
#endif
constexpr int kDecPairs = R9VX_DEC_GU_PAIRS;
constexpr int kDecDnRows = R9VX_DEC_DN_ROWS;
constexpr int kDecWaves = R9VX_DEC_WAVES;

__device__ __forceinline__ bool refused(const FfnArgs &a) {
    return reinterpret_cast<const uint32_t *>(a.ws + a.L.status)[0] != 0u;
}

__device__ __forceinline__ uint32_t token_of(const FfnArgs &a, uint32_t expert, uint32_t pos) {
    if (expert >= a.e) return pos - (a.p + (expert - a.e) * a.t);
    return reinterpret_cast<const uint32_t *>(a.ws + a.L.sorted)[pos] / a.k;
}

/* gate/up GEMV + SwiGLU for one work item; block = 4 waves over Dff rows. */
template <int GU, int MT>
__global__ __launch_bounds__(kDecWaves * 64) void moe_gu_kernel(FfnArgs a) {
    constexpr int kPairs = kDecPairs;
    __shared__ uint32_t lut[256];
    __shared__ uint64_t etab[R9VX_EXP2F_N];
    const uint32_t *status = reinterpret_cast<const uint32_t *>(a.ws + a.L.status);
    if (status[0] != 0u || blockIdx.x >= status[2]) return;
    r9vx_exp2_fill(etab, threadIdx.x, blockDim.x); /* ordered by the LUT's barrier */
    r9vx_u32x4 wk = reinterpret_cast<const r9vx_u32x4 *>(a.ws + a.L.work)[blockIdx.x];
    const uint32_t expert = wk.x, beg = wk.y, cnt = wk.z;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t lpr = 1u << a.gu_lpr_log2, rpi = 64u >> a.gu_lpr_log2;
    const uint32_t lir = lane & (lpr - 1), slot = lane >> a.gu_lpr_log2;
    const uint32_t wave = blockIdx.y * kDecWaves + (threadIdx.x >> 6);
    const uint32_t r0 = wave * rpi * kPairs + slot;
    const uint8_t *wexp = a.w_gu + (uint64_t)expert * 2 * a.dff * a.gu_row_bytes;
    float *h = reinterpret_cast<float *>(a.ws + a.L.h);
    bool lut_ready = false;

    for (uint32_t t0 = 0; t0 < cnt; t0 += MT) {
        const int m = (int)(cnt - t0 < (uint32_t)MT ? cnt - t0 : (uint32_t)MT);
        const uint16_t *xrow[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            uint32_t tok = token_of(a, expert, beg + t0 + (t < m ? t : 0));
            xrow[t] = a.x + (uint64_t)tok * a.dm;
        }
        float ag[kPairs][MT], au[kPairs][MT];
#pragma unroll
        for (int r = 0; r < kPairs; ++r)
#pragma unroll
            for (int t = 0; t < MT; ++t) ag[r][t] = au[r][t] = 0.f;
        for (uint32_t seg = 0; seg < a.gu_nseg; ++seg) {
            uint32_t ci = seg * lpr + lir, klo, khi;
            chunk_k<GU>(ci, klo, khi);
            /* activations (L2-resident), then weights, then the table */
            XRaw<false> xr[MT];
#pragma unroll
            for (int t = 0; t < MT; ++t)
                if (t < m) load_x_raw<false>(xrow[t], klo, khi, xr[t]);
            r9vx_u32x4 qg[kPairs], qu[kPairs];
            Hdr hg[kPairs], hu[kPairs];
#pragma unroll
            for (int r = 0; r < kPairs; ++r) {
                uint32_t row = r0 + r * rpi;
                uint32_t rr = row < a.dff ? row : a.dff - 1;
                load_chunk<GU>(wexp + (uint64_t)rr * a.gu_row_bytes, ci, qg[r], hg[r]);
                load_chunk<GU>(wexp + (uint64_t)(a.dff + rr) * a.gu_row_bytes, ci, qu[r], hu[r]);
            }
            if (!lut_ready) { /* codebook and exp tables visible to every wave */
                if constexpr (GU == R9VX_SCHEME_IQ4_XS) init_iq4_lut(lut, threadIdx.x, blockDim.x);
                __syncthreads();
                lut_ready = true;
            }
            XChunk<GU, false> xc[MT];
#pragma unroll
            for (int t = 0; t < MT; ++t)
                if (t < m) arrange_x<GU, false>(xr[t], xc[t]);
#pragma unroll
            for (int r = 0; r < kPairs; ++r) {
                chunk_dot<GU, false, MT>(qg[r], hg[r], ci & 7, xc, ag[r], lut, m);
                chunk_dot<GU, false, MT>(qu[r], hu[r], ci & 7, xc, au[r], lut, m);
            }
        }
        /* g and u go through the same reduction, so each emitted slot
         * carries both halves of one (row, token) */
        constexpr int V = kPairs * MT;
        float gu[2][V];
#pragma unroll
        for (int r = 0; r < kPairs; ++r)
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                gu[0][r * MT + t] = ag[r][t];
                gu[1][r * MT + t] = au[r][t];
            }
        lane_reduce_w<V, 2>(gu, lane, a.gu_lpr_log2, [&](int idx, const float (&val)[2]) {
            const int r = idx / MT, t = idx % MT;
            const uint32_t row = r0 + r * rpi;
            if (t >= m || row >= a.dff) return;
            const float g = val[0];
            const float act = g / (1.0f + r9vx_expf_tab(-g, etab));
            h[(uint64_t)(beg + t0 + t) * a.dff + row] = act * val[1];
        });
    }
}

/* down GEMV for one work item: o[pos, d] = h[pos, :] . Wd[d, :]. */
template <int DN, int MT>
__global__ __launch_bounds__(kDecWaves * 64) void moe_down_kernel(FfnArgs a) {
    constexpr int kDnRows = kDecDnRows;
    __shared__ uint32_t lut[256];
    const uint32_t *status = reinterpret_cast<const uint32_t *>(a.ws + a.L.status);
    if (status[0] != 0u || blockIdx.x >= status[2]) return;
    r9vx_u32x4 wk = reinterpret_cast<const r9vx_u32x4 *>(a.ws + a.L.work)[blockIdx.x];
    const uint32_t expert = wk.x, beg = wk.y, cnt = wk.z;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t lpr = 1u << a.dn_lpr_log2, rpi = 64u >> a.dn_lpr_log2;
    const uint32_t lir = lane & (lpr - 1), slot = lane >> a.dn_lpr_log2;
    const uint32_t wave = blockIdx.y * kDecWaves + (threadIdx.x >> 6);
    const uint32_t r0 = wave * rpi * kDnRows + slot;
    const uint8_t *wexp = a.w_dn + (uint64_t)expert * a.dm * a.dn_row_bytes;
    const float *h = reinterpret_cast<const float *>(a.ws + a.L.h);
    float *o = reinterpret_cast<float *>(a.ws + a.L.o);
    bool lut_ready = false;

    for (uint32_t t0 = 0; t0 < cnt; t0 += MT) {
        const int m = (int)(cnt - t0 < (uint32_t)MT ? cnt - t0 : (uint32_t)MT);
        float acc[kDnRows][MT];
#pragma unroll
        for (int r = 0; r < kDnRows; ++r)
#pragma unroll
            for (int t = 0; t < MT; ++t) acc[r][t] = 0.f;
        for (uint32_t seg = 0; seg < a.dn_nseg; ++seg) {
            uint32_t ci = seg * lpr + lir, klo, khi;
            chunk_k<DN>(ci, klo, khi);
            XRaw<true> xr[MT];
#pragma unroll
            for (int t = 0; t < MT; ++t)
                if (t < m) load_x_raw<true>(h + (uint64_t)(beg + t0 + t) * a.dff, klo, khi, xr[t]);
            r9vx_u32x4 q[kDnRows];
            Hdr hd[kDnRows];
#pragma unroll
            for (int r = 0; r < kDnRows; ++r) {
                uint32_t row = r0 + r * rpi;
                uint32_t rr = row < a.dm ? row : a.dm - 1;
                load_chunk<DN>(wexp + (uint64_t)rr * a.dn_row_bytes, ci, q[r], hd[r]);
            }
            if constexpr (DN == R9VX_SCHEME_IQ4_XS) {
                if (!lut_ready) {
                    init_iq4_lut(lut, threadIdx.x, blockDim.x);
                    __syncthreads();
                    lut_ready = true;
                }
            }
            XChunk<DN, true> xc[MT];
#pragma unroll
            for (int t = 0; t < MT; ++t)
                if (t < m) arrange_x<DN, true>(xr[t], xc[t]);
#pragma unroll
            for (int r = 0; r < kDnRows; ++r) chunk_dot<DN, true, MT>(q[r], hd[r], ci & 7, xc, acc[r], lut, m);
        }
        constexpr int V = kDnRows * MT;
        float v[1][V];
#pragma unroll
        for (int r = 0; r < kDnRows; ++r)
#pragma unroll
            for (int t = 0; t < MT; ++t) v[0][r * MT + t] = acc[r][t];
        lane_reduce_w<V, 1>(v, lane, a.dn_lpr_log2, [&](int idx, const float (&val)[1]) {
            const int r = idx / MT, t = idx % MT;
            const uint32_t row = r0 + r * rpi;
            if (t >= m || row >= a.dm) return;
            o[(uint64_t)(beg + t0 + t) * a.dm + row] = val[0];
        });
    }
}

}  // namespace

/* ---------------------------------------------------------------- combine */

/* y[t, d] = sum over the token's pairs in ascending sorted position (=
 * ascending expert, then slot) of w * o, then + each shared expert's o.
 * The first K threads rank the token's K positions in LDS (positions are
 * distinct), so every thread then walks the same ordered list from LDS and
 * issues its K row loads before the ordered f32 sum. */
__global__ __launch_bounds__(256) void r9vx_moe_combine_kernel(MoeCombineArgs a) {
    __shared__ uint32_t spos[kMoeMaxK], opos[kMoeMaxK];
    __shared__ float sw[kMoeMaxK], ow[kMoeMaxK];
    const uint32_t *status = reinterpret_cast<const uint32_t *>(a.ws + a.L.status);
    if (status[0] != 0u) return;
    const uint32_t t = blockIdx.y;
    const uint32_t kk = a.k;
    const uint32_t *inv = reinterpret_cast<const uint32_t *>(a.ws + a.L.inv);
    if (threadIdx.x < kk) {
        spos[threadIdx.x] = inv[(uint64_t)t * kk + threadIdx.x];
        sw[threadIdx.x] = a.weights[(uint64_t)t * kk + threadIdx.x];
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
    const float *o = reinterpret_cast<const float *>(a.ws + a.L.o);
    r9vx_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    /* Eight rows in flight at a time; rows[] is indexed by constants only so
     * it stays in registers. */
    for (uint32_t jb = 0; jb < kk; jb += 8) {
        r9vx_f32x4 rows[8];
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j)
            if (jb + j < kk)
                rows[j] = *reinterpret_cast<const r9vx_f32x4 *>(o + (uint64_t)opos[jb + j] * a.dm + d0);
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j) {
            if (jb + j < kk) {
                const float w = ow[jb + j];
                acc.x = acc.x + w * rows[j].x;
                acc.y = acc.y + w * rows[j].y;
                acc.z = acc.z + w * rows[j].z;
                acc.w = acc.w + w * rows[j].w;
            }
        }
    }
    for (uint32_t s = 0; s < a.shared; ++s) {
        r9vx_f32x4 v = *reinterpret_cast<const r9vx_f32x4 *>(o + (uint64_t)(a.p + s * a.t + t) * a.dm + d0);
        acc.x = acc.x + v.x;
        acc.y = acc.y + v.y;
        acc.z = acc.z + v.z;
        acc.w = acc.w + v.w;
    }
    *reinterpret_cast<r9vx_f32x4 *>(a.y + (uint64_t)t * a.dm + d0) = acc;
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

int r9vx_moe_sort_stage(const r9vx_moe_problem &p, const MoeLayout &L, hipStream_t s) {
    SortArgs a{p.ids, p.ws, L, p.t * p.k, p.e, p.k, p.t, p.shared};
    if (a.p <= 1024) {
        hipLaunchKernelGGL(sort_small_kernel, dim3(1), dim3(1024), 0, s, a);
        return (int)hipGetLastError();
    }
    uint32_t nchunk = (a.p + 255) / 256;
    hipLaunchKernelGGL(sort_prep_kernel, dim3(1), dim3(1), 0, s, p.ws, L);
    hipLaunchKernelGGL(sort_count_kernel, dim3(nchunk), dim3(256), 0, s, a);
    hipLaunchKernelGGL(sort_scan_kernel, dim3((p.e + 3) / 4), dim3(256), 0, s, a, nchunk);
    hipLaunchKernelGGL(sort_place_kernel, dim3(nchunk), dim3(256), 0, s, a, nchunk);
    return (int)hipGetLastError();
}

template <int MT>
static void launch_decode_mt(const FfnArgs &f, uint32_t gu_scheme, uint32_t dn_scheme, uint32_t max_work,
                             hipStream_t s) {
    const uint32_t gu_rows_per_block = kDecWaves * (64u >> f.gu_lpr_log2) * kDecPairs;
    const uint32_t dn_rows_per_block = kDecWaves * (64u >> f.dn_lpr_log2) * kDecDnRows;
    dim3 ggu(max_work, (f.dff + gu_rows_per_block - 1) / gu_rows_per_block);
    dim3 gdn(max_work, (f.dm + dn_rows_per_block - 1) / dn_rows_per_block);
    if (gu_scheme == R9VX_SCHEME_IQ4_XS)
        hipLaunchKernelGGL((moe_gu_kernel<R9VX_SCHEME_IQ4_XS, MT>), ggu, dim3(kDecWaves * 64), 0, s, f);
    else
        hipLaunchKernelGGL((moe_gu_kernel<R9VX_SCHEME_Q4_K, MT>), ggu, dim3(kDecWaves * 64), 0, s, f);
    if (dn_scheme == R9VX_SCHEME_Q4_K)
        hipLaunchKernelGGL((moe_down_kernel<R9VX_SCHEME_Q4_K, MT>), gdn, dim3(kDecWaves * 64), 0, s, f);
    else
        hipLaunchKernelGGL((moe_down_kernel<R9VX_SCHEME_IQ4_XS, MT>), gdn, dim3(kDecWaves * 64), 0, s, f);
}

int r9vx_moe_decode_stage(const r9vx_moe_problem &p, const MoeLayout &L, hipStream_t s) {
    FfnArgs f{};
    f.x = p.x;
    f.w_gu = p.w_gu;
    f.w_dn = p.w_dn;
    f.weights = p.weights;
    f.y = p.y;
    f.ws = p.ws;
    f.L = L;
    f.gu_row_bytes = (uint64_t)(p.dm / 256) * (p.scheme_gu == R9VX_SCHEME_Q4_K ? R9VX_Q4K_BYTES : R9VX_IQ4XS_BYTES);
    f.dn_row_bytes = (uint64_t)(p.dff / 256) * (p.scheme_dn == R9VX_SCHEME_Q4_K ? R9VX_Q4K_BYTES : R9VX_IQ4XS_BYTES);
    f.t = p.t;
    f.e = p.e;
    f.k = p.k;
    f.dm = p.dm;
    f.dff = p.dff;
    f.shared = p.shared;
    f.p = p.t * p.k;
    f.gu_lpr_log2 = lpr_for(p.dm, f.gu_nseg);
    f.dn_lpr_log2 = lpr_for(p.dff, f.dn_nseg);
    uint32_t max_work = (f.p < p.e ? f.p : p.e) + p.shared;
    launch_decode_mt<R9VX_DEC_MT>(f, p.scheme_gu, p.scheme_dn, max_work, s);
    return (int)hipGetLastError();
}

int r9vx_moe_combine_stage(const r9vx_moe_problem &p, const MoeLayout &L, hipStream_t s) {
    MoeCombineArgs c{p.weights, p.y, p.ws, L, p.t, p.k, p.dm, p.shared, p.t * p.k};
    dim3 grid((p.dm / 4 + 255) / 256, p.t);
    hipLaunchKernelGGL(r9vx_moe_combine_kernel, grid, dim3(256), 0, s, c);
    return (int)hipGetLastError();
}
