/*
 * moe_gemm.hip -- prefill MoE expert FFN as two grouped fp16-MFMA GEMMs over
 * the permuted (expert, token) rows.
 *
 * T0 meaning: crates/r9v-t0/src/moe_ffn.rs:527-639 (per expert: gather rows,
 * gate/up Branch-D GEMM, act_mul SiLU, down GEMM); the combine is moe.hip's.
 *
 *  tiles : each expert with n pairs (or shared expert with t rows) is
 *          ceil(n / 256) row tiles, listed by the sort (moe.hip).
 *  gate/up: a workgroup owns 256 permuted rows x 128 columns j of h; its
 *          weight tile is gate rows j0.. and the matching up rows Dff+j0..,
 *          and a wave's two column tiles are a gate tile and its up tile, so
 *          g and u of the same (row, j) land in the same lane and register:
 *          h = silu(g) * u is formed in registers (f32).  A rows are gathered
 *          from the scaled fp16 activations by the permutation (no permuted
 *          copy of x).
 *  h16   : each h row scaled by the power of two that brings max|h| below
 *          2^15 and rounded to fp16, in the down weights' K group order.  The
 *          256-row gate/up writes it directly, each 128-column block at its
 *          own scale (max|block| below 2^15), and the 256-row down GEMM
 *          rescales its f32 accumulators by the exponent step at each block
 *          boundary (past kM3MaxBlk blocks h_fix_kernel first brings a row's
 *          blocks to the row's scale).
 *  down  : a workgroup owns 256 rows x 256 output columns of o; the scale is
 *          undone on the f32 accumulators.
 * Both GEMMs run the main loop of r9vx_mma3.h for every weight scheme
 * (weights decoded once per workgroup into LDS, 8 waves, one workgroup per
 * CU); a wave whose 128 rows
 * hold fewer than 4 row tiles of the tile runs only the MFMAs of those.
 * Tiles past the scanned count exit.
 */
#include "r9vx_mma3.h"
#include "r9vx_moe.h"

using namespace r9vx;

namespace {


struct GroupedArgs {
    const _Float16 *x16;
    _Float16 *h16;
    const float *xscale;
    const uint8_t *w_gu;
    const uint8_t *w_dn;
    const uint16_t *s_gu; /* split layout: f16 d rows of w_gu / w_dn (NULL otherwise) */
    const uint16_t *s_dn;
    uint8_t *ws;
    MoeLayout L;
    uint64_t gu_row_bytes, dn_row_bytes;
    uint32_t gu_srow, dn_srow; /* f16 d values per weight row */
    uint32_t t, e, k, dm, dff, p, shared;
    uint32_t h_order; /* K order of the h16 rows: the down scheme for the group orders, 0 natural */
};

__device__ __forceinline__ const uint32_t *ws_u32(const GroupedArgs &a, uint64_t off) {
    return reinterpret_cast<const uint32_t *>(a.ws + off);
}

/* Workgroup -> (row tile, column block), XCD-aware: the hardware deals
 * workgroups to the 8 XCDs round-robin, so XCD x's j-th workgroup takes row
 * tile 8 * (j / ncol) + x and column block j % ncol.  Every column block of a
 * row tile then runs on one XCD, whose L2 fetches the tile's activation rows
 * once instead of once per column block.  The grid is 8 * ncol * (row tiles
 * rounded up to 8). */
__device__ __forceinline__ void xcd_tile(uint32_t ncol, uint32_t &tix, uint32_t &nt) {
    const uint32_t b = blockIdx.x, x = b & 7u, j = b >> 3;
    tix = (j / ncol) * 8u + x;
    nt = j % ncol;
}

__device__ __forceinline__ uint32_t row_token(const GroupedArgs &a, uint32_t expert, uint32_t pos) {
    if (expert >= a.e) return pos - (a.p + (expert - a.e) * a.t);
    return ws_u32(a, a.L.sorted)[pos] / a.k;
}

/* ---------------------------------------------------------------- helpers */

/* 4-byte load into a register that a later main loop's counted wait
 * covers (it is issued before that loop's loads); the destination is tied
 * in and out, and the reader touches it after that wait. */
__device__ __forceinline__ void ld_ahead(uint32_t &d, const void *p) {
    asm volatile("global_load_dword %0, %1, off" : "+v"(d) : "v"(p) : "memory");
}

/* x of the lane that DPP control CTRL names (within a row of 16 lanes). */
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

/* The 4-element chunk (column / 4 within a 128-column block) that holds
 * elements i .. i + 3 (i = 0 or 4) of the group stored at position c (< 128)
 * of the block in an h16 row of order `order` (r9vx_x16.h order_pos's orders,
 * chosen at run time). */
__device__ __forceinline__ uint32_t h_chunk(uint32_t order, uint32_t c, uint32_t i) {
    if (order == R9VX_SCHEME_Q4_K) return order_pos<R9VX_SCHEME_Q4_K>(c, i) / 4;
    if (order == R9VX_SCHEME_IQ4_XS) return order_pos<R9VX_SCHEME_IQ4_XS>(c, i) / 4;
    if (order == R9VX_SCHEME_Q6_K) return order_pos<R9VX_SCHEME_Q6_K>(c, i) / 4;
    return order_pos<0>(c, i) / 4;
}

/* After the gate/up GEMM, for a down GEMM past kM3MaxBlk blocks (which then
 * undoes one power-of-two scale per h16 row): gives each row that scale.  The row's e is the
 * largest of its blocks' (hbe; row_shift is monotonic, so it is row_shift of
 * the row's max|h|) and goes to hexp.  Each block at a smaller e is
 * multiplied by 2^(e_block - e_row), a power of two below 1 -- exact unless
 * a value lands in fp16's subnormal range, where it is rounded a second
 * time -- and its hbe entry becomes e_row, so a second pass changes nothing.
 * Rows whose blocks share one e (every row below 2^15) are only read.  One
 * thread per row. */
__global__ __launch_bounds__(256) void h_fix_kernel(GroupedArgs a, uint32_t nrows) {
    const uint32_t row = blockIdx.x * 256 + threadIdx.x;
    if (row >= nrows) return;
    if (ws_u32(a, a.L.status)[0] != 0u) return;
    const uint32_t nb = a.dff / 128;
    int8_t *const be = reinterpret_cast<int8_t *>(a.ws + a.L.hbe) + (uint64_t)row * r9vx_moe_hbe_stride(a.dff);
    int er = be[0];
    for (uint32_t b = 1; b < nb; ++b) er = be[b] > er ? be[b] : er;
    reinterpret_cast<int32_t *>(a.ws + a.L.hexp)[row] = er;
    for (uint32_t b = 0; b < nb; ++b) {
        const int eb = be[b];
        if (eb == er) continue;
        const float f = ldexpf(1.0f, eb - er);
        r9vx_u32x4 *const blk = reinterpret_cast<r9vx_u32x4 *>(a.h16 + (uint64_t)row * a.dff + 128 * b);
        for (uint32_t c = 0; c < 16; ++c) {
            const r9vx_u32x4 v = blk[c];
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
            uint32_t o[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                o[j] = pack_h2((float)__builtin_bit_cast(_Float16, (uint16_t)(w[j] & 0xFFFFu)) * f,
                               (float)__builtin_bit_cast(_Float16, (uint16_t)(w[j] >> 16)) * f);
            blk[c] = r9vx_u32x4{o[0], o[1], o[2], o[3]};
        }
        be[b] = (int8_t)er;
    }
}

/* ---------------------------------------------------------------- 256-row tiles */

/* Gate/up on the r9vx_mma3.h loop: a workgroup owns a 256-row tile of one
 * expert and 128 columns j of h; its B tile is gate rows j0 .. j0+127 (B rows
 * 0..127) and up rows Dff+j0 .. (B rows 128..255), and wave w's two column
 * tiles are gate 32(w%4) and up 128 + 32(w%4), so g and u of one (row, j)
 * share a lane and register. */
template <int GU>
__global__ __launch_bounds__(512, 1) void moe_gu_m3_kernel(GroupedArgs a) {
    __shared__ __attribute__((aligned(16))) M3Lds sm;
    uint32_t *lut = sm.lut;
    __shared__ float rowsc[kMoeTileM3];
    const uint32_t *status = ws_u32(a, a.L.status);
    uint32_t tix, nt;
    xcd_tile(a.dff / 128, tix, nt);
    /* the status words and the tile entry in one round of loads (the entry
     * index clamped into the list's space; it is used only when tix is a
     * listed tile) */
    const uint32_t st0 = status[0], ntile = status[4];
    const r9vx_u32x4 tile =
        reinterpret_cast<const r9vx_u32x4 *>(a.ws + a.L.tiles3)[tix < a.L.max_tiles3 ? tix : a.L.max_tiles3 - 1];
    if (st0 != 0u || tix >= ntile) return;
    const uint32_t expert = tile.x, pos0 = tile.y, rows = tile.z;
    const uint32_t j0 = nt * 128;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    /* each row's activation scale, loaded now and put in LDS after the main
     * loop (the epilogue is its only reader) */
    const float rsc = tid < rows ? a.xscale[row_token(a, expert, pos0 + (tid < kMoeTileM3 ? tid : 0))] : 0.f;
    if constexpr (GU == R9VX_SCHEME_IQ4_XS) m3_init_iq4_lut(lut, tid, 512);
    if constexpr (GU == R9VX_SCHEME_IQ3_S) {
        __shared__ __attribute__((aligned(16))) uint32_t lut3[kM3Iq3Words];
        lut = lut3;
        m3_init_iq3s_lut(lut, tid, 512);
    }
    __syncthreads();

    const uint32_t wv = __builtin_amdgcn_readfirstlane(wave);
    uint32_t aoff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t r = dma_row(wv, i, lane);
        const uint32_t tok = row_token(a, expert, pos0 + (r < rows ? r : 0));
        aoff[i] = (tok * a.dm + 8 * dma_group(r, lane)) * 2u;
    }
    const uint32_t c = m3_brow(tid);
    const uint32_t wr = c < 128 ? j0 + c : a.dff + j0 + (c - 128);
    M3WRow w{m3_uniform(a.w_gu + (uint64_t)expert * 2 * a.dff * a.gu_row_bytes), wr * (uint32_t)a.gu_row_bytes};
    if constexpr (GU == R9VX_SCHEME_Q8_0 || GU == R9VX_SCHEME_Q6_K) { /* the split layout's d rows */
        w.sbase = m3_uniform(reinterpret_cast<const uint8_t *>(a.s_gu + (uint64_t)expert * 2 * a.dff * a.gu_srow));
        w.soff = wr * a.gu_srow * 2u;
    }
    const uint32_t rh = wv >> 2, cq = wv & 3;
    const uint32_t nr = m3_active_tiles(rows, 128 * rh);
    r9vx_f32x16 acc[4][2];
    m3_run<GU, true>(nr, rows <= 128, sm, a.x16, aoff, w, a.dm / kTileK, tid, wv, lut, 128 * rh, 32 * cq,
                     128 + 32 * cq, acc);
    if (tid < kMoeTileM3) rowsc[tid] = rsc;
    __syncthreads();

    /* The tiles are transposed (m3_run<.., true>): lane l holds row 128 rh +
     * 32 t + (l & 31) and, in acc[t][0][r] / acc[t][1][r], the gate and up
     * values of h column j0 + 32 cq + 8 (r >> 2) + 4 (l >> 5) + (r & 3): four
     * consecutive columns per r >> 2.  The 256 x 128 f32 h tile is staged in
     * LDS (row R's 16-byte chunk c at chunk c ^ (R & 31)). */
    uint8_t *const ot = m3_out_tile(sm);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        if ((uint32_t)t >= nr) break;
        const uint32_t rl = 128 * rh + 32 * t + (lane & 31);
        const float sc = rowsc[rl];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            r9vx_f32x4 v;
            v.x = swiglu_fast(acc[t][0][4 * g + 0] * sc, acc[t][1][4 * g + 0] * sc);
            v.y = swiglu_fast(acc[t][0][4 * g + 1] * sc, acc[t][1][4 * g + 1] * sc);
            v.z = swiglu_fast(acc[t][0][4 * g + 2] * sc, acc[t][1][4 * g + 2] * sc);
            v.w = swiglu_fast(acc[t][0][4 * g + 3] * sc, acc[t][1][4 * g + 3] * sc);
            const uint32_t chunk = (8u * cq + 2u * g + (lane >> 5)) ^ (rl & 31u);
            *reinterpret_cast<r9vx_f32x4 *>(ot + rl * 512u + 16u * chunk) = v;
        }
    }
    __syncthreads();
    /* h leaves as fp16 (h16) in the down weights' K order, each (row, 128-
     * column block) scaled by 2^-row_shift(the block's max|h|), with that max
     * (its e) beside it (hbe), which the 256-row down GEMM undoes block by block
     * (h_fix_kernel gives each row one scale for the other down kernels).  16 lanes
     * take a row: lane g writes granule g & 7 of the block's 64-column step
     * g >> 3, whose elements 0-3 and 4-7 are two 16-byte chunks of the staged
     * f32 row. */
    const uint32_t g = lane & 15, hs = g >> 3, hq = g & 7;
    const uint32_t c_lo = h_chunk(a.h_order, 64 * hs + 8 * hq, 0), c_hi = h_chunk(a.h_order, 64 * hs + 8 * hq, 4);
    int8_t *const hbe = reinterpret_cast<int8_t *>(a.ws + a.L.hbe);
    const uint32_t hstride = r9vx_moe_hbe_stride(a.dff);
    /* every row of the stage is converted (rows past the tile's hold stale
     * values and are not stored), so the 16 lanes of a row reduce by DPP
     * with the whole row active */
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
        const uint32_t R = 32 * i + 4 * wv + (lane >> 4);
        const r9vx_f32x4 lo = *reinterpret_cast<const r9vx_f32x4 *>(ot + R * 512u + 16u * (c_lo ^ (R & 31u)));
        const r9vx_f32x4 hi = *reinterpret_cast<const r9vx_f32x4 *>(ot + R * 512u + 16u * (c_hi ^ (R & 31u)));
        float mx = fmaxf(fmaxf(fmaxf(fabsf(lo.x), fabsf(lo.y)), fmaxf(fabsf(lo.z), fabsf(lo.w))),
                         fmaxf(fmaxf(fabsf(hi.x), fabsf(hi.y)), fmaxf(fabsf(hi.z), fabsf(hi.w))));
        mx = fmaxf(mx, dpp_f32<0xB1>(mx));  /* quad_perm 1,0,3,2 */
        mx = fmaxf(mx, dpp_f32<0x4E>(mx));  /* quad_perm 2,3,0,1 */
        mx = fmaxf(mx, dpp_f32<0x141>(mx)); /* row_half_mirror: l <-> 7 - l */
        mx = fmaxf(mx, dpp_f32<0x140>(mx)); /* row_mirror: l <-> 15 - l */
        const int e = row_shift(mx);
        const float inv = ldexpf(1.0f, -e);
        if (R < rows) {
            *reinterpret_cast<r9vx_u32x4 *>(a.h16 + (uint64_t)(pos0 + R) * a.dff + j0 + 64 * hs + 8 * hq) =
                r9vx_u32x4{pack_h2(lo.x * inv, lo.y * inv), pack_h2(lo.z * inv, lo.w * inv),
                           pack_h2(hi.x * inv, hi.y * inv), pack_h2(hi.z * inv, hi.w * inv)};
            if (g == 0) hbe[(uint64_t)(pos0 + R) * hstride + nt] = (int8_t)e;
        }
    }
}

/* Down on the r9vx_mma3.h loop: 256 rows x 256 output columns per
 * workgroup; wave w's column tiles are 64(w%4) and 64(w%4) + 32. */
template <int DN, int PASSES>
__global__ __launch_bounds__(512, 1) void moe_dn_m3_kernel(GroupedArgs a) {
    __shared__ __attribute__((aligned(16))) M3Lds sm;
    uint32_t *lut = sm.lut;
    __shared__ float rowsc[kMoeTileM3]; /* 2^e that undoes each h row's last block's fp16 scale */
    __shared__ uint32_t bst[kM3MaxBlk * 64]; /* the rows' exponent steps per 128-K block (m3_bsd) */
    const uint32_t *status = ws_u32(a, a.L.status);
    uint32_t tix, nt;
    xcd_tile(a.dm / 256 / PASSES, tix, nt);
    const uint32_t st0 = status[0], ntile = status[4]; /* one round of loads, as in gate/up */
    const r9vx_u32x4 tile =
        reinterpret_cast<const r9vx_u32x4 *>(a.ws + a.L.tiles3)[tix < a.L.max_tiles3 ? tix : a.L.max_tiles3 - 1];
    if (st0 != 0u || tix >= ntile) return;
    const uint32_t expert = tile.x, pos0 = tile.y, rows = tile.z;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    /* h16 row r's 128-column block b is at scale 2^-e(b) (hbe).  Thread
     * r < 256 loads its row's exponents now (ahead of the main loop's loads,
     * which the loop's prologue waits for first) and then puts the steps
     * e(b - 1) - e(b) into bst (byte (r >> 5) & 3 of word 64 b + 32 (r >> 7)
     * + (r & 31); block 0's are 0) and 2^e(last) into rowsc.  Past
     * kM3MaxBlk blocks h_fix_kernel has given each row one scale: the
     * steps are 0 and the thread loads the row's e (hexp) instead. */
    const uint32_t nb = a.dff / 128;
    const bool ahead = nb <= kM3MaxBlk;
    uint32_t be0 = 0u, be1 = 0u;
    if (tid < kMoeTileM3) {
        const uint64_t row = pos0 + (tid < rows ? tid : 0);
        if (ahead) {
            const uint8_t *const berow = a.ws + a.L.hbe + row * r9vx_moe_hbe_stride(a.dff);
            ld_ahead(be0, berow);
            if (nb > 4) ld_ahead(be1, berow + 4);
        } else {
            ld_ahead(be0, a.ws + a.L.hexp + 4 * row);
        }
    }
    auto fill_steps = [&]() {
        if (tid >= kMoeTileM3) return;
        asm volatile("" : "+v"(be0), "+v"(be1));
        uint8_t *const tb = reinterpret_cast<uint8_t *>(bst) + 4 * (32 * (tid >> 7) + (tid & 31)) + ((tid >> 5) & 3);
        int eprev = 0;
        if (ahead) {
#pragma unroll
            for (uint32_t b = 0; b < kM3MaxBlk; ++b) {
                if (b >= nb) break;
                const int e = tid < rows ? (int)(int8_t)(((b < 4 ? be0 : be1) >> (8 * (b & 3))) & 0xFFu) : 0;
                tb[256 * b] = (uint8_t)(b == 0 ? 0 : eprev - e);
                eprev = e;
            }
        } else {
#pragma unroll
            for (uint32_t b = 0; b < kM3MaxBlk; ++b) tb[256 * b] = 0;
            eprev = tid < rows ? (int)be0 : 0;
        }
        rowsc[tid] = tid < rows ? ldexpf(1.0f, eprev) : 0.f;
    };
    if constexpr (DN == R9VX_SCHEME_IQ4_XS) m3_init_iq4_lut(lut, tid, 512);
    if constexpr (DN == R9VX_SCHEME_IQ3_S) {
        __shared__ __attribute__((aligned(16))) uint32_t lut3[kM3Iq3Words];
        lut = lut3;
        m3_init_iq3s_lut(lut, tid, 512);
    }
    __syncthreads();

    const uint32_t wv = __builtin_amdgcn_readfirstlane(wave);
    uint32_t aoff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t r = dma_row(wv, i, lane);
        aoff[i] = ((pos0 + (r < rows ? r : 0)) * a.dff + 8 * dma_group(r, lane)) * 2u;
    }
    const uint32_t rh = wv >> 2, cq = wv & 3;
    const uint32_t nr = m3_active_tiles(rows, 128 * rh);
    /* one 256-column block of the output per pass.  With PASSES = 2 the
     * workgroup's entry, its exponent steps and the h rows' copies (then in
     * L2) serve two blocks, and for tiles of more than 128 rows the second
     * block's weight payload loads are issued before the first block's
     * epilogue, so that their latency passes under it. */
    auto weights = [&](uint32_t n0) {
        M3WRow w{m3_uniform(a.w_dn + ((uint64_t)expert * a.dm + n0) * a.dn_row_bytes),
                 m3_brow(tid) * (uint32_t)a.dn_row_bytes};
        if constexpr (DN == R9VX_SCHEME_Q8_0 || DN == R9VX_SCHEME_Q6_K) {
            w.sbase = m3_uniform(reinterpret_cast<const uint8_t *>(a.s_dn + ((uint64_t)expert * a.dm + n0) * a.dn_srow));
            w.soff = m3_brow(tid) * a.dn_srow * 2u;
        }
        return w;
    };
    const uint32_t nk = a.dff / kTileK;
    auto epilogue = [&](uint32_t n0, r9vx_f32x16 (&acc)[4][2]) {
        /* The tiles are transposed (m3_run<.., true>): lane l holds h row
         * 128 rh + 32 t + (l & 31) and output columns n0 + 64 cq + 32 j +
         * 8 (r >> 2) + 4 (l >> 5) + (r & 3).  o rows are stored as fp16 scaled by
         * a power of two per (row, 64-column block), the block being this wave's
         * two column tiles: its max is this lane's 32 values and lane l ^ 32's.
         * The scale puts the block max in [2^14, 2^15); its inverse is stored
         * beside the rows for the combine.  The fp16 tile is staged in LDS (row
         * R's 8-byte chunk c at chunk c ^ (R & 31): the 32 rows one write
         * instruction covers hit distinct banks), then each row leaves as 32
         * lanes x 16 contiguous bytes. */
        const uint64_t nrows_all = (uint64_t)a.p + (uint64_t)a.shared * a.t;
        _Float16 *o16 = reinterpret_cast<_Float16 *>(a.ws + a.L.o);
        float *oscale = reinterpret_cast<float *>(a.ws + a.L.o + r9vx_moe_oscale_offset(nrows_all, a.dm));
        const uint32_t blk = (n0 + 64 * cq) / 64, nblk = a.dm / 64;
        uint8_t *const ot = m3_out_tile(sm);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            if ((uint32_t)t >= nr) break;
            const uint32_t rl = 128 * rh + 32 * t + (lane & 31);
            const float sc = rl < rows ? rowsc[rl] : 0.f;
            float m = 0.f;
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) m = fmaxf(m, fabsf(acc[t][j][r]));
            m *= sc; /* exact: sc is a power of two */
            m = fmaxf(m, __shfl_xor(m, 32, 64));
            int e = 0;
            (void)frexpf(m, &e); /* m = f 2^e, f in [0.5, 1) */
            const float f = ldexpf(sc, 15 - e); /* a power of two: acc * f = (acc * sc) 2^(15 - e) exactly */
            uint8_t *const orow = ot + rl * 512u;
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const uint32_t chunk = (16u * cq + 8u * j + 2u * g + (lane >> 5)) ^ (rl & 31u);
                    *reinterpret_cast<r9vx_u32x2 *>(orow + 8u * chunk) =
                        r9vx_u32x2{pack_h2h((_Float16)(acc[t][j][4 * g] * f), (_Float16)(acc[t][j][4 * g + 1] * f)),
                                   pack_h2h((_Float16)(acc[t][j][4 * g + 2] * f), (_Float16)(acc[t][j][4 * g + 3] * f))};
                }
            if (lane < 32 && rl < rows) oscale[(uint64_t)(pos0 + rl) * nblk + blk] = ldexpf(1.0f, e - 15);
        }
        __syncthreads();
        const uint32_t q = lane & 31;
#pragma unroll 4
        for (uint32_t i = 0; i < 16; ++i) {
            const uint32_t R = 16 * i + 2 * wv + (lane >> 5);
            if (R >= rows) break; /* rows grow with i */
            const uint32_t s = R & 31u;
            r9vx_u32x4 v = *reinterpret_cast<const r9vx_u32x4 *>(ot + R * 512u + 16u * (q ^ (s >> 1)));
            if (s & 1u) v = r9vx_u32x4{v.z, v.w, v.x, v.y}; /* the granule's halves were swapped */
            *reinterpret_cast<r9vx_u32x4 *>(o16 + (uint64_t)(pos0 + R) * a.dm + n0 + 8 * q) = v;
        }
    };
    const uint32_t n0a = nt * PASSES * 256;
    r9vx_f32x16 acc[4][2];
    m3_run<DN, true, true>(nr, rows <= 128, sm, a.h16, aoff, weights(n0a), nk, tid, wv, lut, 128 * rh, 64 * cq,
                           64 * cq + 32, acc, bst, fill_steps);
    if constexpr (PASSES == 1) {
        __syncthreads();
        epilogue(n0a, acc);
    } else {
        const M3WRow wb = weights(n0a + 256);
        r9vx_u32x4 pay[4], hnext;
        m3_issue_head<DN>(wb, tid, pay, hnext);
        __syncthreads();
        epilogue(n0a, acc);
        __syncthreads(); /* the staged tile is read before the next block's copies */
        /* P0 and H0 have landed (and the epilogue's stores are done) before the
         * loop takes their registers: its entry may copy them */
        wait_vm<0>();
        touch_pay(pay[0]);
        touch_pay(hnext);
        m3_run_pre<DN, true, true>(nr, sm, a.h16, aoff, wb, nk, tid, wv, lut, 128 * rh, 64 * cq, 64 * cq + 32, acc, bst,
                                   pay, hnext);
        __syncthreads();
        epilogue(n0a + 256, acc);
    }
}

}  // namespace

static GroupedArgs grouped_args(const r9vx_moe_problem &p, const MoeLayout &L) {
    GroupedArgs a{};
    a.x16 = reinterpret_cast<const _Float16 *>(p.ws + L.x16);
    a.h16 = reinterpret_cast<_Float16 *>(p.ws + L.h16);
    a.xscale = reinterpret_cast<const float *>(p.ws + L.xscale);
    a.w_gu = p.w_gu;
    a.w_dn = p.w_dn;
    a.s_gu = p.s_gu;
    a.s_dn = p.s_dn;
    a.ws = p.ws;
    a.L = L;
    a.gu_row_bytes = r9vx_row_bytes(p.scheme_gu, p.dm);
    a.dn_row_bytes = r9vx_row_bytes(p.scheme_dn, p.dff);
    a.gu_srow = r9vx_row_scales(p.scheme_gu, p.dm);
    a.dn_srow = r9vx_row_scales(p.scheme_dn, p.dff);
    a.t = p.t;
    a.e = p.e;
    a.k = p.k;
    a.dm = p.dm;
    a.dff = p.dff;
    a.p = p.t * p.k;
    a.shared = p.shared;
    a.h_order = r9vx_group_order(p.scheme_dn);
    return a;
}


int r9vx_moe_grouped_stage(const r9vx_moe_problem &p, const MoeLayout &L, hipStream_t s, bool x16_done) {
    return r9vx_moe_grouped_part(p, L, 0, s, x16_done);
}

/* part 0: the whole grouped stage; 1: the gate/up GEMM only; 2: the down
 * GEMM only (1 and 2 on a workspace the whole stage has filled). */
int r9vx_moe_grouped_part(const r9vx_moe_problem &p, const MoeLayout &L, uint32_t part, hipStream_t s,
                          bool x16_done) {
    GroupedArgs a = grouped_args(p, L);
    if (part == 0 && !x16_done) {
        int rc = r9vx_launch_x_to_f16(p.x, p.t, p.dm, reinterpret_cast<_Float16 *>(p.ws + L.x16),
                                      reinterpret_cast<float *>(p.ws + L.xscale), r9vx_group_order(p.scheme_gu), s);
        if (rc) return rc;
    }
    /* upper bound on row tiles: ceil(P/TM) + one partial tile per work item */
    const uint32_t max_tiles3 = (a.p + kMoeTileM3 - 1) / kMoeTileM3 + (a.p < p.e ? a.p : p.e) +
                                (p.shared ? p.shared * ((p.t + kMoeTileM3 - 1) / kMoeTileM3) : 0);
    const uint32_t tiles3_8 = (max_tiles3 + 7) / 8 * 8; /* xcd_tile's grids */
    const dim3 ggu3(tiles3_8 * (p.dff / 128)), gdn3(tiles3_8 * (p.dm / 256));
    if (part == 0 || part == 1) {
        switch (p.scheme_gu) {
        case R9VX_SCHEME_IQ4_XS: hipLaunchKernelGGL(moe_gu_m3_kernel<R9VX_SCHEME_IQ4_XS>, ggu3, dim3(512), 0, s, a); break;
        case R9VX_SCHEME_Q4_K: hipLaunchKernelGGL(moe_gu_m3_kernel<R9VX_SCHEME_Q4_K>, ggu3, dim3(512), 0, s, a); break;
        case R9VX_SCHEME_Q8_0: hipLaunchKernelGGL(moe_gu_m3_kernel<R9VX_SCHEME_Q8_0>, ggu3, dim3(512), 0, s, a); break;
        case R9VX_SCHEME_Q6_K: hipLaunchKernelGGL(moe_gu_m3_kernel<R9VX_SCHEME_Q6_K>, ggu3, dim3(512), 0, s, a); break;
        default: hipLaunchKernelGGL(moe_gu_m3_kernel<R9VX_SCHEME_IQ3_S>, ggu3, dim3(512), 0, s, a); break;
        }
    }
    const uint32_t nrows = a.p + p.shared * p.t;
    /* the gate/up GEMM writes h16 at a scale per 128-column block, which the
     * down GEMM takes as it is up to kM3MaxBlk blocks; past that every row
     * is brought to one scale first */
    if (p.dff / 128 > kM3MaxBlk && (part == 0 || part == 1))
        hipLaunchKernelGGL(h_fix_kernel, dim3((nrows + 255) / 256), dim3(256), 0, s, a, nrows);
    if (part == 0 || part == 2) {
        /* the 256-row Q4_K down GEMM takes two column blocks per workgroup when Dm / 256 is even */
        const bool two = (p.dm / 256) % 2 == 0;
        const dim3 gdn3_2(tiles3_8 * (p.dm / 512));
        switch (p.scheme_dn) {
        case R9VX_SCHEME_Q4_K:
            if (two)
                hipLaunchKernelGGL((moe_dn_m3_kernel<R9VX_SCHEME_Q4_K, 2>), gdn3_2, dim3(512), 0, s, a);
            else
                hipLaunchKernelGGL((moe_dn_m3_kernel<R9VX_SCHEME_Q4_K, 1>), gdn3, dim3(512), 0, s, a);
            break;
        case R9VX_SCHEME_IQ4_XS: /* (its codebook table leaves no registers for the two-block form) */
            hipLaunchKernelGGL((moe_dn_m3_kernel<R9VX_SCHEME_IQ4_XS, 1>), gdn3, dim3(512), 0, s, a);
            break;
        case R9VX_SCHEME_Q8_0: hipLaunchKernelGGL((moe_dn_m3_kernel<R9VX_SCHEME_Q8_0, 1>), gdn3, dim3(512), 0, s, a); break;
        case R9VX_SCHEME_Q6_K: hipLaunchKernelGGL((moe_dn_m3_kernel<R9VX_SCHEME_Q6_K, 1>), gdn3, dim3(512), 0, s, a); break;
        default: hipLaunchKernelGGL((moe_dn_m3_kernel<R9VX_SCHEME_IQ3_S, 1>), gdn3, dim3(512), 0, s, a); break;
        }
    }
    return (int)hipGetLastError();
}
