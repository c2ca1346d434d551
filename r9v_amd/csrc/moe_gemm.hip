/*
 * moe_gemm.hip -- prefill MoE expert FFN as two grouped fp16-MFMA GEMMs over
 * the permuted (expert, token) rows.
 *
 * T0 meaning: crates/r9v-t0/src/moe_ffn.rs:527-639 (per expert: gather rows,
 * gate/up Branch-D GEMM, act_mul SiLU, down GEMM); the combine is moe.hip's.
 *
 *  tiles : each work item (expert with n pairs, or shared expert with t rows)
 *          becomes ceil(n / 128) row tiles; a one-workgroup scan lays them out.
 *  gate/up: a workgroup owns 128 permuted rows x 128 columns j of h; its
 *          B tile holds gate rows j and up rows Dff+j of the expert (256
 *          weight rows), so g and u of the same (row, j) land in the same lane
 *          and register: h = silu(g) * u is formed in registers (f32) and
 *          written with the row's running max|h|.  A rows are gathered from the
 *          fp16-scaled activations by the permutation (no permuted copy of x).
 *  down  : a workgroup owns 128 rows x 256 output columns; h rows are scaled
 *          by the power of two that brings max|h| below 2^15, rounded to fp16
 *          into LDS, and the scale is undone on the f32 accumulators.
 * Weight tiles are dequantized into LDS as fp16 exactly as in gemm.hip; LDS
 * is single-buffered (48 KiB) so two workgroups share a CU and one's MFMAs
 * overlap the other's dequantization.  Tiles past the scanned count exit.
 */
#include "r9vx_mma.h"
#include "r9vx_moe.h"

using namespace r9vx;

namespace {

constexpr uint32_t kBM = kMoeTileM; /* 128 rows per tile */

struct GroupedArgs {
    const _Float16 *x16;
    const float *xscale;
    const uint8_t *w_gu;
    const uint8_t *w_dn;
    uint8_t *ws;
    MoeLayout L;
    uint64_t gu_row_bytes, dn_row_bytes;
    uint32_t t, e, k, dm, dff, p, shared;
};

__device__ __forceinline__ const uint32_t *ws_u32(const GroupedArgs &a, uint64_t off) {
    return reinterpret_cast<const uint32_t *>(a.ws + off);
}

__device__ __forceinline__ uint32_t row_token(const GroupedArgs &a, uint32_t expert, uint32_t pos) {
    if (expert >= a.e) return pos - (a.p + (expert - a.e) * a.t);
    return ws_u32(a, a.L.sorted)[pos] / a.k;
}

/* One workgroup: scan the work items' tile counts into the tile list and
 * zero the per-row max|h| words. */
__global__ __launch_bounds__(1024) void build_tiles_kernel(GroupedArgs a) {
    __shared__ uint32_t sh[16];
    uint32_t *status = reinterpret_cast<uint32_t *>(a.ws + a.L.status);
    const uint32_t nwork = status[2];
    const r9vx_u32x4 *work = reinterpret_cast<const r9vx_u32x4 *>(a.ws + a.L.work);
    r9vx_u32x4 *tiles = reinterpret_cast<r9vx_u32x4 *>(a.ws + a.L.tiles);
    uint32_t base = 0;
    for (uint32_t w0 = 0; w0 < nwork; w0 += 1024) {
        uint32_t i = w0 + threadIdx.x;
        r9vx_u32x4 wk = i < nwork ? work[i] : r9vx_u32x4{0u, 0u, 0u, 0u};
        uint32_t nt = (wk.z + kBM - 1) / kBM;
        /* block exclusive scan of nt */
        uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
        uint32_t inc = nt;
        for (int off = 1; off < 64; off <<= 1) {
            uint32_t o = __shfl_up(inc, off, 64);
            if (lane >= (uint32_t)off) inc += o;
        }
        __syncthreads();
        if (lane == 63) sh[wv] = inc;
        __syncthreads();
        uint32_t pre = 0, tot = 0;
        for (uint32_t q = 0; q < 16; ++q) {
            if (q < wv) pre += sh[q];
            tot += sh[q];
        }
        uint32_t first = base + pre + inc - nt;
        for (uint32_t j = 0; j < nt; ++j) {
            uint32_t rows = wk.z - j * kBM < kBM ? wk.z - j * kBM : kBM;
            tiles[first + j] = r9vx_u32x4{wk.x, wk.y + j * kBM, rows, 0u};
        }
        base += tot;
        __syncthreads();
    }
    if (threadIdx.x == 0) status[3] = base;
    uint32_t *hmax = reinterpret_cast<uint32_t *>(a.ws + a.L.hmax);
    for (uint32_t i = threadIdx.x; i < a.p + a.shared * a.t; i += 1024) hmax[i] = 0u;
}

/* ---------------------------------------------------------------- gate/up */

constexpr int kNB = 1; /* single-buffered LDS: two workgroups share a CU */

template <int GU>
__global__ __launch_bounds__(256, 2) void moe_gu_mfma_kernel(GroupedArgs a) {
    using S = MmaShape<kBM, kNB>;
    __shared__ __attribute__((aligned(16))) uint8_t lds[S::kLds];
    __shared__ uint32_t rowmax[kBM];
    const uint32_t *status = ws_u32(a, a.L.status);
    const uint32_t ntile_n = a.dff / 128;
    const uint32_t tix = blockIdx.x / ntile_n, nt = blockIdx.x % ntile_n;
    if (status[0] != 0u || tix >= status[3]) return;
    const r9vx_u32x4 tile = reinterpret_cast<const r9vx_u32x4 *>(a.ws + a.L.tiles)[tix];
    const uint32_t expert = tile.x, pos0 = tile.y, rows = tile.z;
    const uint32_t j0 = nt * 128;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid < kBM) rowmax[tid] = 0u;

    AF16Rows<kBM> as;
    as.chunk = tid & 7;
    as.row0 = tid >> 3;
#pragma unroll
    for (int i = 0; i < kBM / 32; ++i) {
        uint32_t r = as.row0 + 32 * i;
        uint32_t tok = row_token(a, expert, pos0 + (r < rows ? r : 0));
        as.row[i] = a.x16 + (uint64_t)tok * a.dm + 8 * as.chunk;
    }
    /* B row t: wave w = t/64 takes gate rows j0+32w.. (t%64 < 32) and the
     * matching up rows, so acc[i][0] is g and acc[i][1] is u of the same j. */
    const uint32_t bw = tid >> 6, bh = (tid >> 5) & 1, bj = tid & 31;
    const uint32_t wr = (bh ? a.dff : 0u) + j0 + 32 * bw + bj;
    const uint8_t *wptr = a.w_gu + ((uint64_t)expert * 2 * a.dff + wr) * a.gu_row_bytes;
    r9vx_f32x16 acc[kBM / 32][2];
    mma_mainloop<GU, kBM, kNB>(lds, as, wptr, a.dm / kTileK, acc);

    float *h = reinterpret_cast<float *>(a.ws + a.L.h);
    const uint32_t col = j0 + 32 * wave + (lane & 31);
#pragma unroll
    for (int i = 0; i < kBM / 32; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t rl = acc_row(i, r, lane);
            if (rl >= rows) continue;
            const float sc = a.xscale[row_token(a, expert, pos0 + rl)];
            const float g = acc[i][0][r] * sc, u = acc[i][1][r] * sc;
            const float v = g / (1.0f + __expf(-g)) * u;
            h[(uint64_t)(pos0 + rl) * a.dff + col] = v;
            atomicMax(&rowmax[rl], __builtin_bit_cast(uint32_t, fabsf(v)));
        }
    }
    __syncthreads();
    if (tid < rows) atomicMax(reinterpret_cast<uint32_t *>(a.ws + a.L.hmax) + pos0 + tid, rowmax[tid]);
}

/* ---------------------------------------------------------------- down */

template <int DN>
__global__ __launch_bounds__(256, 2) void moe_dn_mfma_kernel(GroupedArgs a) {
    using S = MmaShape<kBM, kNB>;
    __shared__ __attribute__((aligned(16))) uint8_t lds[S::kLds];
    const uint32_t *status = ws_u32(a, a.L.status);
    const uint32_t ntile_n = a.dm / 256;
    const uint32_t tix = blockIdx.x / ntile_n, nt = blockIdx.x % ntile_n;
    if (status[0] != 0u || tix >= status[3]) return;
    const r9vx_u32x4 tile = reinterpret_cast<const r9vx_u32x4 *>(a.ws + a.L.tiles)[tix];
    const uint32_t expert = tile.x, pos0 = tile.y, rows = tile.z;
    const uint32_t n0 = nt * 256;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    AF32ScaledRows<kBM> as;
    as.chunk = tid & 7;
    as.row0 = tid >> 3;
    const float *hbase = reinterpret_cast<const float *>(a.ws + a.L.h);
    const uint32_t *hmax = ws_u32(a, a.L.hmax);
#pragma unroll
    for (int i = 0; i < kBM / 32; ++i) {
        uint32_t r = as.row0 + 32 * i;
        uint32_t pos = pos0 + (r < rows ? r : 0);
        as.row[i] = hbase + (uint64_t)pos * a.dff + 8 * as.chunk;
        as.inv[i] = ldexpf(1.0f, -row_shift(__builtin_bit_cast(float, hmax[pos])));
    }
    const uint8_t *wptr = a.w_dn + ((uint64_t)expert * a.dm + n0 + tid) * a.dn_row_bytes;
    r9vx_f32x16 acc[kBM / 32][2];
    mma_mainloop<DN, kBM, kNB>(lds, as, wptr, a.dff / kTileK, acc);

    float *o = reinterpret_cast<float *>(a.ws + a.L.o);
#pragma unroll
    for (int i = 0; i < kBM / 32; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t rl = acc_row(i, r, lane);
            if (rl >= rows) continue;
            const float sc = ldexpf(1.0f, row_shift(__builtin_bit_cast(float, hmax[pos0 + rl])));
#pragma unroll
            for (int j = 0; j < 2; ++j)
                o[(uint64_t)(pos0 + rl) * a.dm + n0 + acc_col(wave, j, lane)] = acc[i][j][r] * sc;
        }
    }
}

}  // namespace

int r9vx_moe_grouped_stage(const r9vx_moe_problem &p, const MoeLayout &L, hipStream_t s) {
    GroupedArgs a{};
    a.x16 = reinterpret_cast<const _Float16 *>(p.ws + L.x16);
    a.xscale = reinterpret_cast<const float *>(p.ws + L.xscale);
    a.w_gu = p.w_gu;
    a.w_dn = p.w_dn;
    a.ws = p.ws;
    a.L = L;
    a.gu_row_bytes = (uint64_t)(p.dm / 256) * (p.scheme_gu == R9VX_SCHEME_Q4_K ? R9VX_Q4K_BYTES : R9VX_IQ4XS_BYTES);
    a.dn_row_bytes = (uint64_t)(p.dff / 256) * (p.scheme_dn == R9VX_SCHEME_Q4_K ? R9VX_Q4K_BYTES : R9VX_IQ4XS_BYTES);
    a.t = p.t;
    a.e = p.e;
    a.k = p.k;
    a.dm = p.dm;
    a.dff = p.dff;
    a.p = p.t * p.k;
    a.shared = p.shared;
    int rc = r9vx_launch_x_to_f16(p.x, p.t, p.dm, reinterpret_cast<_Float16 *>(p.ws + L.x16),
                                  reinterpret_cast<float *>(p.ws + L.xscale), s);
    if (rc) return rc;
    hipLaunchKernelGGL(build_tiles_kernel, dim3(1), dim3(1024), 0, s, a);
    /* upper bound on row tiles: ceil(P/128) + one partial tile per work item */
    const uint32_t max_tiles = (a.p + kBM - 1) / kBM + (a.p < p.e ? a.p : p.e) + (p.shared ? p.shared * ((p.t + kBM - 1) / kBM) : 0);
    dim3 ggu(max_tiles * (p.dff / 128)), gdn(max_tiles * (p.dm / 256));
    if (p.scheme_gu == R9VX_SCHEME_IQ4_XS)
        hipLaunchKernelGGL(moe_gu_mfma_kernel<R9VX_SCHEME_IQ4_XS>, ggu, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(moe_gu_mfma_kernel<R9VX_SCHEME_Q4_K>, ggu, dim3(256), 0, s, a);
    if (p.scheme_dn == R9VX_SCHEME_Q4_K)
        hipLaunchKernelGGL(moe_dn_mfma_kernel<R9VX_SCHEME_Q4_K>, gdn, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(moe_dn_mfma_kernel<R9VX_SCHEME_IQ4_XS>, gdn, dim3(256), 0, s, a);
    return (int)hipGetLastError();
}
