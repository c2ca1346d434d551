/*
 * gemm.hip -- prefill dequant-GEMM on MFMA: y[m, n] = sum_k x[m, k] * w[n, k]
 * for bf16 activations (variants with m_bucket > 8) and GGUF Q4_K / IQ4_XS
 * weights (wire blocks), Q8_0 / Q6_K weights (split layout) and IQ3_S
 * weights (112-byte repacked blocks).
 *
 * T0 meaning: crates/r9v-t0/src/matmul.rs:1940-2414 (Branch D), output cast
 * crates/r9v-t0/src/dtype.rs:102-111 (bf16 RNE); epilogue matmul.rs:2421-2446.
 *
 * Two launches:
 *  1. x_to_f16: one wave per activation row finds max|x|, picks the
 *     power-of-two scale 2^e that keeps the row below 2^15 (e = 0 for any
 *     ordinary activation) and writes the row as fp16 plus the scale, in the
 *     weight scheme's K order.  bf16 values are exact in fp16 inside that
 *     range.
 *  2. gemm3: tiles of up to 256 rows x 256 weight columns on the
 *     r9vx_mma3.h loop (each weight tile decoded once into LDS while the
 *     MFMAs of the previous K step run), the rows of each weight block cut
 *     into chunks sized so that the launch fills whole rounds of the CUs
 *     (plan_chunks); one kernel for every scheme and every n.
 */
#include "r9vx_mma3.h"

using namespace r9vx;

namespace {

/* gemm3's row chunks: blocks [b0, b0 + nb) of 256 weight rows x chunk
 * indices [c0, c0 + nc), nb * nc workgroups, block-fastest. */
struct ChunkGroup {
    uint32_t b0, nb, c0, nc;
};

struct GemmArgs {
    const _Float16 *x16;
    const float *scale;
    const uint8_t *w;
    const uint16_t *ws; /* Q8_0 / Q6_K split layout: f16 d per block */
    const float *bias;
    const float *residual;
    void *y;
    uint64_t w_row_stride;
    uint32_t m, n, k;
    uint32_t y_bf16, epilogue;
    uint32_t ws_row; /* d values per weight row */
    /* gemm3: the 32-row tiles of the m rows (rt of them) are cut, per weight
     * block, into nlo + 1 chunks for blocks < r0 and nlo chunks for the
     * others, as evenly as whole row tiles allow; grp lists the chunks
     * largest first, or with band set (every block nlo chunks, a multiple
     * of 8 in all) XCD x takes the x-th eighth of the (block, chunk) list,
     * a block's chunks consecutively */
    uint32_t rt, nlo, r0, band;
    ChunkGroup grp[4];
};

/* PERM = 0: natural order; R9VX_SCHEME_Q4_K / R9VX_SCHEME_IQ4_XS: each 64-column
 * step stored in that scheme's group order (r9vx_x16.h). */
template <int PERM>
__global__ __launch_bounds__(256) void x_to_f16_kernel(const uint16_t *__restrict__ x, uint32_t m, uint32_t k,
                                                       _Float16 *__restrict__ x16, float *__restrict__ scale) {
    /* one wave per row, four rows per workgroup: no barrier */
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= m) return;
    x16_row<PERM>(x, k, x16, scale, row, threadIdx.x & 63);
}

/* Tiles of up to 256 rows x 256 columns on the r9vx_mma3.h loop (the grouped
 * MoE GEMMs' core): the weight tile is decoded once per workgroup into LDS,
 * every wave reads its B fragments from there, and the accumulators are the
 * transposed tile, so lane l holds output row 128 rh + 32 t + (l & 31) and
 * columns 64 cq + 32 j + 8 (r >> 2) + 4 (l >> 5) + (r & 3) of acc[t][j][r].
 * A workgroup takes the chunk of rows plan_chunks gave its index.  Every n:
 * in a ragged last weight block the threads of rows past n decode row n - 1
 * again and the epilogue stores no column past n.  The launcher runs a
 * bucket as row launches of m k < 2^31 each (the A copy offsets are
 * 32-bit). */
template <int SCHEME>
__global__ __launch_bounds__(512, 1) void gemm3_kernel(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) M3Lds sm;
    __shared__ float rowsc[kM3Rows];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t wg = blockIdx.x, blk = 0, ch = 0;
    if (a.band) {
        const uint32_t t = (wg % 8u) * (gridDim.x / 8u) + wg / 8u;
        blk = t / a.nlo;
        ch = t % a.nlo;
    } else {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t cnt = a.grp[g].nb * a.grp[g].nc;
            if (wg < cnt) {
                blk = a.grp[g].b0 + wg % a.grp[g].nb;
                ch = a.grp[g].c0 + wg / a.grp[g].nb;
                break;
            }
            wg -= cnt;
        }
    }
    /* chunk ch of the block's nch: row tiles ch * per + min(ch, rem) .. */
    const uint32_t nch = blk < a.r0 ? a.nlo + 1 : a.nlo, per = a.rt / nch, rem = a.rt % nch;
    const uint32_t m0 = 32u * (ch * per + (ch < rem ? ch : rem)), n0 = blk * kM3Cols;
    const uint32_t span = 32u * (per + (ch < rem ? 1u : 0u));
    const uint32_t rows = a.m - m0 < span ? a.m - m0 : span;
    const float rsc = tid < rows ? a.scale[m0 + tid] : 0.f;
    uint32_t *lut = sm.lut;
    if constexpr (SCHEME == R9VX_SCHEME_IQ4_XS) m3_init_iq4_lut(lut, tid, 512);
    if constexpr (SCHEME == R9VX_SCHEME_IQ3_S) {
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
        aoff[i] = ((m0 + (r < rows ? r : 0)) * a.k + 8 * dma_group(r, lane)) * 2u;
    }
    /* the decoding thread's weight row; past n (the last block of a ragged n)
     * it decodes row n - 1 again, whose columns are not stored */
    const uint32_t brow = n0 + m3_brow(tid) < a.n ? m3_brow(tid) : a.n - 1 - n0;
    M3WRow w{m3_uniform(a.w + (uint64_t)n0 * a.w_row_stride), brow * (uint32_t)a.w_row_stride};
    if constexpr (SCHEME == R9VX_SCHEME_Q8_0 || SCHEME == R9VX_SCHEME_Q6_K) { /* the split layout's d row */
        w.sbase = m3_uniform(reinterpret_cast<const uint8_t *>(a.ws + (uint64_t)n0 * a.ws_row));
        w.soff = brow * a.ws_row * 2u;
    }
    const uint32_t rh = wv >> 2, cq = wv & 3;
    const uint32_t nr = m3_active_tiles(rows, 128 * rh);
    r9vx_f32x16 acc[4][2];
    m3_run<SCHEME, true>(nr, rows <= 128, sm, a.x16, aoff, w, a.k / kTileK, tid, wv, lut, 128 * rh, 64 * cq, 64 * cq + 32, acc);
    if (tid < kM3Rows) rowsc[tid] = rsc;
    __syncthreads();

    /* y = acc * 2^e (the activation row's scale, exact) [+ bias | + residual]
     * in f32, then the output cast.  bf16 rows are staged in LDS (row R's
     * 8-byte chunk c at chunk c ^ (R & 31)) and leave as whole 512-byte
     * rows; f32 rows are stored 16 bytes per lane from the accumulators.
     * A block past n, or any block when n % 8 != 0 (rows then not 16-byte
     * aligned), reads and writes its columns one at a time, up to n. */
    const bool vec = n0 + kM3Cols <= a.n && (a.n & 7u) == 0; /* uniform */
    uint8_t *const ot = m3_out_tile(sm);
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
        if ((uint32_t)tt >= nr) break;
        const uint32_t rl = 128 * rh + 32 * tt + (lane & 31);
        const uint32_t row = m0 + (rl < rows ? rl : 0);
        const float sc = rowsc[rl];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint32_t cl = 64u * cq + 32u * j + 8u * g + 4u * (lane >> 5);
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = acc[tt][j][4 * g + e] * sc;
                const uint32_t c0 = n0 + cl;
                if (a.epilogue != R9VX_EPILOGUE_NONE) {
                    const float *add = a.epilogue == R9VX_EPILOGUE_BIAS ? a.bias + c0 : a.residual + (uint64_t)row * a.n + c0;
                    if (vec) {
                        const r9vx_f32x4 bb = *reinterpret_cast<const r9vx_f32x4 *>(add);
                        v[0] += bb.x, v[1] += bb.y, v[2] += bb.z, v[3] += bb.w;
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (c0 + e < a.n) v[e] += add[e];
                    }
                }
                if (a.y_bf16) {
                    const uint32_t chunk = (cl >> 2) ^ (rl & 31u);
                    *reinterpret_cast<r9vx_u32x2 *>(ot + rl * 512u + 8u * chunk) = r9vx_u32x2{
                        (uint32_t)r9vx_f32_to_bf16(v[0]) | ((uint32_t)r9vx_f32_to_bf16(v[1]) << 16),
                        (uint32_t)r9vx_f32_to_bf16(v[2]) | ((uint32_t)r9vx_f32_to_bf16(v[3]) << 16)};
                } else if (rl < rows) {
                    float *const yr = reinterpret_cast<float *>(a.y) + (uint64_t)row * a.n + c0;
                    if (vec) {
                        *reinterpret_cast<r9vx_f32x4 *>(yr) = r9vx_f32x4{v[0], v[1], v[2], v[3]};
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (c0 + e < a.n) yr[e] = v[e];
                    }
                }
            }
    }
    if (!a.y_bf16) return;
    __syncthreads();
    const uint32_t q = lane & 31;
    uint16_t *const y = reinterpret_cast<uint16_t *>(a.y);
#pragma unroll 4
    for (uint32_t i = 0; i < 16; ++i) {
        const uint32_t R = 16 * i + 2 * wv + (lane >> 5);
        if (R >= rows) break; /* rows grow with i */
        const uint32_t s = R & 31u;
        r9vx_u32x4 v = *reinterpret_cast<const r9vx_u32x4 *>(ot + R * 512u + 16u * (q ^ (s >> 1)));
        if (s & 1u) v = r9vx_u32x4{v.z, v.w, v.x, v.y}; /* the granule's halves were swapped */
        uint16_t *const yr = y + (uint64_t)(m0 + R) * a.n + n0 + 8 * q;
        if (vec) {
            *reinterpret_cast<r9vx_u32x4 *>(yr) = v;
        } else {
            const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (n0 + 8 * q + e < a.n) yr[e] = (uint16_t)(d[e >> 1] >> (16 * (e & 1)));
        }
    }
}

/* gemm3's plan: the rows of each 256-column weight block are cut into
 * chunks of whole 32-row tiles (at most 8), so that the launch is a whole
 * number of rounds of one workgroup per CU with the rows spread over the
 * CUs as evenly as chunks allow.  A chunk's time is a fixed part (its
 * weight block's loads and decode) plus a part per row tile, so every CU
 * runs as many chunks as the 256-row tiling needs rounds and the row tiles
 * are dealt evenly over them, largest chunks first (the hardware gives each
 * next workgroup to the first CU that frees).  Example (m = 2048, n = 14336,
 * 256 CUs): 448 tiles of 256 rows are 1.75 rounds, the second leaving 64 CUs
 * idle; the plan makes 512 chunks, 48 of 8 row tiles, 416 of 7 and 48 of 6,
 * so a CU runs 7 + 7 or 8 + 6.  With fewer tiles than CUs the chunks shrink
 * until every CU has one.  Which rows share a chunk changes no output bit.
 * Returns the workgroup count. */
uint32_t plan_chunks(GemmArgs &a, uint32_t cus) {
    const uint32_t nb = (a.n + kM3Cols - 1) / kM3Cols, rt = (a.m + 31) / 32;
    const uint64_t tiles = (uint64_t)nb * ((rt + 7) / 8);
    uint64_t q = (tiles + cus - 1) / cus * cus;
    if (q > (uint64_t)nb * rt) q = (uint64_t)nb * rt;
    /* one round either way and no smaller largest chunk: the extra chunks
     * would only decode their weight blocks again (m = 1024, n = 14336) */
    const uint32_t per8 = (rt + 7) / 8, nq = (uint32_t)(q / nb);
    if (tiles <= cus && (rt + nq - 1) / nq == (rt + per8 - 1) / per8) q = tiles;
    a.rt = rt;
    a.nlo = (uint32_t)(q / nb); /* >= ceil(rt / 8): no chunk exceeds 8 row tiles */
    a.r0 = (uint32_t)(q % nb);
    const uint32_t na = a.nlo + 1, qa = rt / na, ra = rt % na, qb = rt / a.nlo, rb = rt % a.nlo;
    struct Sized {
        ChunkGroup g;
        uint32_t tiles;
    } gs[4] = {{{a.r0, nb - a.r0, 0, rb}, qb + 1},
               {{a.r0, nb - a.r0, rb, a.nlo - rb}, qb},
               {{0, a.r0, 0, ra}, qa + 1},
               {{0, a.r0, ra, na - ra}, qa}};
    for (int i = 1; i < 4; ++i)
        for (int j = i; j > 0 && gs[j].tiles > gs[j - 1].tiles; --j) {
            const Sized t = gs[j];
            gs[j] = gs[j - 1];
            gs[j - 1] = t;
        }
    for (int i = 0; i < 4; ++i) a.grp[i] = gs[i].g;
    a.band = a.r0 == 0 && q % 8 == 0;
    return (uint32_t)q;
}

}  // namespace

uint32_t r9vx_device_cus() {
    static uint32_t cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
        cached[dev] = (uint32_t)cus;
    }
    return cached[dev];
}

size_t r9vx_gemm_workspace_bytes(uint32_t m_bucket, uint32_t k) {
    return (((size_t)m_bucket * k * 2 + 255) & ~(size_t)255) + (size_t)m_bucket * 4;
}

int r9vx_launch_x_to_f16(const uint16_t *x, uint32_t m, uint32_t k, _Float16 *x16, float *scale,
                         uint32_t perm_scheme, hipStream_t stream) {
    if (perm_scheme == R9VX_SCHEME_Q4_K)
        hipLaunchKernelGGL(x_to_f16_kernel<R9VX_SCHEME_Q4_K>, dim3((m + 3) / 4), dim3(256), 0, stream, x, m, k, x16, scale);
    else if (perm_scheme == R9VX_SCHEME_IQ4_XS)
        hipLaunchKernelGGL(x_to_f16_kernel<R9VX_SCHEME_IQ4_XS>, dim3((m + 3) / 4), dim3(256), 0, stream, x, m, k, x16, scale);
    else if (perm_scheme == R9VX_SCHEME_Q6_K)
        hipLaunchKernelGGL(x_to_f16_kernel<R9VX_SCHEME_Q6_K>, dim3((m + 3) / 4), dim3(256), 0, stream, x, m, k, x16, scale);
    else
        hipLaunchKernelGGL(x_to_f16_kernel<0>, dim3((m + 3) / 4), dim3(256), 0, stream, x, m, k, x16, scale);
    return (int)hipGetLastError();
}

int r9vx_launch_gemm(const r9vx_gemm_problem &p, hipStream_t stream) {
    _Float16 *x16 = reinterpret_cast<_Float16 *>(p.workspace);
    float *scale = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(p.workspace) +
                                             (((size_t)p.m * p.k * 2 + 255) & ~(size_t)255));
    GemmArgs a{};
    a.x16 = x16;
    a.scale = scale;
    a.w = p.w;
    a.bias = p.bias;
    a.residual = p.residual;
    a.y = p.y;
    a.ws = p.w_scales;
    switch (p.scheme) {
    case R9VX_SCHEME_Q4_K: a.w_row_stride = (uint64_t)(p.k / 256) * R9VX_Q4K_BYTES; break;
    case R9VX_SCHEME_IQ4_XS: a.w_row_stride = (uint64_t)(p.k / 256) * R9VX_IQ4XS_BYTES; break;
    case R9VX_SCHEME_Q6_K: a.w_row_stride = (uint64_t)(p.k / 256) * R9VX_Q6K_BODY, a.ws_row = p.k / 256; break;
    case R9VX_SCHEME_IQ3_S: a.w_row_stride = (uint64_t)(p.k / 256) * R9VX_IQ3S_DEV_BYTES; break;
    default: a.w_row_stride = p.k, a.ws_row = p.k / 32; break; /* Q8_0 */
    }
    a.m = p.m;
    a.n = p.n;
    a.k = p.k;
    a.y_bf16 = p.y_dtype == R9VX_DTYPE_BF16;
    a.epilogue = p.epilogue;
    /* One kernel for every scheme and shape (gemm3_kernel: 256 x 256 tiles,
     * each weight tile decoded once into LDS), so each output element's
     * arithmetic -- the K order of the MFMA steps, how a weight is rounded
     * to fp16 -- follows from the scheme and k alone, never from the
     * launch's row count: a row's outputs are the same bits whatever rows
     * share the launch, at whatever index, and in every bucket above the
     * decode GEMV's.  The A copies address x16 with 32-bit offsets, so rows
     * go in launches of at most 2^31 / k elements' worth (which rows share a
     * launch changes no bit either). */
    const int rc = r9vx_launch_x_to_f16(p.x, p.m, p.k, x16, scale, r9vx_group_order(p.scheme), stream);
    if (rc) return rc;
    const uint32_t cus = r9vx_device_cus();
    const uint32_t max_rows = (uint32_t)(((1ull << 31) - 1) / p.k) & ~31u;
    const size_t ysz = a.y_bf16 ? 2 : 4;
    for (uint32_t r0 = 0; r0 < p.m; r0 += max_rows) {
        GemmArgs b = a;
        b.m = p.m - r0 < max_rows ? p.m - r0 : max_rows;
        b.x16 = x16 + (size_t)r0 * p.k;
        b.scale = scale + r0;
        b.y = reinterpret_cast<uint8_t *>(p.y) + (size_t)r0 * p.n * ysz;
        if (p.residual) b.residual = p.residual + (size_t)r0 * p.n;
        const dim3 grid3(plan_chunks(b, cus));
        switch (p.scheme) {
        case R9VX_SCHEME_Q4_K: hipLaunchKernelGGL((gemm3_kernel<R9VX_SCHEME_Q4_K>), grid3, dim3(512), 0, stream, b); break;
        case R9VX_SCHEME_IQ4_XS: hipLaunchKernelGGL((gemm3_kernel<R9VX_SCHEME_IQ4_XS>), grid3, dim3(512), 0, stream, b); break;
        case R9VX_SCHEME_Q8_0: hipLaunchKernelGGL((gemm3_kernel<R9VX_SCHEME_Q8_0>), grid3, dim3(512), 0, stream, b); break;
        case R9VX_SCHEME_Q6_K: hipLaunchKernelGGL((gemm3_kernel<R9VX_SCHEME_Q6_K>), grid3, dim3(512), 0, stream, b); break;
        default: hipLaunchKernelGGL((gemm3_kernel<R9VX_SCHEME_IQ3_S>), grid3, dim3(512), 0, stream, b); break;
        }
        const int e = (int)hipGetLastError();
        if (e) return e;
    }
    return 0;
}
