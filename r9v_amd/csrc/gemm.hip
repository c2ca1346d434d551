/*
 * gemm.hip -- prefill dequant-GEMM on MFMA: y[m, n] = sum_k x[m, k] * w[n, k]
 * for bf16 activations (variants with m_bucket > 8) and GGUF Q4_K / IQ4_XS weights (wire blocks)
 * or Q8_0 / Q6_K weights (split layout) and IQ3_S weights (112-byte repacked
 * blocks), LDS-decoded tiles only.
 *
 * T0 meaning: crates/r9v-t0/src/matmul.rs:1940-2414 (Branch D), output cast
 * crates/r9v-t0/src/dtype.rs:102-111 (bf16 RNE); epilogue matmul.rs:2421-2446.
 *
 * Two launches:
 *  1. x_to_f16: one workgroup per activation row finds max|x|, picks the
 *     power-of-two scale 2^e that keeps the row below 2^15 (e = 0 for any
 *     ordinary activation) and writes the row as fp16 plus the scale.  bf16
 *     values are exact in fp16 inside that range.
 *  2. gemm: 256 x 256 output tile per workgroup; each K step streams 64
 *     columns of x (fp16) and 32 payload bytes of 256 weight rows from HBM
 *     into registers while the MFMAs consume the previous step from LDS, then
 *     dequantizes the weights (exact f32 formula, one fp16 rounding) into the
 *     other LDS buffer.  gemm2 maps workgroups so that each XCD owns a
 *     contiguous band of weight columns (the 8 M-tiles that reuse a weight
 *     tile run on the same XCD and hit its L2); gemm3 cuts each weight
 *     block's rows into chunks sized so that the launch fills whole rounds
 *     of the CUs (plan_chunks).
 */
#include "r9vx_mma.h"
#include "r9vx_mma2.h"
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
    uint32_t m_tiles, n_tiles;
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

template <int SCHEME, int BM, int NBUF>
__global__ __launch_bounds__(256, NBUF == 1 ? 2 : 1) void gemm_kernel(GemmArgs a) {
    using S = MmaShape<BM, NBUF>;
    __shared__ __attribute__((aligned(16))) uint8_t lds[S::kLds];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    /* XCD-aware tile order: workgroup b runs on XCD b % 8; each XCD takes a
     * contiguous band of weight columns so the M tiles sharing a weight tile
     * hit the same L2. */
    const uint32_t total = a.m_tiles * a.n_tiles;
    uint32_t t = blockIdx.x;
    if (total % 8 == 0) t = (blockIdx.x % 8) * (total / 8) + blockIdx.x / 8;
    const uint32_t n_tile = t / a.m_tiles, m_tile = t % a.m_tiles;
    const uint32_t m0 = m_tile * BM, n0 = n_tile * 256;

    AF16Rows<BM> as;
    as.chunk = tid & 7;
    as.row0 = tid >> 3;
#pragma unroll
    for (int i = 0; i < BM / 32; ++i) {
        uint32_t r = m0 + as.row0 + 32 * i;
        as.row[i] = a.x16 + (uint64_t)(r < a.m ? r : a.m - 1) * a.k + 8 * as.chunk;
    }
    const uint32_t wrow = n0 + tid < a.n ? n0 + tid : a.n - 1;
    r9vx_f32x16 acc[BM / 32][2];
    mma_mainloop<SCHEME, BM, NBUF>(lds, as, a.w + (uint64_t)wrow * a.w_row_stride, a.k / kTileK, acc,
                                   a.ws ? a.ws + (uint64_t)wrow * a.ws_row : nullptr);

    /* Epilogue through LDS, 32 rows at a time: the accumulators go to a
     * 32 x 256 f32 stage (row stride 260 floats, so the two half-waves'
     * rows land on different banks), then every wave writes whole output
     * rows with 4 consecutive columns per lane.  acc is only ever indexed
     * with compile-time constants, so it stays in registers. */
    constexpr uint32_t kSRow = 260;
    float *stage = reinterpret_cast<float *>(lds);
    const bool vec = (a.n & 3u) == 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < BM / 32; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                stage[(acc_row(0, r, lane)) * kSRow + acc_col(wave, j, lane)] = acc[i][j][r];
        __syncthreads();
        const uint32_t cl = 4 * (tid & 63);
        const uint32_t col = n0 + cl;
        for (uint32_t q = 0; q < 8; ++q) {
            const uint32_t rl = (tid >> 6) + 4 * q;
            const uint32_t row = m0 + i * 32 + rl;
            if (row >= a.m || col >= a.n) continue;
            const r9vx_f32x4 acc4 = *reinterpret_cast<const r9vx_f32x4 *>(stage + rl * kSRow + cl);
            const float sc = a.scale[row];
            float v[4] = {acc4.x * sc, acc4.y * sc, acc4.z * sc, acc4.w * sc};
            const uint64_t o = (uint64_t)row * a.n + col;
            if (vec) {
                if (a.epilogue == R9VX_EPILOGUE_BIAS) {
                    const r9vx_f32x4 b = *reinterpret_cast<const r9vx_f32x4 *>(a.bias + col);
                    v[0] += b.x, v[1] += b.y, v[2] += b.z, v[3] += b.w;
                }
                if (a.epilogue == R9VX_EPILOGUE_RESIDUAL) {
                    const r9vx_f32x4 b = *reinterpret_cast<const r9vx_f32x4 *>(a.residual + o);
                    v[0] += b.x, v[1] += b.y, v[2] += b.z, v[3] += b.w;
                }
                if (a.y_bf16) {
                    const uint32_t lo = (uint32_t)r9vx_f32_to_bf16(v[0]) | ((uint32_t)r9vx_f32_to_bf16(v[1]) << 16);
                    const uint32_t hi = (uint32_t)r9vx_f32_to_bf16(v[2]) | ((uint32_t)r9vx_f32_to_bf16(v[3]) << 16);
                    *reinterpret_cast<r9vx_u32x2 *>(reinterpret_cast<uint16_t *>(a.y) + o) = r9vx_u32x2{lo, hi};
                } else {
                    *reinterpret_cast<r9vx_f32x4 *>(reinterpret_cast<float *>(a.y) + o) =
                        r9vx_f32x4{v[0], v[1], v[2], v[3]};
                }
            } else {
                for (uint32_t c = 0; c < 4 && col + c < a.n; ++c) {
                    float x = v[c];
                    if (a.epilogue == R9VX_EPILOGUE_BIAS) x += a.bias[col + c];
                    if (a.epilogue == R9VX_EPILOGUE_RESIDUAL) x += a.residual[o + c];
                    if (a.y_bf16)
                        reinterpret_cast<uint16_t *>(a.y)[o + c] = r9vx_f32_to_bf16(x);
                    else
                        reinterpret_cast<float *>(a.y)[o + c] = x;
                }
            }
        }
        __syncthreads();
    }
}

/* 256 x 256 tiles, 8 waves, weights decoded into MFMA operand registers. */
constexpr int kM2Rows = 256, kM2Cols = 256, kM2StageBytes = kM2Rows * 128;

template <int SCHEME>
__global__ __launch_bounds__(512, 1) void gemm2_kernel(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t st0[kM2StageBytes];
    __shared__ __attribute__((aligned(16))) uint8_t st1[kM2StageBytes];
    __shared__ __attribute__((aligned(16))) uint8_t st2[kM2StageBytes];
    __shared__ __attribute__((aligned(16))) uint8_t st3[kM2StageBytes];
    __shared__ __attribute__((aligned(16))) float lutf[512];
    uint8_t *const stages[4] = {st0, st1, st2, st3};
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t total = a.m_tiles * a.n_tiles;
    uint32_t t = blockIdx.x;
    if (total % 8 == 0) t = (blockIdx.x % 8) * (total / 8) + blockIdx.x / 8;
    const uint32_t n_tile = t / a.m_tiles, m_tile = t % a.m_tiles;
    const uint32_t m0 = m_tile * kM2Rows, n0 = n_tile * kM2Cols;

    if constexpr (SCHEME == R9VX_SCHEME_IQ4_XS) init_iq4_lut_f32(reinterpret_cast<r9vx_f32x4 *>(lutf), tid);
    __syncthreads(); /* the codebook table, before any load is in flight */

    const _Float16 *asrc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t r = dma_row(wave, i, lane);
        const uint32_t rr = m0 + r < a.m ? m0 + r : a.m - 1;
        asrc[i] = a.x16 + (uint64_t)rr * a.k + 8 * dma_group(r, lane);
    }
    const uint32_t col = n0 + 32 * wave + (lane & 31);
    const uint8_t *const wrow[1] = {a.w + (uint64_t)(col < a.n ? col : a.n - 1) * a.w_row_stride};

    r9vx_f32x16 acc2[8][1];
    /* K % 256 == 0: a multiple of 4 steps */
    m2_mainloop<SCHEME, 8, 1>(stages, asrc, wrow, a.k / kTileK, wave, lane, lutf, acc2);
    __syncthreads();

    /* epilogue through LDS, 16 rows at a time (stage row stride 260 floats):
     * accumulator registers 8u..8u+7 of tile i are rows 32i + 16u + .. */
    constexpr uint32_t kSRow = 260;
    float *stage = reinterpret_cast<float *>(st0);
    const bool vec = (a.n & 3u) == 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
#pragma unroll
            for (int r = 0; r < 8; ++r)
                stage[(8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * kSRow + 32 * wave + (lane & 31)] =
                    acc2[i][0][8 * u + r];
            __syncthreads();
            const uint32_t cl = 4 * (tid & 63);
            const uint32_t c = n0 + cl;
#pragma unroll
            for (uint32_t q = 0; q < 2; ++q) {
                const uint32_t rl = (tid >> 6) + 8 * q;
                const uint32_t row = m0 + i * 32 + u * 16 + rl;
                if (row >= a.m || c >= a.n) continue;
                const r9vx_f32x4 acc4 = *reinterpret_cast<const r9vx_f32x4 *>(stage + rl * kSRow + cl);
                const float sc = a.scale[row];
                float v[4] = {acc4.x * sc, acc4.y * sc, acc4.z * sc, acc4.w * sc};
                const uint64_t o = (uint64_t)row * a.n + c;
                if (vec) {
                    if (a.epilogue == R9VX_EPILOGUE_BIAS) {
                        const r9vx_f32x4 bb = *reinterpret_cast<const r9vx_f32x4 *>(a.bias + c);
                        v[0] += bb.x, v[1] += bb.y, v[2] += bb.z, v[3] += bb.w;
                    }
                    if (a.epilogue == R9VX_EPILOGUE_RESIDUAL) {
                        const r9vx_f32x4 bb = *reinterpret_cast<const r9vx_f32x4 *>(a.residual + o);
                        v[0] += bb.x, v[1] += bb.y, v[2] += bb.z, v[3] += bb.w;
                    }
                    if (a.y_bf16) {
                        const uint32_t lo =
                            (uint32_t)r9vx_f32_to_bf16(v[0]) | ((uint32_t)r9vx_f32_to_bf16(v[1]) << 16);
                        const uint32_t hi =
                            (uint32_t)r9vx_f32_to_bf16(v[2]) | ((uint32_t)r9vx_f32_to_bf16(v[3]) << 16);
                        *reinterpret_cast<r9vx_u32x2 *>(reinterpret_cast<uint16_t *>(a.y) + o) = r9vx_u32x2{lo, hi};
                    } else {
                        *reinterpret_cast<r9vx_f32x4 *>(reinterpret_cast<float *>(a.y) + o) =
                            r9vx_f32x4{v[0], v[1], v[2], v[3]};
                    }
                } else {
                    for (uint32_t cc = 0; cc < 4 && c + cc < a.n; ++cc) {
                        float x = v[cc];
                        if (a.epilogue == R9VX_EPILOGUE_BIAS) x += a.bias[c + cc];
                        if (a.epilogue == R9VX_EPILOGUE_RESIDUAL) x += a.residual[o + cc];
                        if (a.y_bf16)
                            reinterpret_cast<uint16_t *>(a.y)[o + cc] = r9vx_f32_to_bf16(x);
                        else
                            reinterpret_cast<float *>(a.y)[o + cc] = x;
                    }
                }
            }
            __syncthreads();
        }
    }
}

/* Tiles of up to 256 rows x 256 columns on the r9vx_mma3.h loop (the grouped
 * MoE GEMMs' core): the weight tile is decoded once per workgroup into LDS,
 * every wave reads its B fragments from there, and the accumulators are the
 * transposed tile, so lane l holds output row 128 rh + 32 t + (l & 31) and
 * columns 64 cq + 32 j + 8 (r >> 2) + 4 (l >> 5) + (r & 3) of acc[t][j][r].
 * A workgroup takes the chunk of rows plan_chunks gave its index.  The
 * launcher takes it for n % 256 == 0 and m k < 2^31 (the A copy offsets are
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
    M3WRow w{m3_uniform(a.w + (uint64_t)n0 * a.w_row_stride), m3_brow(tid) * (uint32_t)a.w_row_stride};
    if constexpr (SCHEME == R9VX_SCHEME_Q8_0 || SCHEME == R9VX_SCHEME_Q6_K) { /* the split layout's d row */
        w.sbase = m3_uniform(reinterpret_cast<const uint8_t *>(a.ws + (uint64_t)n0 * a.ws_row));
        w.soff = m3_brow(tid) * a.ws_row * 2u;
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
     * rows; f32 rows are stored 16 bytes per lane from the accumulators. */
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
                if (a.epilogue == R9VX_EPILOGUE_BIAS) {
                    const r9vx_f32x4 bb = *reinterpret_cast<const r9vx_f32x4 *>(a.bias + n0 + cl);
                    v[0] += bb.x, v[1] += bb.y, v[2] += bb.z, v[3] += bb.w;
                } else if (a.epilogue == R9VX_EPILOGUE_RESIDUAL) {
                    const r9vx_f32x4 bb =
                        *reinterpret_cast<const r9vx_f32x4 *>(a.residual + (uint64_t)row * a.n + n0 + cl);
                    v[0] += bb.x, v[1] += bb.y, v[2] += bb.z, v[3] += bb.w;
                }
                if (a.y_bf16) {
                    const uint32_t chunk = (cl >> 2) ^ (rl & 31u);
                    *reinterpret_cast<r9vx_u32x2 *>(ot + rl * 512u + 8u * chunk) = r9vx_u32x2{
                        (uint32_t)r9vx_f32_to_bf16(v[0]) | ((uint32_t)r9vx_f32_to_bf16(v[1]) << 16),
                        (uint32_t)r9vx_f32_to_bf16(v[2]) | ((uint32_t)r9vx_f32_to_bf16(v[3]) << 16)};
                } else if (rl < rows) {
                    *reinterpret_cast<r9vx_f32x4 *>(reinterpret_cast<float *>(a.y) + (uint64_t)row * a.n + n0 + cl) =
                        r9vx_f32x4{v[0], v[1], v[2], v[3]};
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
        *reinterpret_cast<r9vx_u32x4 *>(y + (uint64_t)(m0 + R) * a.n + n0 + 8 * q) = v;
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
    const uint32_t nb = a.n / kM3Cols, rt = (a.m + 31) / 32;
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
    /* The kernel, and with it each output element's arithmetic (the K order
     * of the MFMA steps, how a weight is rounded to fp16), follows from the
     * variant's static keys alone -- scheme, n, k and the bucket's 32-bit
     * addressing bound -- never from the launch's row count: a row's outputs
     * are the same bits whatever rows share the launch, at whatever index,
     * and in every bucket above the decode GEMV's.  Q4_K / IQ4_XS run the
     * 256 x 256 tiles (gemm3 for N % 256 == 0, gemm2 otherwise), Q8_0 / Q6_K /
     * IQ3_S gemm3 for N % 256 == 0 and the 128-row LDS-decoded tile
     * otherwise. */
    const bool split = p.scheme == R9VX_SCHEME_Q8_0 || p.scheme == R9VX_SCHEME_Q6_K || p.scheme == R9VX_SCHEME_IQ3_S;
    const bool m3_shape = p.n % kM3Cols == 0 && (uint64_t)p.m_bucket * p.k < (1ull << 31);
    if (split && m3_shape) {
        /* the split and IQ3_S layouts on the 256 x 256 loop, x in their K order */
        const int rc = r9vx_launch_x_to_f16(p.x, p.m, p.k, x16, scale, r9vx_group_order(p.scheme), stream);
        if (rc) return rc;
        a.m_tiles = (p.m + kM2Rows - 1) / kM2Rows;
        a.n_tiles = (p.n + kM2Cols - 1) / kM2Cols;
        const dim3 grid3(plan_chunks(a, r9vx_device_cus()));
        if (p.scheme == R9VX_SCHEME_Q8_0)
            hipLaunchKernelGGL((gemm3_kernel<R9VX_SCHEME_Q8_0>), grid3, dim3(512), 0, stream, a);
        else if (p.scheme == R9VX_SCHEME_Q6_K)
            hipLaunchKernelGGL((gemm3_kernel<R9VX_SCHEME_Q6_K>), grid3, dim3(512), 0, stream, a);
        else
            hipLaunchKernelGGL((gemm3_kernel<R9VX_SCHEME_IQ3_S>), grid3, dim3(512), 0, stream, a);
        return (int)hipGetLastError();
    }
    if (!split) {
        if (p.scheme == R9VX_SCHEME_Q4_K)
            hipLaunchKernelGGL(x_to_f16_kernel<R9VX_SCHEME_Q4_K>, dim3((p.m + 3) / 4), dim3(256), 0, stream, p.x, p.m, p.k, x16,
                               scale);
        else
            hipLaunchKernelGGL(x_to_f16_kernel<R9VX_SCHEME_IQ4_XS>, dim3((p.m + 3) / 4), dim3(256), 0, stream, p.x, p.m, p.k,
                               x16, scale);
        a.m_tiles = (p.m + kM2Rows - 1) / kM2Rows;
        a.n_tiles = (p.n + kM2Cols - 1) / kM2Cols;
        dim3 grid(a.m_tiles * a.n_tiles);
        if (p.n % kM3Cols == 0 && (uint64_t)p.m_bucket * p.k < (1ull << 31)) {
            const dim3 grid3(plan_chunks(a, r9vx_device_cus()));
            if (p.scheme == R9VX_SCHEME_Q4_K)
                hipLaunchKernelGGL((gemm3_kernel<R9VX_SCHEME_Q4_K>), grid3, dim3(512), 0, stream, a);
            else
                hipLaunchKernelGGL((gemm3_kernel<R9VX_SCHEME_IQ4_XS>), grid3, dim3(512), 0, stream, a);
            return (int)hipGetLastError();
        }
        if (p.scheme == R9VX_SCHEME_Q4_K)
            hipLaunchKernelGGL((gemm2_kernel<R9VX_SCHEME_Q4_K>), grid, dim3(512), 0, stream, a);
        else
            hipLaunchKernelGGL((gemm2_kernel<R9VX_SCHEME_IQ4_XS>), grid, dim3(512), 0, stream, a);
        return (int)hipGetLastError();
    }
    hipLaunchKernelGGL(x_to_f16_kernel<0>, dim3((p.m + 3) / 4), dim3(256), 0, stream, p.x, p.m, p.k, x16, scale);
    a.m_tiles = (p.m + 127) / 128;
    a.n_tiles = (p.n + 255) / 256;
    dim3 grid(a.m_tiles * a.n_tiles);
    /* Q8_0 / Q6_K / IQ3_S at N % 256 != 0 take this LDS-decoded tile (their steps do not
     * fit the register-decoded core's 16-byte lane payload). */
    switch (p.scheme) {
    case R9VX_SCHEME_Q6_K: hipLaunchKernelGGL((gemm_kernel<R9VX_SCHEME_Q6_K, 128, 1>), grid, dim3(256), 0, stream, a); break;
    case R9VX_SCHEME_IQ3_S: hipLaunchKernelGGL((gemm_kernel<R9VX_SCHEME_IQ3_S, 128, 1>), grid, dim3(256), 0, stream, a); break;
    default: hipLaunchKernelGGL((gemm_kernel<R9VX_SCHEME_Q8_0, 128, 1>), grid, dim3(256), 0, stream, a); break;
    }
    return (int)hipGetLastError();
}
