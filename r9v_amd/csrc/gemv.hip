/*
 * gemv.hip -- decode-time dequant-fused GEMV, y[m, n] = sum_k x[m, k] * w[n, k],
 * for GGUF Q4_K / IQ4_XS weights (wire blocks), Q8_0 / Q6_K weights (split
 * layout: body + f16 d array) and IQ3_S weights (112-byte repacked blocks),
 * and m <= 8 activation rows.
 *
 * T0 meaning: crates/r9v-t0/src/matmul.rs:1940-2414 (Branch D, f32
 * accumulate); weight decode crates/r9v-format/src/ggml.rs:1131-1150 (Q4_K)
 * and crates/r9v-format/src/iq.rs:578-598 (IQ4_XS).
 *
 * Bandwidth-bound design for CDNA4 wave64 (no MFMA):
 *  - A lane owns a fixed set of 16-byte payload chunks (32 weights each) at the
 *    same K positions in every row, so its activation slice is loaded and
 *    re-arranged into registers once and reused for all R rows it visits.
 *  - A row's chunks are spread over LPR consecutive lanes, so one 128-bit load
 *    instruction of a wave reads whole contiguous row segments (coalesced).
 *    All of a lane's weight loads for its R rows are issued before any math.
 *  - bf16 activations use v_dot2_f32_bf16 (two MACs per lane-op, f32
 *    accumulate).  Q4_K nibbles become bf16 with one AND-OR: 0x4300|q is the
 *    bf16 of 128+q, and the 128*sum(x) offset is folded into the min term.
 *    IQ4_XS nibble pairs index a 256-entry LDS table of bf16 codebook pairs.
 *  - f32 activations (config 0) use exact nibble->f32 conversion and f32 FMA.
 *  - Per-row partials are summed across the LPR lanes with a butterfly.
 */
#include <type_traits>

#include "r9vx_expf.h"
#include "r9vx_gemv_core.h"

namespace {

struct GemvArgs {
    const uint8_t *w;
    const uint16_t *ws; /* split layouts: f16 d per block */
    const void *x;
    const float *bias;
    const float *residual;
    void *y;
    uint64_t w_row_stride;
    uint64_t x_row_stride;
    uint32_t n;
    uint32_t k;
    uint32_t lpr_log2; /* lanes per row = 1 << lpr_log2 */
    uint32_t nseg;     /* K segments of LPR*SPL chunks */
    uint32_t y_bf16;
    uint32_t epilogue;
    uint32_t ws_row; /* d values per weight row */
};

constexpr bool split_scheme(int s) { return s == R9VX_SCHEME_Q8_0 || s == R9VX_SCHEME_Q6_K; }
/* schemes whose chunks are carried as a Payload2 */
constexpr bool pay2_scheme(int s) { return split_scheme(s) || s == R9VX_SCHEME_IQ3_S; }
/* LDS table words: the IQ3_S codebook as bf16 quads, the IQ4_XS pair table */
constexpr int lut_words(int s) { return s == R9VX_SCHEME_IQ3_S ? 1024 : 256; }

/* Rows per lane group per wave and waves per workgroup, by activation row
 * count (measured on MI355X at K=2048/4096): two rows in two-wave groups
 * for M <= 2, three rows in one-wave groups above, where the per-row math
 * grows and the activation registers are shared by more rows. */
constexpr int rows_for(int m) { return m <= 2 ? 2 : 3; }
constexpr int waves_for(int m) { return m <= 2 ? 2 : 1; }

using namespace r9vx;

/* LPRL = 6: 64 lanes per row, a single K segment (K = 2048*SPL), f32 y and
 * no epilogue, all fixed at compile time (measured 0.4-0.6 us faster per
 * launch at configs[1] than the general form), and RR rows per lane group
 * chosen by the launcher to balance the waves over the SIMDs (NS = 0: the
 * same with the K segment count read from the arguments); LPRL = 0:
 * lanes per row, segment count and epilogue come from the arguments and
 * the rows per lane group from rows_for(M). */
/* XS (single-segment 64-lane form only): four waves per workgroup, one per
 * SIMD of a CU, share the activation slices: the workgroup copies them once
 * into LDS in lane order (piece j of chunk s of row t for lane l at
 * ((s M + t) NP + j) 64 + l, so each wave's 16-byte reads are contiguous
 * across its lanes) and every wave reads its slices from there, instead of
 * each wave loading all of x from L2. */
template <int SCHEME, int M, bool XF32, int SPL, int LPRL, int RR, int NS = 1, bool XS = false>
__global__ __launch_bounds__(XS ? 256 : waves_for(M) * 64) void gemv_kernel(GemvArgs a) {
    static_assert(!XS || (LPRL == 6 && NS == 1), "x staging needs the single-segment 64-lane form");
    constexpr int kRows = RR ? RR : rows_for(M), kWaves = XS ? 4 : waves_for(M);
    constexpr int kNP = XF32 ? 8 : 4; /* 16-byte pieces of a lane's chunk of one x row */
    constexpr int kPieces = XS ? SPL * M * kNP * 64 : 1;
    constexpr int kPass = (kPieces + 255) / 256;
    __shared__ __attribute__((aligned(16))) uint32_t lut[lut_words(SCHEME)];
    __shared__ __attribute__((aligned(16))) r9vx_u32x4 xs[kPieces];
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = blockIdx.x * kWaves + (threadIdx.x >> 6);
    const uint32_t lprl = LPRL ? (uint32_t)LPRL : a.lpr_log2;
    const uint32_t lpr = 1u << lprl;
    const uint32_t rpi = 64u >> lprl; /* row slots per wave */
    const uint32_t lir = lane & (lpr - 1);
    const uint32_t slot = lane >> lprl;
    const uint32_t row0 = wave * rpi * kRows + slot;

    float acc[kRows][M];
#pragma unroll
    for (int r = 0; r < kRows; ++r)
#pragma unroll
        for (int t = 0; t < M; ++t) acc[r][t] = 0.f;

    const uint32_t nseg = (LPRL && NS == 1) ? 1u : a.nseg;
    for (uint32_t seg = 0; seg < nseg; ++seg) {
        uint32_t cis[SPL];
#pragma unroll
        for (int s = 0; s < SPL; ++s) cis[s] = seg * lpr * SPL + s * lpr + lir;
        /* 1. the activation loads (L2-resident after the first wave), then
         * every weight load of this wave: loads complete in order, so the
         * math on row 0 can start while later rows are still in flight */
        XRaw<XF32> xr[SPL][M];
        r9vx_u32x4 xst[kPass];
        if constexpr (XS) {
            /* this thread's pieces of the workgroup's copy */
#pragma unroll
            for (int q = 0; q < kPass; ++q) {
                const uint32_t idx = threadIdx.x + 256u * q;
                if (kPieces % 256 == 0 || idx < (uint32_t)kPieces) {
                    const uint32_t l = idx & 63u, j = (idx >> 6) % kNP, t = (idx >> 6) / kNP % M,
                                   sp = (idx >> 6) / kNP / M;
                    uint32_t klo, khi;
                    chunk_k<SCHEME>(sp * 64u + l, klo, khi);
                    constexpr uint32_t kPer = XF32 ? 4 : 8; /* elements per piece */
                    const uint32_t e = j < kNP / 2 ? klo + kPer * j : khi + kPer * (j - kNP / 2);
                    const uint8_t *xb = reinterpret_cast<const uint8_t *>(a.x) +
                                        ((uint64_t)t * a.x_row_stride + e) * (XF32 ? 4 : 2);
                    xst[q] = *reinterpret_cast<const r9vx_u32x4 *>(xb);
                }
            }
        } else {
#pragma unroll
            for (int s = 0; s < SPL; ++s) {
                uint32_t klo, khi;
                chunk_k<SCHEME>(cis[s], klo, khi);
#pragma unroll
                for (int t = 0; t < M; ++t) {
                    const uint8_t *xb = reinterpret_cast<const uint8_t *>(a.x) +
                                        (uint64_t)t * a.x_row_stride * (XF32 ? 4 : 2);
                    load_x_raw<XF32>(xb, klo, khi, xr[s][t]);
                }
            }
        }
        /* keep every activation load ahead of the weight loads: loads
         * complete in order, so an activation load scheduled after a weight
         * load would hold the activation re-arrangement until HBM answers */
        __builtin_amdgcn_sched_barrier(0);
        using Pay = typename std::conditional<pay2_scheme(SCHEME), Payload2, r9vx_u32x4>::type;
        Pay qs[kRows][SPL];
        Hdr hd[kRows][SPL];
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            uint32_t row = row0 + r * rpi;
            uint32_t rr = row < a.n ? row : a.n - 1; /* clamp: loads stay in bounds */
            const uint8_t *wrow = a.w + (uint64_t)rr * a.w_row_stride;
#pragma unroll
            for (int s = 0; s < SPL; ++s) {
                if constexpr (SCHEME == R9VX_SCHEME_IQ3_S)
                    load_chunk_iq3s(wrow, cis[s], qs[r][s], hd[r][s]);
                else if constexpr (split_scheme(SCHEME))
                    load_chunk_split<SCHEME>(wrow, a.ws + (uint64_t)rr * a.ws_row, cis[s], qs[r][s], hd[r][s]);
                else
                    load_chunk<SCHEME, true>(wrow, cis[s], qs[r][s], hd[r][s]); /* read once: non-temporal */
            }
        }
        /* 2. the codebook table is built (and the activation copy stored)
         * while the weight loads are in flight */
        if constexpr (SCHEME == R9VX_SCHEME_IQ4_XS) {
            if ((LPRL != 0 && NS == 1) || seg == 0) {
                build_iq4_lut(lut, threadIdx.x, blockDim.x);
                if constexpr (!XS) __syncthreads();
            }
        } else if constexpr (SCHEME == R9VX_SCHEME_IQ3_S) {
            if ((LPRL != 0 && NS == 1) || seg == 0) {
                build_iq3s_lut(lut, threadIdx.x, blockDim.x);
                if constexpr (!XS) __syncthreads();
            }
        }
        if constexpr (XS) {
#pragma unroll
            for (int q = 0; q < kPass; ++q) {
                const uint32_t idx = threadIdx.x + 256u * q;
                if (kPieces % 256 == 0 || idx < (uint32_t)kPieces) xs[idx] = xst[q];
            }
            __syncthreads();
#pragma unroll
            for (int s = 0; s < SPL; ++s)
#pragma unroll
                for (int t = 0; t < M; ++t)
#pragma unroll
                    for (int j = 0; j < kNP; ++j) {
                        const r9vx_u32x4 v = xs[((s * M + t) * kNP + j) * 64 + lane];
                        if constexpr (XF32)
                            xr[s][t].v[j] = __builtin_bit_cast(r9vx_f32x4, v);
                        else
                            xr[s][t].v[j] = v;
                    }
        }
        XChunk<SCHEME, XF32> xc[SPL][M];
#pragma unroll
        for (int s = 0; s < SPL; ++s)
#pragma unroll
            for (int t = 0; t < M; ++t) arrange_x<SCHEME, XF32>(xr[s][t], xc[s][t]);
#pragma unroll
        for (int r = 0; r < kRows; ++r)
#pragma unroll
            for (int s = 0; s < SPL; ++s) {
                if constexpr (SCHEME == R9VX_SCHEME_IQ3_S)
                    chunk_dot_iq3s<M>(qs[r][s], hd[r][s], cis[s] & 7, xc[s], acc[r], lut);
                else if constexpr (split_scheme(SCHEME))
                    chunk_dot_split<SCHEME, M>(qs[r][s], hd[r][s], cis[s] & 7, xc[s], acc[r]);
                else
                    chunk_dot<SCHEME, XF32, M>(qs[r][s], hd[r][s], cis[s] & 7, xc[s], acc[r], lut);
            }
    }

    /* cross-lane sums of all kRows*M partials at once; the lanes that end
     * up holding a sum apply the epilogue and store it */
    constexpr int V = kRows * M;
    float v[1][V];
#pragma unroll
    for (int r = 0; r < kRows; ++r)
#pragma unroll
        for (int t = 0; t < M; ++t) v[0][r * M + t] = acc[r][t];
    auto emit = [&](int idx, const float (&val)[1]) {
        const int r = idx / M, t = idx % M;
        const uint32_t row = row0 + r * rpi;
        if (row >= a.n) return;
        float y = val[0];
        if constexpr (LPRL != 0) {
            reinterpret_cast<float *>(a.y)[(uint64_t)t * a.n + row] = y;
            return;
        }
        if (a.epilogue == R9VX_EPILOGUE_BIAS) y += a.bias[row];
        if (a.epilogue == R9VX_EPILOGUE_RESIDUAL) y += a.residual[(uint64_t)t * a.n + row];
        const uint64_t o = (uint64_t)t * a.n + row;
        if (a.y_bf16)
            reinterpret_cast<uint16_t *>(a.y)[o] = r9vx_f32_to_bf16(y);
        else
            reinterpret_cast<float *>(a.y)[o] = y;
    };
    if constexpr (LPRL != 0)
        lane_reduce<V, 1 << LPRL, 1>(v, lane, emit);
    else
        lane_reduce_w<V, 1>(v, lane, a.lpr_log2, emit);
}

/* The streaming form for one activation row over many output rows (m = 1,
 * one 64-lane K segment per row, f32 y, no epilogue, n >= 12 x SIMDs): a
 * wave walks the row groups gw, gw + W, ... (RR rows each, W waves in the
 * grid, `steps` groups per wave at most), loading the next group's weights
 * before it computes the current one (two register buffers; a group past
 * the end repeats the last group's loads, so every path issues the same
 * loads), with its activation slices loaded and arranged once.  The row
 * sums wait in LDS until the wave's last load is issued: a store between
 * two loads would make the next wait a wait for the store as well.  Per row
 * the arithmetic is gemv_kernel's (the lane's chunks lir, lir + 64 in that
 * order, the same cross-lane tree), so the outputs are the same bits. */
constexpr uint32_t kStreamMaxSteps = 16;
/* rows per group and waves per SIMD: measured (Q4_K 32768 x 4096, IQ4_XS
 * 32768 x 2048, Q4_K 14336 x 4096, graph-replayed) against (2, 3), (4, 2),
 * (1, 4), (2, 4) and (4, 3), which were 2-50% slower */
constexpr uint32_t kStreamRows = 2, kStreamWavesPerSimd = 2;

template <int SCHEME, bool XF32, int SPL, int RR>
__global__ __launch_bounds__(256) void gemv_stream_kernel(GemvArgs a, uint32_t steps) {
    using Pay = typename std::conditional<pay2_scheme(SCHEME), Payload2, r9vx_u32x4>::type;
    __shared__ __attribute__((aligned(16))) uint32_t lut[lut_words(SCHEME)];
    __shared__ float ob[4][kStreamMaxSteps * RR];
    const uint32_t lane = threadIdx.x & 63, wl = threadIdx.x >> 6;
    const uint32_t gw = blockIdx.x * 4 + wl, nw = gridDim.x * 4;
    const uint32_t ngroups = (a.n + RR - 1) / RR;
    uint32_t cis[SPL];
#pragma unroll
    for (int s = 0; s < SPL; ++s) cis[s] = (uint32_t)s * 64u + lane;
    XRaw<XF32> xr[SPL];
#pragma unroll
    for (int s = 0; s < SPL; ++s) {
        uint32_t klo, khi;
        chunk_k<SCHEME>(cis[s], klo, khi);
        load_x_raw<XF32>(a.x, klo, khi, xr[s]);
    }
    __builtin_amdgcn_sched_barrier(0);
    Pay qa[RR][SPL], qb[RR][SPL];
    Hdr ha[RR][SPL], hb[RR][SPL];
    auto issue = [&](uint32_t step, Pay (&q)[RR][SPL], Hdr (&h)[RR][SPL]) {
        uint32_t g = gw + step * nw;
        if (g >= ngroups) g = ngroups - 1;
#pragma unroll
        for (int r = 0; r < RR; ++r) {
            const uint32_t row = g * RR + (uint32_t)r, rr = row < a.n ? row : a.n - 1;
            const uint8_t *wrow = a.w + (uint64_t)rr * a.w_row_stride;
#pragma unroll
            for (int s = 0; s < SPL; ++s) load_chunk<SCHEME>(wrow, cis[s], q[r][s], h[r][s]);
        }
    };
    issue(0, qa, ha);
    if constexpr (SCHEME == R9VX_SCHEME_IQ4_XS) {
        build_iq4_lut(lut, threadIdx.x, blockDim.x);
        __syncthreads();
    }
    XChunk<SCHEME, XF32> xc[SPL][1];
#pragma unroll
    for (int s = 0; s < SPL; ++s) arrange_x<SCHEME, XF32>(xr[s], xc[s][0]);
    float *const obw = ob[wl];
    auto compute = [&](uint32_t step, const Pay (&q)[RR][SPL], const Hdr (&h)[RR][SPL]) {
        float acc[RR][1];
#pragma unroll
        for (int r = 0; r < RR; ++r) {
            acc[r][0] = 0.f;
#pragma unroll
            for (int s = 0; s < SPL; ++s) chunk_dot<SCHEME, XF32, 1>(q[r][s], h[r][s], cis[s] & 7, xc[s], acc[r], lut);
        }
        float v[1][RR];
#pragma unroll
        for (int r = 0; r < RR; ++r) v[0][r] = acc[r][0];
        lane_reduce<RR, 64, 1>(v, lane, [&](int idx, const float (&val)[1]) { obw[step * RR + idx] = val[0]; });
    };
    for (uint32_t step = 0; step < steps; step += 2) {
        issue(step + 1, qb, hb);
        compute(step, qa, ha);
        if (step + 1 >= steps) break;
        issue(step + 2, qa, ha);
        compute(step + 1, qb, hb);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float *const y = reinterpret_cast<float *>(a.y);
    for (uint32_t j = lane; j < steps * RR; j += 64) {
        const uint32_t g = gw + (j / RR) * nw, row = g * RR + j % RR;
        if (g < ngroups && row < a.n) y[row] = obw[j];
    }
}

template <int SCHEME, bool XF32, int SPL>
int launch_stream(const GemvArgs &a, uint32_t simds, hipStream_t s) {
    const uint32_t ngroups = (a.n + kStreamRows - 1) / kStreamRows;
    uint32_t waves = kStreamWavesPerSimd * simds;
    if ((ngroups + waves - 1) / waves > kStreamMaxSteps) waves = (ngroups + kStreamMaxSteps - 1) / kStreamMaxSteps;
    const uint32_t wgs = (waves + 3) / 4, steps = (ngroups + wgs * 4 - 1) / (wgs * 4);
    hipLaunchKernelGGL((gemv_stream_kernel<SCHEME, XF32, SPL, kStreamRows>), dim3(wgs), dim3(256), 0, s, a, steps);
    return (int)hipGetLastError();
}

/* The gated (SwiGLU) form: y[m, j] = silu(x[m] . w[j]) * (x[m] . w[n + j])
 * over stacked weights (gate rows [0, n), up rows [n, 2n)), the matmul +
 * act_mul pair of T0 (crates/r9v-t0/src/act_mul.rs:86-99 with SiLU
 * x / (1 + exp(-x)), crates/r9v-t0/src/activation.rs:135-138) in one launch.
 * A lane group computes the gate and the up row of each of its output rows;
 * the two partial arrays are summed across the lanes together, so the lane
 * that receives a row's gate sum also holds its up sum.  bf16 activations,
 * general lane mapping (runtime lanes per row and K segments).  PAIRS gate/up
 * row pairs per lane group: the launcher takes two when n >= 8 x SIMDs and
 * one below (measured, Q4_K, graph replay: n = 14336, K = 4096, M = 4:
 * 39.2 us at two against 49.1 at one and 64.9 at three; n = 2816, K = 2048,
 * M = 8: 11.5 us at one against 21.3 at two). */
template <int SCHEME, int M, int SPL, int PAIRS>
__global__ __launch_bounds__(waves_for(M) * 64) void gemv_gated_kernel(GemvArgs a) {
    constexpr int kRows = PAIRS, kWaves = waves_for(M);
    __shared__ __attribute__((aligned(16))) uint32_t lut[lut_words(SCHEME)];
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = blockIdx.x * kWaves + (threadIdx.x >> 6);
    const uint32_t lprl = a.lpr_log2, lpr = 1u << lprl, rpi = 64u >> lprl;
    const uint32_t lir = lane & (lpr - 1), slot = lane >> lprl;
    const uint32_t row0 = wave * rpi * kRows + slot;

    float acc[2][kRows][M];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < kRows; ++r)
#pragma unroll
            for (int t = 0; t < M; ++t) acc[h][r][t] = 0.f;

    for (uint32_t seg = 0; seg < a.nseg; ++seg) {
        uint32_t cis[SPL];
#pragma unroll
        for (int s = 0; s < SPL; ++s) cis[s] = seg * lpr * SPL + s * lpr + lir;
        XRaw<false> xr[SPL][M];
#pragma unroll
        for (int s = 0; s < SPL; ++s) {
            uint32_t klo, khi;
            chunk_k<SCHEME>(cis[s], klo, khi);
#pragma unroll
            for (int t = 0; t < M; ++t)
                load_x_raw<false>(reinterpret_cast<const uint8_t *>(a.x) + (uint64_t)t * a.x_row_stride * 2, klo,
                                  khi, xr[s][t]);
        }
        __builtin_amdgcn_sched_barrier(0);
        using Pay = typename std::conditional<pay2_scheme(SCHEME), Payload2, r9vx_u32x4>::type;
        Pay qs[2][kRows][SPL];
        Hdr hd[2][kRows][SPL];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
                const uint32_t row = row0 + r * rpi;
                const uint64_t wr = (uint64_t)(row < a.n ? row : a.n - 1) + (uint64_t)h * a.n;
                const uint8_t *wrow = a.w + wr * a.w_row_stride;
#pragma unroll
                for (int s = 0; s < SPL; ++s) {
                    if constexpr (SCHEME == R9VX_SCHEME_IQ3_S)
                        load_chunk_iq3s(wrow, cis[s], qs[h][r][s], hd[h][r][s]);
                    else if constexpr (split_scheme(SCHEME))
                        load_chunk_split<SCHEME>(wrow, a.ws + wr * a.ws_row, cis[s], qs[h][r][s], hd[h][r][s]);
                    else
                        load_chunk<SCHEME>(wrow, cis[s], qs[h][r][s], hd[h][r][s]);
                }
            }
        if constexpr (SCHEME == R9VX_SCHEME_IQ4_XS) {
            if (seg == 0) {
                build_iq4_lut(lut, threadIdx.x, blockDim.x);
                __syncthreads();
            }
        } else if constexpr (SCHEME == R9VX_SCHEME_IQ3_S) {
            if (seg == 0) {
                build_iq3s_lut(lut, threadIdx.x, blockDim.x);
                __syncthreads();
            }
        }
        XChunk<SCHEME, false> xc[SPL][M];
#pragma unroll
        for (int s = 0; s < SPL; ++s)
#pragma unroll
            for (int t = 0; t < M; ++t) arrange_x<SCHEME, false>(xr[s][t], xc[s][t]);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int r = 0; r < kRows; ++r)
#pragma unroll
                for (int s = 0; s < SPL; ++s) {
                    if constexpr (SCHEME == R9VX_SCHEME_IQ3_S)
                        chunk_dot_iq3s<M>(qs[h][r][s], hd[h][r][s], cis[s] & 7, xc[s], acc[h][r], lut);
                    else if constexpr (split_scheme(SCHEME))
                        chunk_dot_split<SCHEME, M>(qs[h][r][s], hd[h][r][s], cis[s] & 7, xc[s], acc[h][r]);
                    else
                        chunk_dot<SCHEME, false, M>(qs[h][r][s], hd[h][r][s], cis[s] & 7, xc[s], acc[h][r], lut);
                }
    }

    constexpr int V = kRows * M;
    float v[2][V];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < kRows; ++r)
#pragma unroll
            for (int t = 0; t < M; ++t) v[h][r * M + t] = acc[h][r][t];
    lane_reduce_w<V, 2>(v, lane, a.lpr_log2, [&](int idx, const float (&val)[2]) {
        const int r = idx / M, t = idx % M;
        const uint32_t row = row0 + r * rpi;
        if (row >= a.n) return;
        const float g = val[0];
        const float act = g / (1.0f + r9vx_expf(-g));
        const float y = act * val[1];
        const uint64_t o = (uint64_t)t * a.n + row;
        if (a.y_bf16)
            reinterpret_cast<uint16_t *>(a.y)[o] = r9vx_f32_to_bf16(y);
        else
            reinterpret_cast<float *>(a.y)[o] = y;
    });
}

template <int SCHEME, int SPL, int PAIRS, int MM>
int launch_gated(const GemvArgs &a, uint32_t m, uint32_t groups, hipStream_t s) {
    if constexpr (MM == 0) {
        return (int)hipErrorInvalidValue;
    } else {
        if (m != MM) return launch_gated<SCHEME, SPL, PAIRS, MM - 1>(a, m, groups, s);
        const uint32_t rows_per_wave = groups * PAIRS;
        const uint32_t waves = (a.n + rows_per_wave - 1) / rows_per_wave;
        const dim3 grid((waves + waves_for(MM) - 1) / waves_for(MM));
        hipLaunchKernelGGL((gemv_gated_kernel<SCHEME, MM, SPL, PAIRS>), grid, dim3(waves_for(MM) * 64), 0, s, a);
        return (int)hipGetLastError();
    }
}

uint32_t device_simds();

template <int SCHEME>
int launch_gated_scheme(const GemvArgs &a, uint32_t m, int spl, uint32_t g, hipStream_t s) {
    /* IQ3_S carries a wider chunk (payload, signs and side word): two row
     * pairs at M >= 6 need more registers than a wave has at two waves per
     * SIMD and the compiler moves arrays to scratch, so those run one pair */
    constexpr int kTwoPairMaxM = SCHEME == R9VX_SCHEME_IQ3_S ? 5 : 8;
    if (a.n >= 8 * device_simds() && (int)m <= kTwoPairMaxM)
        return spl == 2 ? launch_gated<SCHEME, 2, 2, 4>(a, m, g, s) : launch_gated<SCHEME, 1, 2, kTwoPairMaxM>(a, m, g, s);
    return spl == 2 ? launch_gated<SCHEME, 2, 1, 4>(a, m, g, s) : launch_gated<SCHEME, 1, 1, 8>(a, m, g, s);
}

/* SIMDs of the current device (4 per CU), for the wave-balance rule. */
uint32_t device_simds() { return 4u * r9vx_device_cus(); }

/* Rows per lane group for the compile-time form at M >= 3: the R in 2..5 whose wave
 * count ceil(n / R) gives the busiest SIMD the least work,
 * ceil(waves / simds) * (R + x): from M >= 3 a wave's activation loads and
 * re-arrangement cost about one row's dot products whatever R is (x = 1);
 * for one or two rows they are small (x = 0).  Ties go to the larger R.
 * At n = 5120 this is R = 5 (1024 waves, one per SIMD), measured 5.28 us
 * against 5.47 us for R = 3 at M = 5; at n = 14336, M = 4 it is R = 5 where
 * x = 0 took R = 2 (Q4_K, K = 4096: 25.1 -> 21.6 us), while M = 1 there
 * keeps R = 2 (12.5 us against 13.4 at R = 5). */
uint32_t balanced_rows(uint32_t n, uint32_t simds, uint32_t x) {
    uint32_t best = 2, best_cost = ~0u;
    for (uint32_t r = 2; r <= 5; ++r) {
        const uint32_t waves = (n + r - 1) / r;
        const uint32_t cost = (waves + simds - 1) / simds * (r + x);
        if (cost <= best_cost) best = r, best_cost = cost;
    }
    return best;
}

template <int SCHEME, bool XF32, int SPL, int MM, int LPRL, int RR, int NS = 1, bool XS = false>
int launch_rows(const GemvArgs &a, uint32_t rows_per_slot_group, hipStream_t s) {
    /* rows_per_slot_group = lane groups per wave (64 / LPR) */
    const uint32_t rows_per_wave = rows_per_slot_group * (RR ? RR : rows_for(MM));
    const uint32_t waves = (a.n + rows_per_wave - 1) / rows_per_wave;
    const uint32_t wpg = XS ? 4 : waves_for(MM);
    const dim3 grid((waves + wpg - 1) / wpg);
    hipLaunchKernelGGL((gemv_kernel<SCHEME, MM, XF32, SPL, LPRL, RR, NS, XS>), grid, dim3(wpg * 64), 0, s, a);
    return (int)hipGetLastError();
}

constexpr bool kXStage = true;

template <int SCHEME, bool XF32, int SPL, int MM>
int launch_one(const GemvArgs &a, uint32_t m, uint32_t rows_per_slot_group, hipStream_t s) {
    if constexpr (MM == 0) {
        return (int)hipErrorInvalidValue;
    } else {
        if (m != MM) return launch_one<SCHEME, XF32, SPL, MM - 1>(a, m, rows_per_slot_group, s);
        if constexpr (MM == 1 && (SCHEME == R9VX_SCHEME_Q4_K || SCHEME == R9VX_SCHEME_IQ4_XS)) {
            /* one activation row over many rows: the streaming form */
            if (a.lpr_log2 == 6 && a.nseg == 1 && a.epilogue == R9VX_EPILOGUE_NONE && !a.y_bf16) {
                const uint32_t simds = device_simds();
                if (a.n >= 12 * simds) return launch_stream<SCHEME, XF32, SPL>(a, simds, s);
            }
        }
        if (a.lpr_log2 == 6 && a.nseg == 1 && a.epilogue == R9VX_EPILOGUE_NONE && !a.y_bf16) {
            /* one or two activation rows: two rows per lane group while
             * the launch is latency-bound (n = 5120, M = 1: 3.90 us against
             * 3.98-4.22 us for R = 3..5); from n >= 8 * SIMDs the launch is
             * issue-bound and more rows per group amortise the per-wave work
             * (n = 20480, M = 1: 7.52 us at R = 4 against 8.05 at R = 2;
             * n = 51200: 15.0 against 16.6 us) */
            const uint32_t simds = device_simds();
            switch (MM <= 2 && a.n < 8 * simds ? 2u : balanced_rows(a.n, simds, MM >= 3 ? 1u : 0u)) {
            case 2: return launch_rows<SCHEME, XF32, SPL, MM, 6, 2, 1, kXStage>(a, 1, s);
            case 3: return launch_rows<SCHEME, XF32, SPL, MM, 6, 3, 1, kXStage>(a, 1, s);
            case 4: return launch_rows<SCHEME, XF32, SPL, MM, 6, 4, 1, kXStage>(a, 1, s);
            default: return launch_rows<SCHEME, XF32, SPL, MM, 6, 5, 1, kXStage>(a, 1, s);
            }
        }
        if constexpr (!XF32) {
            /* several K segments of 64 lanes (K >= 8192, K = 14336, or
             * K = 4096 at M >= 5): the same compile-time form with the
             * segment count read at run time */
            if (a.lpr_log2 == 6 && a.nseg > 1 && a.epilogue == R9VX_EPILOGUE_NONE && !a.y_bf16) {
                const uint32_t simds = device_simds();
                switch (MM <= 2 && a.n < 8 * simds ? 2u : balanced_rows(a.n, simds, MM >= 3 ? 1u : 0u)) {
                case 2: return launch_rows<SCHEME, XF32, SPL, MM, 6, 2, 0>(a, 1, s);
                case 3: return launch_rows<SCHEME, XF32, SPL, MM, 6, 3, 0>(a, 1, s);
                case 4: return launch_rows<SCHEME, XF32, SPL, MM, 6, 4, 0>(a, 1, s);
                default: return launch_rows<SCHEME, XF32, SPL, MM, 6, 5, 0>(a, 1, s);
                }
            }
        }
        return launch_rows<SCHEME, XF32, SPL, MM, 0, 0>(a, rows_per_slot_group, s);
    }
}

/* Two chunks per lane are only instantiated for the row counts the launcher
 * picks them for (M <= 4 bf16, M <= 2 f32). */
template <int SCHEME>
int launch_scheme(const GemvArgs &a, uint32_t m, bool xf32, int spl, uint32_t g, hipStream_t s) {
    if (xf32) return spl == 2 ? launch_one<SCHEME, true, 2, 2>(a, m, g, s) : launch_one<SCHEME, true, 1, 8>(a, m, g, s);
    return spl == 2 ? launch_one<SCHEME, false, 2, 4>(a, m, g, s) : launch_one<SCHEME, false, 1, 8>(a, m, g, s);
}

/* Q8_0 / Q6_K: bf16 activations only (T0 takes no f32 activations; the f32
 * GEMV form exists for configs[0]'s Q4_K case). */
template <int SCHEME>
int launch_scheme_split(const GemvArgs &a, uint32_t m, int spl, uint32_t g, hipStream_t s) {
    return spl == 2 ? launch_one<SCHEME, false, 2, 4>(a, m, g, s) : launch_one<SCHEME, false, 1, 8>(a, m, g, s);
}

}  // namespace

/* m <= 8 rows, K % 256 == 0.  Rows of x are x_row_stride elements apart. */
int r9vx_launch_gemv(const r9vx_gemv_problem &p, hipStream_t stream) {
    const uint32_t cpr = p.k / 32; /* 16-byte chunks per row, a multiple of 8 */
    /* Two chunks per lane when a row has >= 128 chunks and the activation
     * registers fit (M rows x 2 chunks).  This choice, the rows per lane
     * group, the activation staging and the streaming form for m = 1 follow
     * m, but none of them changes a row's arithmetic: a lane always owns the chunks lir, lir + 64, ... of
     * every row and adds them in that order (two per segment or one), and the
     * cross-lane sum over the 64 lanes is the same tree for every value, so
     * a row's outputs are the same bits for every m of a bucket <= 8. */
    int spl = (cpr % 128 == 0 && p.m <= (p.x_dtype == R9VX_DTYPE_F32 ? 2u : 4u)) ? 2 : 1;
    uint32_t lpr = 64;
    while (lpr > 8 && (cpr / spl) % lpr) lpr >>= 1;
    if ((cpr / spl) < lpr) lpr = cpr / spl;
    uint32_t lpr_log2 = 0;
    while ((1u << lpr_log2) < lpr) ++lpr_log2;
    GemvArgs a;
    a.w = p.w;
    a.ws = p.w_scales;
    a.ws_row = p.scheme == R9VX_SCHEME_Q8_0 ? p.k / 32 : p.k / 256;
    a.x = p.x;
    a.bias = p.bias;
    a.residual = p.residual;
    a.y = p.y;
    a.w_row_stride = p.w_row_stride;
    a.x_row_stride = p.x_row_stride;
    a.n = p.n;
    a.k = p.k;
    a.lpr_log2 = lpr_log2;
    a.nseg = cpr / (lpr * spl);
    a.y_bf16 = p.y_dtype == R9VX_DTYPE_BF16;
    a.epilogue = p.epilogue;
    const uint32_t groups = 64 / lpr;
    const bool xf32 = p.x_dtype == R9VX_DTYPE_F32;
    if (p.epilogue == R9VX_EPILOGUE_SWIGLU) {
        if (xf32) return (int)hipErrorInvalidValue;
        switch (p.scheme) {
        case R9VX_SCHEME_Q4_K: return launch_gated_scheme<R9VX_SCHEME_Q4_K>(a, p.m, spl, groups, stream);
        case R9VX_SCHEME_IQ4_XS: return launch_gated_scheme<R9VX_SCHEME_IQ4_XS>(a, p.m, spl, groups, stream);
        case R9VX_SCHEME_Q6_K: return launch_gated_scheme<R9VX_SCHEME_Q6_K>(a, p.m, spl, groups, stream);
        case R9VX_SCHEME_IQ3_S: return launch_gated_scheme<R9VX_SCHEME_IQ3_S>(a, p.m, spl, groups, stream);
        default: return launch_gated_scheme<R9VX_SCHEME_Q8_0>(a, p.m, spl, groups, stream);
        }
    }
    if (p.scheme == R9VX_SCHEME_Q4_K) return launch_scheme<R9VX_SCHEME_Q4_K>(a, p.m, xf32, spl, groups, stream);
    if (p.scheme == R9VX_SCHEME_IQ4_XS) return launch_scheme<R9VX_SCHEME_IQ4_XS>(a, p.m, xf32, spl, groups, stream);
    if (xf32) return (int)hipErrorInvalidValue;
    if (p.scheme == R9VX_SCHEME_Q6_K) return launch_scheme_split<R9VX_SCHEME_Q6_K>(a, p.m, spl, groups, stream);
    if (p.scheme == R9VX_SCHEME_IQ3_S) return launch_scheme_split<R9VX_SCHEME_IQ3_S>(a, p.m, spl, groups, stream);
    return launch_scheme_split<R9VX_SCHEME_Q8_0>(a, p.m, spl, groups, stream);
}
