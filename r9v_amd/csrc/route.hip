/*
 * route.hip -- moe_route on the GPU, bit-exact with T0
 * (crates/r9v-t0/src/moe_route.rs:312-418).
 *
 * One wave per token row.  Every f32 operation of the reference is repeated
 * in the same order with the same rounding:
 *   s = logit (+ bias)                                   (:320-328)
 *   softmax: max; v = exp(s - max) with r9vx_expf (bit-identical to the host
 *   glibc expf that Rust f32::exp calls); sum of v in ascending expert order
 *   by a single lane; score = v / sum (IEEE divide)       (:331-346)
 *   sigmoid: 1 / (1 + exp(-s))                            (:347-351)
 *   top-K by (score desc under total_cmp, id asc)         (:372-373)
 *   w = score * scale, running f32 sum in selection order, w / sum (:374-398)
 * The max and the top-K selection are order-independent, so they use wave
 * reductions; the one order-dependent sum runs sequentially.
 *
 * Refusal before mutation (:313-418): a check pass flags non-finite logits,
 * bias or post-bias scores, and a zero selected sum under sigmoid
 * renormalisation, in the launch's status word; the compute pass writes
 * nothing when the word is set.  The word is the caller's (the _ex launch),
 * the workspace's (routing from hidden states) or, for the plain launch, one
 * library word per device.  T <= 8 runs both passes in one workgroup, one wave per row.
 */
#include <map>
#include <mutex>

#include "r9vx_device.h"
#include "r9vx_expf.h"
#include "r9vx_internal.h"

namespace {

/* The status words of plain r9vx_moe_route_launch calls on this device: one
 * per stream that has made such a call (slot assigned on the stream's first
 * call, at most kRouteStreamWords streams per device). */
constexpr uint32_t kRouteStreamWords = 64;
__device__ uint32_t g_route_status[kRouteStreamWords];

constexpr int kMaxK = 32;

struct RouteArgs {
    const float *logits;
    const float *bias;
    uint32_t *ids;
    float *weights;
    uint32_t *status; /* this launch's status word */
    uint32_t t, e, k, scoring, renormalize;
    float scale;
};

/* Wave-wide max without LDS: a DPP butterfly inside each 16-lane row (row
 * mirror, half-row mirror, quad reversal, quad pair swap), then the gfx950
 * permlane swaps pair rows 0/1, 2/3 and halves 0/1.  Every lane ends with
 * the result. */
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ void swap_halves16(uint32_t x, uint32_t &a, uint32_t &b) {
    auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    a = r[0];
    b = r[1];
}
__device__ __forceinline__ void swap_halves32(uint32_t x, uint32_t &a, uint32_t &b) {
    auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    a = r[0];
    b = r[1];
}

__device__ __forceinline__ float wave_max(float v) {
    uint32_t x = __builtin_bit_cast(uint32_t, v);
#define R9VX_FMAX_STEP(CTRL) x = __builtin_bit_cast(uint32_t, fmaxf(__builtin_bit_cast(float, x), \
                                                               __builtin_bit_cast(float, dpp_u32<CTRL>(x))))
    R9VX_FMAX_STEP(0x140);
    R9VX_FMAX_STEP(0x141);
    R9VX_FMAX_STEP(0x1B);
    R9VX_FMAX_STEP(0xB1);
#undef R9VX_FMAX_STEP
    uint32_t a, b;
    swap_halves16(x, a, b);
    x = __builtin_bit_cast(uint32_t, fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b)));
    swap_halves32(x, a, b);
    return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}

/* total_cmp order key of a float as an unsigned integer (larger = greater). */
__device__ __forceinline__ uint32_t total_order(float v) {
    uint32_t b = __builtin_bit_cast(uint32_t, v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

/* Status bits for one row (0 = valid). */
__device__ __forceinline__ uint32_t check_row(const RouteArgs &a, uint32_t row, uint32_t lane) {
    uint32_t bad = 0;
    float smax = -__builtin_huge_valf();
    for (uint32_t c = lane; c < a.e; c += 64) {
        float l = a.logits[(uint64_t)row * a.e + c];
        float s = l;
        if (a.bias) {
            float b = a.bias[c];
            if (!__builtin_isfinite(b)) bad |= R9VX_STATUS_NONFINITE;
            s = l + b;
        }
        if (!__builtin_isfinite(l) || !__builtin_isfinite(s)) bad |= R9VX_STATUS_NONFINITE;
        smax = fmaxf(smax, s);
    }
    /* sigmoid + renormalise: the K selected scores are all zero exactly when
     * the largest score 1/(1+exp(-smax)) is zero. */
    if (a.scoring == R9VX_SCORING_SIGMOID && a.renormalize) {
        smax = wave_max(smax);
        float top = 1.0f / (1.0f + r9vx_expf(-smax));
        if (top == 0.0f) bad |= R9VX_STATUS_DEGENERATE;
    }
    for (int off = 32; off > 0; off >>= 1) bad |= __shfl_xor(bad, off, 64);
    return bad;
}

/* sum_{c=0}^{E-1} v[c] in ascending c with one f32 accumulator, v[c] held by
 * lane c % 64 in register c / 64.  The wave stores the values to its LDS
 * slice in column order and every lane then runs the same sequential chain
 * over broadcast LDS reads, so the order and the roundings are exactly the
 * reference's loop. */
template <int PER>
__device__ __forceinline__ float ordered_sum(const float (&v)[PER], uint32_t e, uint32_t lane, float *buf) {
    /* columns past E hold +0.0, which leaves a sum of values >= 0 bit for
     * bit unchanged, so the chain has a compile-time length and its LDS reads
     * can run ahead of the adds (eight quads per unrolled group) */
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const uint32_t c = lane + 64 * i;
        buf[c] = c < e ? v[i] : 0.0f;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const r9vx_f32x4 *b4 = reinterpret_cast<const r9vx_f32x4 *>(buf);
    float sum = 0.0f;
#pragma unroll 8
    for (int q = 0; q < PER * 16; ++q) {
        const r9vx_f32x4 x = b4[q];
        sum = sum + x.x;
        sum = sum + x.y;
        sum = sum + x.z;
        sum = sum + x.w;
    }
    return sum;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
#define R9VX_UMAX32_STEP(CTRL) x = max(x, dpp_u32<CTRL>(x))
    R9VX_UMAX32_STEP(0x140);
    R9VX_UMAX32_STEP(0x141);
    R9VX_UMAX32_STEP(0x1B);
    R9VX_UMAX32_STEP(0xB1);
#undef R9VX_UMAX32_STEP
    uint32_t a, b;
    swap_halves16(x, a, b);
    x = max(a, b);
    swap_halves32(x, a, b);
    return max(a, b);
}

/* Lane `lane` holds s[c] for c = lane + 64 i (i < PER, E <= 64 PER); -inf
 * past E.  The loads are unconditional (clamped column) so that all of them
 * are in flight at once; the bias branch is uniform. */
/* Device-coherent load (agent scope, past this CU's L1): the fused router
 * reads logits that other workgroups wrote. */
__device__ __forceinline__ float ld_coherent(const float *p) {
    return __builtin_bit_cast(float, __hip_atomic_load(reinterpret_cast<uint32_t *>(const_cast<float *>(p)),
                                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

template <int PER, bool COH = false>
__device__ __forceinline__ void load_row(const RouteArgs &a, uint32_t row, uint32_t lane, float (&sc)[PER],
                                         float (&lg)[PER], float (&bs)[PER]) {
    const float *lrow = a.logits + (uint64_t)row * a.e;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const uint32_t c = lane + 64 * i;
        lg[i] = COH ? ld_coherent(lrow + (c < a.e ? c : a.e - 1)) : lrow[c < a.e ? c : a.e - 1];
    }
    if (a.bias) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const uint32_t c = lane + 64 * i;
            bs[i] = a.bias[c < a.e ? c : a.e - 1];
        }
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const uint32_t c = lane + 64 * i;
        if (!a.bias) bs[i] = 0.0f;
        sc[i] = c < a.e ? (a.bias ? lg[i] + bs[i] : lg[i]) : -__builtin_huge_valf();
        if (c >= a.e) lg[i] = bs[i] = 0.0f;
    }
}

/* Status bits of one loaded row (the tests of check_row). */
template <int PER>
__device__ __forceinline__ uint32_t check_loaded(const RouteArgs &a, uint32_t lane, const float (&sc)[PER],
                                                 const float (&lg)[PER], const float (&bs)[PER],
                                                 const uint64_t *etab) {
    uint32_t bad = 0;
    float smax = -__builtin_huge_valf();
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const uint32_t c = lane + 64 * i;
        if (c < a.e) {
            if (!__builtin_isfinite(lg[i]) || !__builtin_isfinite(bs[i]) || !__builtin_isfinite(sc[i]))
                bad |= R9VX_STATUS_NONFINITE;
            smax = fmaxf(smax, sc[i]);
        }
    }
    if (a.scoring == R9VX_SCORING_SIGMOID && a.renormalize) {
        smax = wave_max(smax);
        float top = 1.0f / (1.0f + r9vx_expf_tab(-smax, etab));
        if (top == 0.0f) bad |= R9VX_STATUS_DEGENERATE;
    }
    return bad;
}

/* The n largest of v (lane l holds v[c] for c = l + 64 i) in the
 * reference's order: descending score, ties to the smaller column.  Lane
 * j < n returns the j-th (column, score).  The composite key (score order,
 * ~column) makes every candidate distinct, so a wave max picks exactly the
 * reference's next element.  Each lane sorts its PER keys once (descending,
 * Batcher's odd-even merge network); a round takes the wave max of the lanes'
 * first keys and the winning lane drops its first key.  A padding slot or an
 * exhausted lane holds 0, below every valid key (scores are >= 0, whose
 * order keys are >= 0x80000000).  The wave max runs on the score half; the
 * column half is needed only when several lanes tie on it.  n <= E. */
template <int PER>
__device__ __forceinline__ void select_top(const float (&v)[PER], uint32_t e, uint32_t n, uint32_t lane,
                                           uint32_t &my_col, float &my_v) {
    uint64_t key[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const uint32_t c = lane + 64 * i;
        key[i] = c < e ? ((uint64_t)total_order(v[i]) << 32) | (uint64_t)(0xFFFFFFFFu - c) : 0;
    }
#pragma unroll
    for (int p = 1; p < PER; p *= 2)
#pragma unroll
        for (int k = p; k >= 1; k /= 2)
#pragma unroll
            for (int j = k % p; j + k < PER; j += 2 * k)
#pragma unroll
                for (int i = 0; i < k && i + j + k < PER; ++i)
                    if ((i + j) / (2 * p) == (i + j + k) / (2 * p)) {
                        const uint64_t x = key[i + j], y = key[i + j + k];
                        key[i + j] = x > y ? x : y;
                        key[i + j + k] = x > y ? y : x;
                    }
    my_col = 0;
    my_v = 0.0f;
    for (uint32_t j = 0; j < n; ++j) {
        const uint32_t bh = (uint32_t)(key[0] >> 32), bl = (uint32_t)key[0];
        const uint32_t mh = wave_max_u32(bh);
        const uint64_t tied = __ballot(bh == mh);
        uint32_t ml;
        if ((tied & (tied - 1)) == 0)
            ml = (uint32_t)__builtin_amdgcn_readlane((int)bl, (int)__builtin_ctzll(tied));
        else
            ml = wave_max_u32(bh == mh ? bl : 0u);
        if (bh == mh && bl == ml) { /* the winning lane */
#pragma unroll
            for (int i = 0; i + 1 < PER; ++i) key[i] = key[i + 1];
            key[PER - 1] = 0;
        }
        if (lane == j) {
            my_col = 0xFFFFFFFFu - ml;
            my_v = __builtin_bit_cast(float, (mh & 0x80000000u) ? (mh & 0x7FFFFFFFu) : ~mh);
        }
    }
}

/* Weights of the K selections (lane j < K holds the j-th score): w = score *
 * scale, renormalised by their sum taken in selection order. */
__device__ __forceinline__ float select_weight(const RouteArgs &a, uint32_t lane, float score) {
    const float w = score * a.scale;
    if (!a.renormalize) return w;
    float selected_sum = 0.0f;
    for (uint32_t j = 0; j < a.k; ++j)
        selected_sum = selected_sum + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), (int)j));
    return w / selected_sum;
}

/* Softmax numerators of one loaded row: sc <- exp(sc - max) (padding holds
 * -inf: exp(-inf - max) = 0). */
template <int PER>
__device__ __forceinline__ void softmax_exp(float (&sc)[PER], const uint64_t *etab) {
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int i = 0; i < PER; ++i) mx = fmaxf(mx, sc[i]);
    mx = wave_max(mx);
#pragma unroll
    for (int i = 0; i < PER; ++i) sc[i] = r9vx_expf_tab_nb(sc[i] - mx, etab);
}

/* Scores, top-K and weights of one loaded row; lane j < K returns the j-th
 * selection in (id, w). */
template <int PER>
__device__ __forceinline__ void route_loaded(const RouteArgs &a, uint32_t lane, float (&sc)[PER],
                                             const uint64_t *etab, float *buf, uint32_t &my_id, float &my_w) {
    if (a.scoring == R9VX_SCORING_SOFTMAX) {
        softmax_exp<PER>(sc, etab);
        const float sum = ordered_sum<PER>(sc, a.e, lane, buf);
#pragma unroll
        for (int i = 0; i < PER; ++i) sc[i] = sc[i] / sum;
    } else {
#pragma unroll
        for (int i = 0; i < PER; ++i) sc[i] = 1.0f / (1.0f + r9vx_expf_tab_nb(-sc[i], etab));
    }
    float score;
    select_top<PER>(sc, a.e, a.k, lane, my_id, score);
    my_w = select_weight(a, lane, score);
}

__global__ void clear_status_kernel(uint32_t *status) { *status = 0u; }

__global__ __launch_bounds__(256) void route_check_kernel(RouteArgs a) {
    uint32_t lane = threadIdx.x & 63;
    uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.t) return;
    uint32_t bad = check_row(a, row, lane);
    if (bad && lane == 0) atomicOr(a.status, bad);
}

/* Grid-wide form: runs after route_check_kernel. */
template <int PER>
__global__ __launch_bounds__(256) void route_kernel(RouteArgs a) {
    __shared__ uint64_t etab[R9VX_EXP2F_N];
    __shared__ __attribute__((aligned(16))) float sbuf[4][PER * 64];
    r9vx_exp2_fill(etab, threadIdx.x, blockDim.x);
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t row = blockIdx.x * 4 + wv;
    if (row >= a.t) return;
    if (__atomic_load_n(a.status, __ATOMIC_RELAXED) != 0u) return;
    float sc[PER], lg[PER], bs[PER];
    load_row<PER>(a, row, lane, sc, lg, bs);
    uint32_t id;
    float w;
    route_loaded<PER>(a, lane, sc, etab, sbuf[wv], id, w);
    if (lane < a.k) {
        a.ids[(uint64_t)row * a.k + lane] = id;
        a.weights[(uint64_t)row * a.k + lane] = w;
    }
}

/* Small-T form: one workgroup of four waves per row.  Softmax: waves 0 and
 * 1 compute the row's exp(s - max); wave 0 takes the ordered sum while wave 1
 * selects the K + 1 largest numerators (the quotients p = e / sum have the
 * same order unless two of them round to the same p), then wave 1 divides
 * its K + 1 selections by the sum: if the K + 1 quotients strictly
 * decrease, the numerators' order is the reference's and its K selections
 * stand; otherwise (equal or one-ulp-apart numerators whose quotients round
 * equal) wave 1 divides every value and selects on the quotients.  Sigmoid
 * scores need no sum: wave 1 routes alone.  The batch-level refusal (no row
 * is written if any row is bad): every workgroup checks every row, on its
 * waves 2 and 3 (alternate rows, all their loads in flight at once) while
 * waves 0 and 1 route, so the rows' workgroups run on separate CUs without
 * talking to each other; workgroup 0 writes the status word. */
constexpr uint32_t kRouteSmallT = 8;

template <int PER>
struct CheckRows {
    static constexpr int R = kRouteSmallT / 2;
    float lg[R][PER], bs[PER];
    /* rows first, first + 2, ... (< T) and the bias: loads only */
    __device__ __forceinline__ void load(const RouteArgs &a, uint32_t first, uint32_t lane) {
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const uint32_t r = first + 2 * j < a.t ? first + 2 * j : 0u; /* rows past T: row 0, unused */
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const uint32_t c = lane + 64 * i;
                lg[j][i] = a.logits[(uint64_t)r * a.e + (c < a.e ? c : a.e - 1)];
            }
        }
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const uint32_t c = lane + 64 * i;
            bs[i] = a.bias ? a.bias[c < a.e ? c : a.e - 1] : 0.0f;
        }
    }
    /* the rows' status bits, or-ed */
    __device__ __forceinline__ uint32_t check(const RouteArgs &a, uint32_t first, uint32_t lane,
                                              const uint64_t *etab) const {
        uint32_t bad = 0;
#pragma unroll
        for (int j = 0; j < R; ++j) {
            if (first + 2 * j >= a.t) break;
            float sc[PER], l[PER], b[PER];
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const uint32_t c = lane + 64 * i;
                sc[i] = c < a.e ? (a.bias ? lg[j][i] + bs[i] : lg[j][i]) : -__builtin_huge_valf();
                l[i] = c < a.e ? lg[j][i] : 0.0f;
                b[i] = c < a.e ? bs[i] : 0.0f;
            }
            const uint32_t bad_row = check_loaded<PER>(a, lane, sc, l, b, etab);
            if (__ballot(bad_row & R9VX_STATUS_NONFINITE)) bad |= R9VX_STATUS_NONFINITE;
            if (__ballot(bad_row & R9VX_STATUS_DEGENERATE)) bad |= R9VX_STATUS_DEGENERATE;
        }
        return bad;
    }
};

template <int PER>
__global__ __launch_bounds__(256) void route_small_kernel(RouteArgs a) {
    __shared__ uint32_t bad_all;
    __shared__ uint64_t etab[R9VX_EXP2F_N];
    __shared__ __attribute__((aligned(16))) float sbuf[PER * 64];
    __shared__ float row_sum;
    const uint32_t lane = threadIdx.x & 63, role = threadIdx.x >> 6, row = blockIdx.x;
    r9vx_exp2_fill(etab, threadIdx.x, blockDim.x);
    if (threadIdx.x == 0) bad_all = 0;
    float sc[PER], lg[PER], bs[PER];
    CheckRows<PER> cr;
    if (role < 2)
        load_row<PER>(a, row, lane, sc, lg, bs);
    else
        cr.load(a, role - 2, lane);
    __syncthreads();
    if (role >= 2) { /* the checking waves */
        const uint32_t bad = cr.check(a, role - 2, lane, etab);
        if (bad && lane == 0) atomicOr(&bad_all, bad);
        __syncthreads();
        return;
    }
    const bool softmax = a.scoring == R9VX_SCORING_SOFTMAX;
    uint32_t id = 0, col = 0;
    float w = 0.0f, ev = 0.0f;
    const uint32_t nsel = a.k < a.e ? a.k + 1 : a.k; /* the K + 1-th decides the boundary */
    if (softmax) {
        softmax_exp<PER>(sc, etab);
        if (role == 0) {
            const float sum = ordered_sum<PER>(sc, a.e, lane, sbuf);
            if (lane == 0) row_sum = sum;
        } else {
            select_top<PER>(sc, a.e, nsel, lane, col, ev);
        }
    }
    __syncthreads();
    const uint32_t bad_batch = bad_all;
    if (row == 0 && threadIdx.x == 0) *a.status = bad_batch;
    if (bad_batch || role == 0) return;
    if (softmax) {
        const float sum = row_sum;
        const float p = ev / sum;
        const float pn = __shfl_down(p, 1, 64);
        if (__ballot(lane + 1 < nsel && !(p > pn)) == 0ull) {
            id = col;
            w = select_weight(a, lane, p);
        } else { /* equal quotients: select on the quotients themselves */
#pragma unroll
            for (int i = 0; i < PER; ++i) sc[i] = sc[i] / sum;
            float score;
            select_top<PER>(sc, a.e, a.k, lane, id, score);
            w = select_weight(a, lane, score);
        }
    } else {
        route_loaded<PER>(a, lane, sc, etab, sbuf, id, w);
    }
    if (lane < a.k) {
        a.ids[(uint64_t)row * a.k + lane] = id;
        a.weights[(uint64_t)row * a.k + lane] = w;
    }
}

/* Routing from hidden states, t <= 8: the router logits x . w_r^T and
 * moe_route in one launch, with every logit accumulated in T0's order (one
 * f32 accumulator, k ascending, each product rounded before it is added:
 * crates/r9v-t0/src/matmul.rs:1940-2414; the library is built with
 * -ffp-contract=off), so the ids and weights equal T0's matmul followed by
 * moe_route bit for bit.  A logit is a sequential sum over K, so the
 * parallelism is one lane per (expert, token): workgroup (bx, t) has its
 * first wave compute experts 64bx .. 64bx+63 of token t.  The router weight
 * is in the k4-interleaved device layout [dm/4][E][4] (r9vx_router_repack),
 * so the 16-byte loads of a wave (4 consecutive K values of 64 consecutive
 * experts) read 1 KiB contiguous, one stage of 32 K values ahead, and x is
 * staged once as f32 in LDS (broadcast reads).  A logit's adds are a
 * dependent chain -- measured 5.45 ns per K value on MI355X (multiply and
 * dependent add), so 11 us per 2048 values whatever the memory system does;
 * deeper weight prefetch (a four-stage ring) measured slower.
 * The last workgroup to finish (a counter in the caller's workspace, left at
 * zero again) routes the whole batch with all four waves and the batch-level
 * refusal of route_small_kernel. */
struct RouteHiddenArgs {
    const uint16_t *x; /* bf16 [t, dm] */
    const float *w;    /* f32 [e, dm] */
    uint32_t *counter; /* workspace word, zero between launches */
    uint32_t dm;       /* a multiple of 64 */
    RouteArgs r;       /* r.logits: the workspace logits [t, e] */
};

constexpr int kRhStage = 8; /* 16-byte weight loads (32 K values) per stage */

/* x values of one stage: f32 read from the token's row in LDS (the same
 * address in every lane: a broadcast read). */
struct RhX {
    r9vx_f32x4 v[kRhStage];
};

__device__ __forceinline__ void rh_load_x(RhX &x, const float *xs) {
#pragma unroll
    for (int i = 0; i < kRhStage; ++i) x.v[i] = *reinterpret_cast<const r9vx_f32x4 *>(xs + 4 * i);
}

__device__ __forceinline__ float rh_stage(float acc, const r9vx_f32x4 (&w)[kRhStage], const RhX &x) {
#pragma unroll
    for (int i = 0; i < kRhStage; ++i) {
        acc = acc + x.v[i].x * w[i].x;
        acc = acc + x.v[i].y * w[i].y;
        acc = acc + x.v[i].z * w[i].z;
        acc = acc + x.v[i].w * w[i].w;
    }
    return acc;
}

/* Stage loads: slab j of the k4 layout holds K values 4j .. 4j+3 of every
 * expert, 4 E floats per slab. */
__device__ __forceinline__ void rh_load(r9vx_f32x4 (&w)[kRhStage], const float *wr, uint64_t slab_floats) {
#pragma unroll
    for (int i = 0; i < kRhStage; ++i) w[i] = *reinterpret_cast<const r9vx_f32x4 *>(wr + slab_floats * i);
}

constexpr uint32_t kRhMaxDm = 8192; /* x row staged in LDS as f32 */

template <int PER>
__global__ __launch_bounds__(256) void route_hidden_kernel(RouteHiddenArgs a) {
    __shared__ __attribute__((aligned(16))) float xs[kRhMaxDm];
    __shared__ uint32_t is_last, bad_all;
    __shared__ uint64_t etab[R9VX_EXP2F_N];
    __shared__ __attribute__((aligned(16))) float sbuf[4][PER * 64];
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t E = a.r.e, T = a.r.t;
    if (wv == 0) {
        const uint32_t e = blockIdx.x * 64 + lane, tok = blockIdx.y;
        const uint64_t slab = 4ull * E; /* floats per 4-K slab */
        const float *wr = a.w + 4ull * (e < E ? e : E - 1);
        r9vx_f32x4 wa[kRhStage], wb[kRhStage];
        rh_load(wa, wr, slab);
        /* the token's x row -> LDS as f32 (exact), while the first weights load */
        const uint16_t *xr = a.x + (uint64_t)tok * a.dm;
        for (uint32_t k = 4 * lane; k < a.dm; k += 256) {
            const r9vx_u32x2 xb = *reinterpret_cast<const r9vx_u32x2 *>(xr + k);
            *reinterpret_cast<r9vx_f32x4 *>(xs + k) =
                r9vx_f32x4{__builtin_bit_cast(float, xb.x << 16), __builtin_bit_cast(float, xb.x & 0xFFFF0000u),
                           __builtin_bit_cast(float, xb.y << 16), __builtin_bit_cast(float, xb.y & 0xFFFF0000u)};
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float acc = 0.0f;
        RhX xa, xb;
        rh_load_x(xa, xs);
        for (uint32_t k = 0; k < a.dm; k += 64) {
            rh_load(wb, wr + slab * ((k + 32) / 4), slab);
            rh_load_x(xb, xs + k + 32);
            acc = rh_stage(acc, wa, xa);
            if (k + 64 < a.dm) {
                rh_load(wa, wr + slab * ((k + 64) / 4), slab);
                rh_load_x(xa, xs + k + 64);
            }
            acc = rh_stage(acc, wb, xb);
        }
        if (e < E) const_cast<float *>(a.r.logits)[(uint64_t)tok * E + e] = acc;
    }
    __threadfence(); /* this workgroup's logits are visible device-wide before it is counted */
    __syncthreads();
    if (threadIdx.x == 0) is_last = atomicAdd(a.counter, 1u) == gridDim.x * gridDim.y - 1;
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    r9vx_exp2_fill(etab, threadIdx.x, blockDim.x);
    if (threadIdx.x == 0) bad_all = 0;
    __syncthreads();
    uint32_t id[2] = {0, 0};
    float w[2] = {0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t row = wv + 4 * j;
        if (row >= T) continue;
        float sc[PER], lg[PER], bs[PER];
        load_row<PER, true>(a.r, row, lane, sc, lg, bs);
        const uint32_t bad_row = check_loaded<PER>(a.r, lane, sc, lg, bs, etab);
        uint32_t bad = 0;
        if (__ballot(bad_row & R9VX_STATUS_NONFINITE)) bad |= R9VX_STATUS_NONFINITE;
        if (__ballot(bad_row & R9VX_STATUS_DEGENERATE)) bad |= R9VX_STATUS_DEGENERATE;
        if (bad && lane == 0) atomicOr(&bad_all, bad);
        if (!bad) route_loaded<PER>(a.r, lane, sc, etab, sbuf[wv], id[j], w[j]);
    }
    __syncthreads();
    const uint32_t bad = bad_all;
    if (threadIdx.x == 0) {
        *a.r.status = bad;
        atomicExch(a.counter, 0u);
    }
    if (bad) return;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t row = wv + 4 * j;
        if (row < T && lane < a.r.k) {
            a.r.ids[(uint64_t)row * a.r.k + lane] = id[j];
            a.r.weights[(uint64_t)row * a.r.k + lane] = w[j];
        }
    }
}

}  // namespace

/* [E, dm] -> k4-interleaved [dm/4][E][4]: thread per (slab, expert). */
__global__ __launch_bounds__(256) void router_repack_kernel(const float *__restrict__ w, uint32_t e, uint32_t dm,
                                                            float *__restrict__ out) {
    const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (uint64_t)e * (dm / 4)) return;
    const uint32_t ex = (uint32_t)(gid % e), j = (uint32_t)(gid / e);
    *reinterpret_cast<r9vx_f32x4 *>(out + 4 * gid) =
        *reinterpret_cast<const r9vx_f32x4 *>(w + (uint64_t)ex * dm + 4 * j);
}

int r9vx_launch_router_repack(const float *w, uint32_t e, uint32_t dm, float *out, hipStream_t stream) {
    const uint64_t n = (uint64_t)e * (dm / 4);
    hipLaunchKernelGGL(router_repack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, w, e, dm, out);
    return (int)hipGetLastError();
}

int r9vx_launch_route_hidden(const r9vx_route_hidden_problem &p, hipStream_t stream) {
    RouteHiddenArgs a{p.x, p.w, p.counter, p.dm,
                      RouteArgs{p.logits, p.bias, p.ids, p.weights, p.status, p.t, p.e, p.k, p.scoring, p.renormalize,
                                p.scale}};
    const dim3 grid((p.e + 63) / 64, p.t);
    const uint32_t per = (p.e + 63) / 64;
    if (per <= 1)
        hipLaunchKernelGGL((route_hidden_kernel<1>), grid, dim3(256), 0, stream, a);
    else if (per <= 2)
        hipLaunchKernelGGL((route_hidden_kernel<2>), grid, dim3(256), 0, stream, a);
    else if (per <= 4)
        hipLaunchKernelGGL((route_hidden_kernel<4>), grid, dim3(256), 0, stream, a);
    else if (per <= 8)
        hipLaunchKernelGGL((route_hidden_kernel<8>), grid, dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL((route_hidden_kernel<16>), grid, dim3(256), 0, stream, a);
    return (int)hipGetLastError();
}

template <int PER>
static int launch_route_per(const RouteArgs &a, hipStream_t stream) {
    if (a.t <= kRouteSmallT) {
        hipLaunchKernelGGL((route_small_kernel<PER>), dim3(a.t), dim3(256), 0, stream, a);
        return (int)hipGetLastError();
    }
    hipLaunchKernelGGL(clear_status_kernel, dim3(1), dim3(1), 0, stream, a.status);
    dim3 grid((a.t + 3) / 4);
    hipLaunchKernelGGL(route_check_kernel, grid, dim3(256), 0, stream, a);
    hipLaunchKernelGGL((route_kernel<PER>), grid, dim3(256), 0, stream, a);
    return (int)hipGetLastError();
}

/* The plain-launch status word of `stream` on the current device: the
 * device array's address is looked up once per device, and a stream gets
 * the next free slot on its first call.  nullptr with *err set when the
 * device cannot be queried, or with *full set when every slot is taken. */
static std::mutex g_word_mu;
static uint32_t *g_words[64];
static std::map<hipStream_t, uint32_t> g_word_slot[64];

static uint32_t *stream_status_word(hipStream_t stream, bool assign, hipError_t *err, bool *full) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess && (dev < 0 || dev >= 64)) e = hipErrorInvalidDevice;
    if (e != hipSuccess) {
        *err = e;
        return nullptr;
    }
    std::lock_guard<std::mutex> g(g_word_mu);
    if (!g_words[dev]) {
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(g_route_status));
        if (e != hipSuccess || !ptr) {
            *err = e != hipSuccess ? e : hipErrorInvalidSymbol;
            return nullptr;
        }
        g_words[dev] = static_cast<uint32_t *>(ptr);
    }
    auto &slots = g_word_slot[dev];
    auto it = slots.find(stream);
    if (it != slots.end()) return g_words[dev] + it->second;
    if (!assign) return nullptr; /* no plain launch on this stream yet */
    if (slots.size() >= kRouteStreamWords) {
        *full = true;
        return nullptr;
    }
    const uint32_t slot = (uint32_t)slots.size();
    slots.emplace(stream, slot);
    return g_words[dev] + slot;
}

uint32_t r9vx_route_stream_words() { return kRouteStreamWords; }

int r9vx_launch_route(const r9vx_route_problem &p, hipStream_t stream, bool *no_word) {
    hipError_t err = hipSuccess;
    bool full = false;
    uint32_t *status = p.status ? p.status : stream_status_word(stream, true, &err, &full);
    if (!status) {
        if (full && no_word) *no_word = true;
        return full ? (int)hipErrorOutOfMemory : (int)err;
    }
    RouteArgs a{p.logits, p.bias, p.ids, p.weights, status, p.t, p.e, p.k, p.scoring, p.renormalize, p.scale};
    /* registers per lane: the next power of two >= ceil(E / 64) */
    const uint32_t per = (p.e + 63) / 64;
    if (per <= 1) return launch_route_per<1>(a, stream);
    if (per <= 2) return launch_route_per<2>(a, stream);
    if (per <= 4) return launch_route_per<4>(a, stream);
    if (per <= 8) return launch_route_per<8>(a, stream);
    return launch_route_per<16>(a, stream);
}

int r9vx_read_route_status(uint32_t *status, hipStream_t stream) {
    hipError_t err = hipSuccess;
    bool full = false;
    uint32_t *word = stream_status_word(stream, false, &err, &full);
    if (!word) {
        if (err != hipSuccess) return (int)err;
        *status = 0u; /* no plain launch on this stream: nothing refused */
        return (int)hipStreamSynchronize(stream);
    }
    int rc = (int)hipMemcpyAsync(status, word, sizeof(uint32_t), hipMemcpyDeviceToHost, stream);
    if (rc) return rc;
    rc = (int)hipStreamSynchronize(stream);
    if (rc) return rc;
    hipLaunchKernelGGL(clear_status_kernel, dim3(1), dim3(1), 0, stream, word);
    return (int)hipGetLastError();
}
