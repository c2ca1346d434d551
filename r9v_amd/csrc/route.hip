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
 * renormalisation, in a device status word; the compute pass writes nothing
 * when the word is set.  T <= 8 runs both passes in one workgroup, one wave per row.
 */
#include "r9vx_device.h"
#include "r9vx_expf.h"
#include "r9vx_internal.h"

namespace {

__device__ uint32_t g_route_status;

constexpr int kMaxPerLane = 16; /* E <= 1024 */
constexpr int kMaxK = 32;

struct RouteArgs {
    const float *logits;
    const float *bias;
    uint32_t *ids;
    float *weights;
    uint32_t t, e, k, scoring, renormalize;
    float scale;
};

__device__ __forceinline__ float wave_max(float v) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    for (int off = 32; off > 0; off >>= 1) {
        uint64_t o = __shfl_xor(v, off, 64);
        v = o > v ? o : v;
    }
    return v;
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
 * lane c % 64 in register c / 64.  Every lane runs the same chain: each term
 * is broadcast with readlane, so the order and the roundings are exactly the
 * reference's sequential loop. */
__device__ __forceinline__ float ordered_sum(const float (&v)[kMaxPerLane], uint32_t e) {
    /* a rotating copy keeps the register index static while the outer loop
     * stays rolled (64 broadcasts per iteration, not 64 * 16) */
    float q[kMaxPerLane];
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) q[i] = v[i];
    float sum = 0.0f;
    for (uint32_t base = 0; base < e; base += 64) {
        const int bits = __builtin_bit_cast(int, q[0]);
        if (base + 64 <= e) {
#pragma unroll
            for (int l = 0; l < 64; ++l) sum = sum + __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, l));
        } else {
            for (uint32_t l = 0; l < e - base; ++l)
                sum = sum + __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, (int)l));
        }
#pragma unroll
        for (int i = 0; i + 1 < kMaxPerLane; ++i) q[i] = q[i + 1];
    }
    return sum;
}

__device__ __forceinline__ void route_row(const RouteArgs &a, uint32_t row, uint32_t lane) {
    const uint32_t per = (a.e + 63) / 64;
    float sc[kMaxPerLane];
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
        uint32_t c = lane + 64 * i;
        float s = -__builtin_huge_valf();
        if (i < (int)per && c < a.e) {
            s = a.logits[(uint64_t)row * a.e + c];
            if (a.bias) s = s + a.bias[c];
        }
        sc[i] = s;
    }
    if (a.scoring == R9VX_SCORING_SOFTMAX) {
        float mx = -__builtin_huge_valf();
#pragma unroll
        for (int i = 0; i < kMaxPerLane; ++i) mx = fmaxf(mx, sc[i]);
        mx = wave_max(mx);
#pragma unroll
        for (int i = 0; i < kMaxPerLane; ++i) {
            uint32_t c = lane + 64 * i;
            sc[i] = (i < (int)per && c < a.e) ? r9vx_expf(sc[i] - mx) : 0.0f;
        }
        const float sum = ordered_sum(sc, a.e);
#pragma unroll
        for (int i = 0; i < kMaxPerLane; ++i) {
            uint32_t c = lane + 64 * i;
            if (i < (int)per && c < a.e) sc[i] = sc[i] / sum;
        }
    } else {
#pragma unroll
        for (int i = 0; i < kMaxPerLane; ++i) {
            uint32_t c = lane + 64 * i;
            if (i < (int)per && c < a.e) sc[i] = 1.0f / (1.0f + r9vx_expf(-sc[i]));
        }
    }
    /* Top-K: the composite key (score order, ~id) makes every candidate
     * distinct, so a wave max picks exactly the reference's next element. */
    uint32_t my_id = 0;
    float my_w = 0.0f;
    float selected_sum = 0.0f;
    uint32_t taken = 0; /* bit i: element lane+64i already selected */
    for (uint32_t j = 0; j < a.k; ++j) {
        uint64_t best = 0;
#pragma unroll
        for (int i = 0; i < kMaxPerLane; ++i) {
            uint32_t c = lane + 64 * i;
            if (i < (int)per && c < a.e && !((taken >> i) & 1u)) {
                uint64_t key = ((uint64_t)total_order(sc[i]) << 32) | (uint64_t)(0xFFFFFFFFu - c);
                best = key > best ? key : best;
            }
        }
        best = wave_max_u64(best);
        uint32_t col = 0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFu);
        if ((col & 63u) == lane) taken |= 1u << (col >> 6);
        float score = __builtin_bit_cast(float, (uint32_t)(best >> 32) & 0x80000000u
                                                    ? (uint32_t)(best >> 32) & 0x7FFFFFFFu
                                                    : ~(uint32_t)(best >> 32));
        float w = score * a.scale;
        selected_sum = selected_sum + w;
        if (lane == j) {
            my_id = col;
            my_w = w;
        }
    }
    if (a.renormalize) my_w = my_w / selected_sum;
    if (lane < a.k) {
        a.ids[(uint64_t)row * a.k + lane] = my_id;
        a.weights[(uint64_t)row * a.k + lane] = my_w;
    }
}

__global__ void clear_status_kernel() { g_route_status = 0u; }

__global__ __launch_bounds__(256) void route_check_kernel(RouteArgs a) {
    uint32_t lane = threadIdx.x & 63;
    uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.t) return;
    uint32_t bad = check_row(a, row, lane);
    if (bad && lane == 0) atomicOr(&g_route_status, bad);
}

/* Grid-wide form: runs after route_check_kernel. */
__global__ __launch_bounds__(256) void route_kernel(RouteArgs a) {
    uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    uint32_t row = blockIdx.x * 4 + wv;
    if (row >= a.t) return;
    if (__atomic_load_n(&g_route_status, __ATOMIC_RELAXED) != 0u) return;
    route_row(a, row, lane);
}

/* Single-workgroup form for small T: check every row, then compute. */
__global__ __launch_bounds__(512) void route_small_kernel(RouteArgs a) {
    __shared__ uint32_t bad_all;
    uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if (threadIdx.x == 0) bad_all = 0;
    __syncthreads();
    for (uint32_t row = wv; row < a.t; row += nw) {
        uint32_t bad = check_row(a, row, lane);
        if (bad && lane == 0) atomicOr(&bad_all, bad);
    }
    __syncthreads();
    uint32_t bad = bad_all;
    if (threadIdx.x == 0) g_route_status = bad;
    if (bad) return;
    for (uint32_t row = wv; row < a.t; row += nw) route_row(a, row, lane);
}

}  // namespace

int r9vx_launch_route(const r9vx_route_problem &p, hipStream_t stream) {
    RouteArgs a{p.logits, p.bias, p.ids, p.weights, p.t, p.e, p.k, p.scoring, p.renormalize, p.scale};
    if (p.t <= 8) {
        uint32_t waves = p.t;
        hipLaunchKernelGGL(route_small_kernel, dim3(1), dim3(64 * waves), 0, stream, a);
        return (int)hipGetLastError();
    }
    hipLaunchKernelGGL(clear_status_kernel, dim3(1), dim3(1), 0, stream);
    dim3 grid((p.t + 3) / 4);
    hipLaunchKernelGGL(route_check_kernel, grid, dim3(256), 0, stream, a);
    hipLaunchKernelGGL(route_kernel, grid, dim3(256), 0, stream, a);
    return (int)hipGetLastError();
}

int r9vx_read_route_status(uint32_t *status, hipStream_t stream) {
    int rc = (int)hipMemcpyFromSymbolAsync(status, HIP_SYMBOL(g_route_status), sizeof(uint32_t), 0,
                                           hipMemcpyDeviceToHost, stream);
    if (rc) return rc;
    rc = (int)hipStreamSynchronize(stream);
    if (rc) return rc;
    hipLaunchKernelGGL(clear_status_kernel, dim3(1), dim3(1), 0, stream);
    return (int)hipGetLastError();
}
