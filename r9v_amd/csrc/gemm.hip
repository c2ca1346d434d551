/*
 * gemm.hip -- prefill dequant-GEMM on MFMA: y[m, n] = sum_k x[m, k] * w[n, k]
 * for bf16 activations (m > 8) and GGUF Q4_K / IQ4_XS weights.
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
 *     other LDS buffer.  Workgroups are mapped so that each XCD owns a
 *     contiguous band of weight columns: the 8 M-tiles that reuse a weight
 *     tile run on the same XCD and hit its L2.
 */
#include "r9vx_mfma.h"

using namespace r9vx;

namespace {

struct GemmArgs {
    const _Float16 *x16;
    const float *scale;
    const uint8_t *w;
    const float *bias;
    const float *residual;
    void *y;
    uint64_t w_row_stride;
    uint32_t m, n, k;
    uint32_t m_tiles, n_tiles;
    uint32_t y_bf16, epilogue;
};

__global__ __launch_bounds__(256) void x_to_f16_kernel(const uint16_t *__restrict__ x, uint32_t k,
                                                       _Float16 *__restrict__ x16, float *__restrict__ scale) {
    __shared__ float red[4];
    const uint32_t row = blockIdx.x;
    const uint16_t *xr = x + (uint64_t)row * k;
    float mx = 0.f;
    for (uint32_t c = threadIdx.x * 8; c < k; c += 256 * 8) {
        r9vx_u32x4 v = *reinterpret_cast<const r9vx_u32x4 *>(xr + c);
        uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            mx = fmaxf(mx, fabsf(__builtin_bit_cast(float, w[i] << 16)));
            mx = fmaxf(mx, fabsf(__builtin_bit_cast(float, w[i] & 0xFFFF0000u)));
        }
    }
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const int e = row_shift(mx);
    const float inv = ldexpf(1.0f, -e);
    if (threadIdx.x == 0) scale[row] = ldexpf(1.0f, e);
    _Float16 *orow = x16 + (uint64_t)row * k;
    for (uint32_t c = threadIdx.x * 8; c < k; c += 256 * 8) {
        r9vx_u32x4 v = *reinterpret_cast<const r9vx_u32x4 *>(xr + c);
        uint32_t w[4] = {v.x, v.y, v.z, v.w};
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            o[i] = pack_h2(__builtin_bit_cast(float, w[i] << 16) * inv,
                           __builtin_bit_cast(float, w[i] & 0xFFFF0000u) * inv);
        *reinterpret_cast<r9vx_u32x4 *>(orow + c) = r9vx_u32x4{o[0], o[1], o[2], o[3]};
    }
}

template <int SCHEME>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[2][2][kStageHalfs * 2];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t wm = wave & 1, wn = wave >> 1;

    /* XCD-aware tile order: workgroup b runs on XCD b % 8. */
    const uint32_t total = a.m_tiles * a.n_tiles;
    uint32_t t = blockIdx.x;
    if (total % 8 == 0) t = (blockIdx.x % 8) * (total / 8) + blockIdx.x / 8;
    const uint32_t n_tile = t / a.m_tiles, m_tile = t % a.m_tiles;
    const uint32_t m0 = m_tile * kTileM, n0 = n_tile * kTileN;
    const uint32_t kt_n = a.k / kTileK;

    /* global -> register assignment */
    const uint32_t ac = tid & 7;      /* A: 16-byte chunk of the 128-byte row slice */
    const uint32_t ar0 = tid >> 3;    /* A: rows ar0 + 32 i */
    const uint32_t wr = tid;          /* B: one weight row per thread */
    const uint32_t wrow = n0 + wr < a.n ? n0 + wr : a.n - 1;
    const uint8_t *wptr = a.w + (uint64_t)wrow * a.w_row_stride;
    const _Float16 *xrow[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        uint32_t r = m0 + ar0 + 32 * i;
        xrow[i] = a.x16 + (uint64_t)(r < a.m ? r : a.m - 1) * a.k + 8 * ac;
    }

    r9vx_u32x4 ra[8], q0, q1, hdr;
    auto gload = [&](uint32_t kt) {
#pragma unroll
        for (int i = 0; i < 8; ++i) ra[i] = *reinterpret_cast<const r9vx_u32x4 *>(xrow[i] + kt * kTileK);
        load_w64<SCHEME>(wptr, kt, q0, q1, hdr);
    };
    auto lstore = [&](uint32_t buf, uint32_t kt) {
        uint8_t *A = lds[buf][0];
        uint8_t *B = lds[buf][1];
#pragma unroll
        for (int i = 0; i < 8; ++i) *reinterpret_cast<r9vx_u32x4 *>(A + lds_chunk(ar0 + 32 * i, ac)) = ra[i];
        r9vx_u32x4 wq[8];
        dequant_row64<SCHEME>(q0, q1, hdr, kt & 3, wq);
#pragma unroll
        for (int c = 0; c < 8; ++c) *reinterpret_cast<r9vx_u32x4 *>(B + lds_chunk(wr, c)) = wq[c];
    };

    r9vx_f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    gload(0);
    lstore(0, 0);
    __syncthreads();

    const uint32_t frow = lane & 31, fchk = lane >> 5;
    for (uint32_t kt = 0; kt < kt_n; ++kt) {
        const uint32_t cur = kt & 1;
        const bool more = kt + 1 < kt_n;
        if (more) gload(kt + 1);
        const uint8_t *A = lds[cur][0];
        const uint8_t *B = lds[cur][1];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            half8 af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                af[i] = *reinterpret_cast<const half8 *>(A + lds_chunk(wm * 128 + i * 32 + frow, 2 * s + fchk));
#pragma unroll
            for (int j = 0; j < 4; ++j)
                bf[j] = *reinterpret_cast<const half8 *>(B + lds_chunk(wn * 128 + j * 32 + frow, 2 * s + fchk));
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (more) lstore(cur ^ 1, kt + 1);
        __syncthreads();
    }

    /* epilogue: D[i][j] of a 32x32 tile sits in lane l, register r at
     * row 8*(r/4) + 4*(l/32) + r%4, column l%32. */
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t row = m0 + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (row >= a.m) continue;
            const float sc = a.scale[row];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t col = n0 + wn * 128 + j * 32 + (lane & 31);
                if (col >= a.n) continue;
                float v = acc[i][j][r] * sc;
                if (a.epilogue == R9VX_EPILOGUE_BIAS) v += a.bias[col];
                if (a.epilogue == R9VX_EPILOGUE_RESIDUAL) v += a.residual[(uint64_t)row * a.n + col];
                const uint64_t o = (uint64_t)row * a.n + col;
                if (a.y_bf16)
                    reinterpret_cast<uint16_t *>(a.y)[o] = r9vx_f32_to_bf16(v);
                else
                    reinterpret_cast<float *>(a.y)[o] = v;
            }
        }
    }
}

}  // namespace

size_t r9vx_gemm_workspace_bytes(uint32_t m_bucket, uint32_t k) {
    return (((size_t)m_bucket * k * 2 + 255) & ~(size_t)255) + (size_t)m_bucket * 4;
}

int r9vx_launch_x_to_f16(const uint16_t *x, uint32_t m, uint32_t k, _Float16 *x16, float *scale,
                         hipStream_t stream) {
    hipLaunchKernelGGL(x_to_f16_kernel, dim3(m), dim3(256), 0, stream, x, k, x16, scale);
    return (int)hipGetLastError();
}

int r9vx_launch_gemm(const r9vx_gemm_problem &p, hipStream_t stream) {
    _Float16 *x16 = reinterpret_cast<_Float16 *>(p.workspace);
    float *scale = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(p.workspace) +
                                             (((size_t)p.m * p.k * 2 + 255) & ~(size_t)255));
    hipLaunchKernelGGL(x_to_f16_kernel, dim3(p.m), dim3(256), 0, stream, p.x, p.k, x16, scale);
    GemmArgs a{};
    a.x16 = x16;
    a.scale = scale;
    a.w = p.w;
    a.bias = p.bias;
    a.residual = p.residual;
    a.y = p.y;
    a.w_row_stride = (uint64_t)(p.k / 256) * (p.scheme == R9VX_SCHEME_Q4_K ? R9VX_Q4K_BYTES : R9VX_IQ4XS_BYTES);
    a.m = p.m;
    a.n = p.n;
    a.k = p.k;
    a.m_tiles = (p.m + kTileM - 1) / kTileM;
    a.n_tiles = (p.n + kTileN - 1) / kTileN;
    a.y_bf16 = p.y_dtype == R9VX_DTYPE_BF16;
    a.epilogue = p.epilogue;
    dim3 grid(a.m_tiles * a.n_tiles);
    if (p.scheme == R9VX_SCHEME_Q4_K)
        hipLaunchKernelGGL(gemm_kernel<R9VX_SCHEME_Q4_K>, grid, dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(gemm_kernel<R9VX_SCHEME_IQ4_XS>, grid, dim3(256), 0, stream, a);
    return (int)hipGetLastError();
}
