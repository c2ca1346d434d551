/*
 * r9vx_mma.h -- the main loop of the dequant-to-LDS MFMA GEMM that the dense
 * prefill matmul runs for Q8_0 / Q6_K / IQ3_S weights when N % 256 != 0.
 *
 * Workgroup: 256 threads = 4 waves, output tile BM x 256.  Wave w owns the
 * 64 output columns [64w, 64w+64) and all BM rows: (BM/32) x 2 tiles of
 * v_mfma_f32_32x32x16_f16, BM accumulator registers.  Per K step of 64:
 *   A: BM rows x 64 fp16 from the caller's activation source -> LDS
 *   B: 256 weight rows x 32 payload bytes (one row per thread) -> dequantized
 *      with the exact f32 formula (crates/r9v-format/src/ggml.rs:1131-1150,
 *      iq.rs:578-598), rounded once to fp16 -> LDS
 * LDS rows are 128 bytes of eight 16-byte chunks stored at chunk ^ (row & 7).
 * NBUF = 2 double-buffers LDS (one barrier per step, next step's loads and
 * dequant overlap this step's MFMAs); NBUF = 1 single-buffers it (two barriers
 * per step) so that two workgroups share a CU and interleave.
 */
#ifndef R9VX_MMA_H
#define R9VX_MMA_H

#include "r9vx_mfma.h"

namespace r9vx {

template <int BM, int NBUF>
struct MmaShape {
    static constexpr int kABytes = BM * 128;
    static constexpr int kBBytes = 256 * 128;
    static constexpr int kStage = kABytes + kBBytes;
    static constexpr int kLds = NBUF * kStage + 256 * 8; /* + IQ4 f32 pair table */
    static constexpr int kMT = BM / 32;                  /* 32-row tiles per wave */
};

__device__ __forceinline__ uint32_t cvt_pk_h2(float a, float b) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    h2 r;
    r.x = (_Float16)a;
    r.y = (_Float16)b;
    return __builtin_bit_cast(uint32_t, r);
}

/* Weight bytes one thread carries for one K step. */
struct WRegs {
    r9vx_u32x4 q0, q1, hdr;
};

/* Dequantizes one weight row's 64 K values of step ks (0..3 in the super-
 * block) and stores them as 8 chunks of LDS row `row`. */
template <int SCHEME>
__device__ __forceinline__ void dequant_store(const WRegs &w, uint32_t ks, uint8_t *B, uint32_t row,
                                              const float *lutf) {
    uint32_t b[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
    if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
        const float d = r9vx_f16_to_f32((uint16_t)(w.hdr.x & 0xFFFF));
        const float dmin = r9vx_f16_to_f32((uint16_t)(w.hdr.x >> 16));
        uint32_t sc[2], mn[2];
        r9vx_q4k_scale_pair(w.hdr, ks, sc, mn);
        const float dl0 = d * (float)sc[0], nml0 = -(dmin * (float)mn[0]);
        const float dl1 = d * (float)sc[1], nml1 = -(dmin * (float)mn[1]);
        uint32_t lo[16], hi[16];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t l4 = b[i] & 0x0F0F0F0Fu, h4 = (b[i] >> 4) & 0x0F0F0F0Fu;
            float l[4], h[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                l[j] = fmaf(dl0, (float)((l4 >> (8 * j)) & 0xFFu), nml0);
                h[j] = fmaf(dl1, (float)((h4 >> (8 * j)) & 0xFFu), nml1);
            }
            lo[2 * i] = cvt_pk_h2(l[0], l[1]);
            lo[2 * i + 1] = cvt_pk_h2(l[2], l[3]);
            hi[2 * i] = cvt_pk_h2(h[0], h[1]);
            hi[2 * i + 1] = cvt_pk_h2(h[2], h[3]);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            *reinterpret_cast<r9vx_u32x4 *>(B + lds_chunk(row, c)) =
                r9vx_u32x4{lo[4 * c], lo[4 * c + 1], lo[4 * c + 2], lo[4 * c + 3]};
            *reinterpret_cast<r9vx_u32x4 *>(B + lds_chunk(row, 4 + c)) =
                r9vx_u32x4{hi[4 * c], hi[4 * c + 1], hi[4 * c + 2], hi[4 * c + 3]};
        }
    } else {
        const float d = r9vx_f16_to_f32((uint16_t)(w.hdr.x & 0xFFFF));
        const r9vx_u32x2 h2{w.hdr.x, w.hdr.y};
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const float dl = d * r9vx_iq4xs_scale(h2, 2 * ks + s);
            uint32_t lo[8], hi[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t wd = b[4 * s + i];
                float l[4], h[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float *e = lutf + 2 * ((wd >> (8 * j)) & 0xFFu);
                    l[j] = dl * e[0];
                    h[j] = dl * e[1];
                }
                lo[2 * i] = cvt_pk_h2(l[0], l[1]);
                lo[2 * i + 1] = cvt_pk_h2(l[2], l[3]);
                hi[2 * i] = cvt_pk_h2(h[0], h[1]);
                hi[2 * i + 1] = cvt_pk_h2(h[2], h[3]);
            }
            *reinterpret_cast<r9vx_u32x4 *>(B + lds_chunk(row, 4 * s + 0)) = r9vx_u32x4{lo[0], lo[1], lo[2], lo[3]};
            *reinterpret_cast<r9vx_u32x4 *>(B + lds_chunk(row, 4 * s + 1)) = r9vx_u32x4{lo[4], lo[5], lo[6], lo[7]};
            *reinterpret_cast<r9vx_u32x4 *>(B + lds_chunk(row, 4 * s + 2)) = r9vx_u32x4{hi[0], hi[1], hi[2], hi[3]};
            *reinterpret_cast<r9vx_u32x4 *>(B + lds_chunk(row, 4 * s + 3)) = r9vx_u32x4{hi[4], hi[5], hi[6], hi[7]};
        }
    }
}

template <int SCHEME>
__device__ __forceinline__ void load_w(const uint8_t *row, uint32_t kt, WRegs &w) {
    load_w64<SCHEME>(row, kt, w.q0, w.q1, w.hdr);
}

/* Q8_0 / Q6_K in the split layout (body row + f16 d row).  One K step of 64:
 *   Q8_0: blocks 2kt, 2kt+1: 64 body bytes and their two d values;
 *   Q6_K: step ks = kt%4 of super-block kt/4 covers values 64ks..64ks+63:
 *         value t takes nibble ks%2 of ql byte 64(ks/2)+t, bit pair
 *         2(ks%2) + t/32 of qh byte 32(ks/2) + t%32, and scale 4ks + t/16
 *         (crates/r9v-format/src/ggml.rs:817-850). */
struct WRegsQ80 {
    r9vx_u32x4 q[4];
    uint32_t d2;
};
struct WRegsQ6K {
    r9vx_u32x4 ql[4], qh[2];
    uint32_t sc4, d;
};
/* IQ3_S in its 112-byte device blocks: step ks = kt%4 of block kt/4 covers
 * groups 2ks and 2ks+1: index bytes 16ks..16ks+15, sign words 2ks and
 * 2ks+1 (bytes 64 + 8ks), and the block's side word (qh, scales, d). */
struct WRegsIq3 {
    r9vx_u32x4 q, side;
    r9vx_u32x2 sg;
};
template <int SCHEME>
struct WRegsFor {
    using T = WRegs;
};
template <>
struct WRegsFor<R9VX_SCHEME_IQ3_S> {
    using T = WRegsIq3;
};
template <>
struct WRegsFor<R9VX_SCHEME_Q8_0> {
    using T = WRegsQ80;
};
template <>
struct WRegsFor<R9VX_SCHEME_Q6_K> {
    using T = WRegsQ6K;
};

template <int SCHEME>
__device__ __forceinline__ void load_w_any(const uint8_t *row, const uint16_t *srow, uint32_t kt,
                                           typename WRegsFor<SCHEME>::T &w) {
    if constexpr (SCHEME == R9VX_SCHEME_Q8_0) {
        const uint8_t *p = row + 64 * (uint64_t)kt;
#pragma unroll
        for (int i = 0; i < 4; ++i) w.q[i] = r9vx_ld128(p + 16 * i);
        w.d2 = *reinterpret_cast<const uint32_t *>(srow + 2 * kt);
    } else if constexpr (SCHEME == R9VX_SCHEME_IQ3_S) {
        const uint8_t *b = row + (uint64_t)(kt >> 2) * R9VX_IQ3S_DEV_BYTES;
        const uint32_t ks = kt & 3;
        w.q = r9vx_ld128(b + 16 * ks);
        w.sg = *reinterpret_cast<const r9vx_u32x2 *>(b + 64 + 8 * ks);
        w.side = r9vx_ld128(b + 96);
    } else if constexpr (SCHEME == R9VX_SCHEME_Q6_K) {
        const uint32_t blk = kt >> 2, ks = kt & 3, g = ks >> 1;
        const uint8_t *b = row + (uint64_t)blk * R9VX_Q6K_BODY;
#pragma unroll
        for (int i = 0; i < 4; ++i) w.ql[i] = r9vx_ld128(b + 64 * g + 16 * i);
        w.qh[0] = r9vx_ld128(b + 128 + 32 * g);
        w.qh[1] = r9vx_ld128(b + 128 + 32 * g + 16);
        w.sc4 = *reinterpret_cast<const uint32_t *>(b + 192 + 4 * ks);
        w.d = srow[blk];
    } else {
        load_w<SCHEME>(row, kt, w);
    }
}

__device__ __forceinline__ uint32_t u32x4_at(const r9vx_u32x4 &v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

/* Dequantizes one weight row's 64 K values of step ks in natural K order
 * into the 8 LDS chunks of B row `row`: each value with the exact f32
 * formula, then one fp16 rounding. */
template <int SCHEME>
__device__ __forceinline__ void dequant_store_any(const typename WRegsFor<SCHEME>::T &w, uint32_t ks, uint8_t *B,
                                                  uint32_t row, const float *lutf) {
    if constexpr (SCHEME == R9VX_SCHEME_Q8_0) {
        const float d0 = r9vx_f16_to_f32((uint16_t)(w.d2 & 0xFFFF)), d1 = r9vx_f16_to_f32((uint16_t)(w.d2 >> 16));
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const float d = c < 4 ? d0 : d1;
            uint32_t h[4];
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const uint32_t dw = u32x4_at(w.q[c >> 1], 2 * (c & 1) + half);
                h[2 * half] = cvt_pk_h2(d * (float)(int8_t)(dw & 0xFF), d * (float)(int8_t)((dw >> 8) & 0xFF));
                h[2 * half + 1] = cvt_pk_h2(d * (float)(int8_t)((dw >> 16) & 0xFF), d * (float)(int8_t)(dw >> 24));
            }
            *reinterpret_cast<r9vx_u32x4 *>(B + lds_chunk(row, c)) = r9vx_u32x4{h[0], h[1], h[2], h[3]};
        }
    } else if constexpr (SCHEME == R9VX_SCHEME_IQ3_S) {
        /* weight 4i + b of group g = (d (1 + 2 s_g)) grid[idx_i][b], negated
         * when bit 4i + b of the group's sign word is set
         * (crates/r9v-format/src/iq.rs:698-722) */
        const float d = r9vx_f16_to_f32((uint16_t)(w.side.w & 0xFFFF));
#pragma unroll
        for (int gg = 0; gg < 2; ++gg) {
            const uint32_t g = 2 * ks + gg;
            const uint32_t qh = ((g < 4 ? w.side.x : w.side.y) >> (8 * (g & 3))) & 0xFF;
            const float db = d * (1.0f + 2.0f * (float)((w.side.z >> (4 * g)) & 0xF));
            const uint32_t sgw = gg ? w.sg.y : w.sg.x;
#pragma unroll
            for (int c4 = 0; c4 < 4; ++c4) {
                uint32_t h[4];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int i = 2 * c4 + e, byte = 8 * gg + i;
                    const uint32_t idx = ((u32x4_at(w.q, byte >> 2) >> (8 * (byte & 3))) & 0xFF) | (((qh >> i) & 1u) << 8);
                    const uint32_t gw = kIq3sGrid[idx];
                    float v[4];
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const float m = db * (float)((gw >> (8 * b)) & 0xFF);
                        v[b] = ((sgw >> (4 * i + b)) & 1u) ? m * -1.0f : m;
                    }
                    h[2 * e] = cvt_pk_h2(v[0], v[1]);
                    h[2 * e + 1] = cvt_pk_h2(v[2], v[3]);
                }
                *reinterpret_cast<r9vx_u32x4 *>(B + lds_chunk(row, 4 * gg + c4)) = r9vx_u32x4{h[0], h[1], h[2], h[3]};
            }
        }
    } else if constexpr (SCHEME == R9VX_SCHEME_Q6_K) {
        const float d = r9vx_f16_to_f32((uint16_t)w.d);
        const uint32_t nib = 4 * (ks & 1);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const float dl = d * (float)(int8_t)((w.sc4 >> (8 * (c >> 1))) & 0xFF);
            const uint32_t pair = 4 * (ks & 1) + 2 * (c >> 2);
            uint32_t h[4];
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const int i = 2 * c + half; /* dword of the 64 values: t = 4i .. 4i+3 */
                const uint32_t qlw = u32x4_at(w.ql[i >> 2], i & 3);
                const uint32_t qhw = u32x4_at(w.qh[(i & 7) >> 2], i & 3);
                const uint32_t q6 = ((qlw >> nib) & 0x0F0F0F0Fu) | (((qhw >> pair) & 0x03030303u) << 4);
                float v[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = dl * ((float)((q6 >> (8 * j)) & 0xFF) - 32.0f);
                h[2 * half] = cvt_pk_h2(v[0], v[1]);
                h[2 * half + 1] = cvt_pk_h2(v[2], v[3]);
            }
            *reinterpret_cast<r9vx_u32x4 *>(B + lds_chunk(row, c)) = r9vx_u32x4{h[0], h[1], h[2], h[3]};
        }
    } else {
        dequant_store<SCHEME>(w, ks, B, row, lutf);
    }
}

/* MFMAs of one K step from LDS stage (A, B) into acc[BM/32][2].  The
 * fragments of slice s+1 are read while slice s's MFMAs run (two fragment
 * sets in registers), so no MFMA waits on its own LDS read. */
template <int BM>
__device__ __forceinline__ void mma_step(const uint8_t *A, const uint8_t *B, uint32_t wave, uint32_t lane,
                                         r9vx_f32x16 (&acc)[BM / 32][2]) {
    constexpr int MT = BM / 32;
    const uint32_t frow = lane & 31, fchk = lane >> 5;
    half8 af[2][MT], bf[2][2];
    auto load = [&](int s, int buf) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
            bf[buf][j] = *reinterpret_cast<const half8 *>(B + lds_chunk(wave * 64 + j * 32 + frow, 2 * s + fchk));
#pragma unroll
        for (int i = 0; i < MT; ++i)
            af[buf][i] = *reinterpret_cast<const half8 *>(A + lds_chunk(i * 32 + frow, 2 * s + fchk));
    };
    load(0, 0);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int cur = s & 1;
        if (s < 3) load(s + 1, cur ^ 1);
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cur][i], bf[cur][j], acc[i][j], 0, 0, 0);
    }
}

/*
 * The main loop.  ASrc supplies activations:
 *   typename ASrc::Regs;  void load(uint32_t kt, Regs&);  void store(const Regs&, uint8_t *A)
 * `wrow` is this thread's weight row (LDS B row = threadIdx.x); kt_n K steps.
 */
template <int SCHEME, int BM, int NBUF, typename ASrc>
__device__ __forceinline__ void mma_mainloop(uint8_t *lds, ASrc &asrc, const uint8_t *wrow, uint32_t kt_n,
                                             r9vx_f32x16 (&acc)[BM / 32][2], const uint16_t *srow = nullptr) {
    using S = MmaShape<BM, NBUF>;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *lutf = reinterpret_cast<const float *>(lds + NBUF * S::kStage);
    if constexpr (SCHEME == R9VX_SCHEME_IQ4_XS)
        init_iq4_lut_f32(reinterpret_cast<r9vx_f32x4 *>(lds + NBUF * S::kStage), tid);
#pragma unroll
    for (int i = 0; i < BM / 32; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    typename ASrc::Regs ra;
    typename WRegsFor<SCHEME>::T wq;
    asrc.load(0, ra);
    load_w_any<SCHEME>(wrow, srow, 0, wq);
    __syncthreads(); /* the codebook table */
    asrc.store(ra, lds);
    dequant_store_any<SCHEME>(wq, 0, lds + S::kABytes, tid, lutf);
    __syncthreads();
    if constexpr (NBUF == 2) {
        for (uint32_t kt = 0; kt < kt_n; ++kt) {
            const uint32_t cur = kt & 1;
            const bool more = kt + 1 < kt_n;
            if (more) {
                asrc.load(kt + 1, ra);
                load_w_any<SCHEME>(wrow, srow, kt + 1, wq);
            }
            uint8_t *st = lds + cur * S::kStage;
            mma_step<BM>(st, st + S::kABytes, wave, lane, acc);
            if (more) {
                uint8_t *nx = lds + (cur ^ 1) * S::kStage;
                asrc.store(ra, nx);
                dequant_store_any<SCHEME>(wq, (kt + 1) & 3, nx + S::kABytes, tid, lutf);
            }
            __syncthreads();
        }
    } else {
        for (uint32_t kt = 0; kt < kt_n; ++kt) {
            const bool more = kt + 1 < kt_n;
            if (more) {
                asrc.load(kt + 1, ra);
                load_w_any<SCHEME>(wrow, srow, kt + 1, wq);
            }
            mma_step<BM>(lds, lds + S::kABytes, wave, lane, acc);
            __syncthreads();
            if (more) {
                asrc.store(ra, lds);
                dequant_store_any<SCHEME>(wq, (kt + 1) & 3, lds + S::kABytes, tid, lutf);
            }
            __syncthreads();
        }
    }
}

/* Row / column of accumulator register r of tile (i, j) for this lane. */
__device__ __forceinline__ uint32_t acc_row(int i, int r, uint32_t lane) {
    return (uint32_t)(i * 32 + 8 * (r >> 2) + 4 * (int)(lane >> 5) + (r & 3));
}
__device__ __forceinline__ uint32_t acc_col(uint32_t wave, int j, uint32_t lane) {
    return wave * 64 + (uint32_t)j * 32 + (lane & 31);
}

/* A source: fp16 rows (row pointers precomputed per thread). */
template <int BM>
struct AF16Rows {
    static constexpr int kPer = BM / 32; /* rows per thread (one 16-byte chunk each) */
    struct Regs {
        r9vx_u32x4 v[BM / 32];
    };
    const _Float16 *row[BM / 32];
    uint32_t chunk, row0;
    __device__ __forceinline__ void load(uint32_t kt, Regs &r) const {
#pragma unroll
        for (int i = 0; i < kPer; ++i) r.v[i] = *reinterpret_cast<const r9vx_u32x4 *>(row[i] + kt * 64);
    }
    __device__ __forceinline__ void store(const Regs &r, uint8_t *A) const {
#pragma unroll
        for (int i = 0; i < kPer; ++i) *reinterpret_cast<r9vx_u32x4 *>(A + lds_chunk(row0 + 32 * i, chunk)) = r.v[i];
    }
};

}  // namespace r9vx

#endif
