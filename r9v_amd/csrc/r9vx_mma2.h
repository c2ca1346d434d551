/*
 * r9vx_mma2.h -- dequant-GEMM main loop with the weights decoded straight
 * into MFMA operand registers.
 *
 * Workgroup: 512 threads = 8 waves, two per SIMD (one wave per SIMD leaves
 * the matrix pipe idle between MFMAs; two keep it near peak).  Output tile
 * 256 x 256; wave w owns the 32 output columns [32w, 32w+32) and all 256
 * rows: eight v_mfma_f32_32x32x16_f16 tiles, 128 accumulator registers.
 *
 * K runs in steps of 64 (one Q4_K sub-block pair / two IQ4_XS sub-blocks:
 * 32 payload bytes per weight row).  Within a step the eight 16-byte "groups"
 * q = 0..7 of a row hold the 8 K positions that 4 payload bytes decode to
 * (their 4 low nibbles, then their 4 high nibbles):
 *   Q4_K   (crates/r9v-format/src/ggml.rs:744-790): bytes 4q..4q+3 ->
 *          k = 4q..4q+3 and 32+4q..32+4q+3
 *   IQ4_XS (crates/r9v-format/src/iq.rs:274-293):  bytes 4q..4q+3 ->
 *          k = 32(q/4) + 4(q%4) + {0..3} and the same + 16
 * Lane l of a wave (column 32w + l%32, half h = l/32) loads the 16 payload
 * bytes of groups 4h..4h+3 and, for MFMA slice s, decodes group q = 4h + s
 * into its 8-fp16 B operand.  The activations are stored by x_to_f16 in the
 * same group order, so the A operand of slice s is group 4h + s of the row:
 * one 16-byte LDS read.  A K-permutation applied to both operands leaves
 * every dot product unchanged.
 *
 * Activations reach LDS by direct global->LDS loads (no registers) into a
 * 4-stage ring, three steps ahead; the weight payload is loaded two steps
 * ahead into registers.  The main loop is unrolled by the 4 steps of a
 * super-block, so stage, register set and sub-block index are compile-time
 * constants and the body has no branches.  LDS rows are 128 bytes of eight
 * 16-byte groups stored at slot group ^ swz(row), swz(row) = (row >> 1) & 7:
 * with 64 four-byte LDS banks a 128-byte row covers half the banks, so the
 * 16 rows that one LDS read cycle serves (8 even, 8 odd) must use 8 distinct
 * slots per parity to be conflict-free.
 */
#ifndef R9VX_MMA2_H
#define R9VX_MMA2_H

#include "r9vx_mfma.h"

namespace r9vx {

constexpr int kM2Rows = 256;       /* output rows per tile */
constexpr int kM2Cols = 256;       /* output columns per tile */
constexpr int kM2Waves = 8;
constexpr int kM2Stages = 4;
constexpr int kM2StageBytes = kM2Rows * 128;

/* LDS slot swizzle of a 128-byte A row. */
__host__ __device__ constexpr uint32_t m2_swz(uint32_t row) { return (row >> 1) & 7u; }

/* K offset (within a 64-step) of element i (0..7) of group q. */
template <int SCHEME>
__host__ __device__ constexpr uint32_t group_k(uint32_t q, uint32_t i) {
    if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
        return (i < 4 ? 0u : 32u) + 4 * q + (i & 3);
    } else {
        return 32 * (q >> 2) + (i < 4 ? 0u : 16u) + 4 * (q & 3) + (i & 3);
    }
}

/* The weight bytes one lane needs for one K step. */
struct BRaw {
    r9vx_u32x4 p;   /* payload bytes 16h..16h+15 of the step */
    r9vx_u32x4 hdr; /* block header (Q4_K 16 bytes; IQ4_XS 8 bytes in .x/.y) */
};

/* The main loop issues its loads as inline assembly so that the compiler's
 * automatic waits (which cannot tell a copy into one LDS stage from reads of
 * another, and count only the loads they know of) never stall on loads of
 * later steps; it waits for them itself (wait_vm) before each step's
 * barrier, and touch() marks the point after which the registers hold the
 * loaded data. */
template <int SCHEME>
__device__ __forceinline__ void load_braw(const uint8_t *row, uint32_t kt, uint32_t h, BRaw &b) {
    const uint32_t blk = kt >> 2, ks = kt & 3;
    if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
        const uint8_t *bp = row + (uint64_t)blk * R9VX_Q4K_BYTES;
        const uint8_t *pp = bp + 16 + 32 * ks + 16 * h;
        asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(b.hdr) : "v"(bp) : "memory");
        asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(b.p) : "v"(pp) : "memory");
    } else {
        const uint8_t *bp = row + (uint64_t)blk * R9VX_IQ4XS_BYTES;
        const uint8_t *pp = bp + 8 + 32 * ks + 16 * h;
        r9vx_u32x2 hh;
        asm volatile("global_load_dwordx2 %0, %1, off" : "=v"(hh) : "v"(bp) : "memory");
        asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(b.p) : "v"(pp) : "memory");
        b.hdr = r9vx_u32x4{hh.x, hh.y, 0u, 0u};
    }
}

/* After the wait that covers b's loads: the registers now hold the data. */
template <int SCHEME>
__device__ __forceinline__ void touch(BRaw &b) {
    if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
        asm volatile("" : "+v"(b.hdr), "+v"(b.p));
    } else {
        r9vx_u32x2 hh{b.hdr.x, b.hdr.y};
        asm volatile("" : "+v"(hh), "+v"(b.p));
        b.hdr = r9vx_u32x4{hh.x, hh.y, 0u, 0u};
    }
}

/* Per-step scale terms of one lane. */
struct BScale {
    float dl0, nml0, dl1, nml1; /* Q4_K: low nibbles (sub-block 2ks), high (2ks+1); IQ4_XS: dl0 */
};

template <int SCHEME, int KS>
__device__ __forceinline__ BScale braw_scale(const BRaw &b, uint32_t h) {
    BScale s;
    const float d = r9vx_f16_to_f32((uint16_t)(b.hdr.x & 0xFFFF));
    if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
        const float dmin = r9vx_f16_to_f32((uint16_t)(b.hdr.x >> 16));
        uint32_t sc[2], mn[2];
        r9vx_q4k_scale_pair(b.hdr, KS, sc, mn); /* KS constant: no branches */
        s.dl0 = d * (float)sc[0];
        s.nml0 = -(dmin * (float)mn[0]);
        s.dl1 = d * (float)sc[1];
        s.nml1 = -(dmin * (float)mn[1]);
    } else {
        s.dl0 = d * r9vx_iq4xs_scale(r9vx_u32x2{b.hdr.x, b.hdr.y}, 2 * KS + h);
        s.nml0 = s.dl1 = s.nml1 = 0.f;
    }
    return s;
}

__device__ __forceinline__ uint32_t cvt_pk_h2_2(float a, float b) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    h2 r;
    r.x = (_Float16)a;
    r.y = (_Float16)b;
    return __builtin_bit_cast(uint32_t, r);
}

/* B operand of slice s: group 4h + s = payload dword s, decoded with the
 * exact f32 formula and rounded once to fp16. */
template <int SCHEME>
__device__ __forceinline__ half8 decode_bfrag(const BRaw &b, const BScale &sc, int s, const float *lutf) {
    const uint32_t dw = s == 0 ? b.p.x : s == 1 ? b.p.y : s == 2 ? b.p.z : b.p.w;
    uint32_t o[4];
    if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
        const uint32_t l4 = dw & 0x0F0F0F0Fu, h4 = (dw >> 4) & 0x0F0F0F0Fu;
        float l[4], hv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            l[j] = fmaf(sc.dl0, (float)((l4 >> (8 * j)) & 0xFFu), sc.nml0);
            hv[j] = fmaf(sc.dl1, (float)((h4 >> (8 * j)) & 0xFFu), sc.nml1);
        }
        o[0] = cvt_pk_h2_2(l[0], l[1]);
        o[1] = cvt_pk_h2_2(l[2], l[3]);
        o[2] = cvt_pk_h2_2(hv[0], hv[1]);
        o[3] = cvt_pk_h2_2(hv[2], hv[3]);
    } else {
        float l[4], hv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float *e = lutf + 2 * ((dw >> (8 * j)) & 0xFFu);
            l[j] = sc.dl0 * e[0];
            hv[j] = sc.dl0 * e[1];
        }
        o[0] = cvt_pk_h2_2(l[0], l[1]);
        o[1] = cvt_pk_h2_2(l[2], l[3]);
        o[2] = cvt_pk_h2_2(hv[0], hv[1]);
        o[3] = cvt_pk_h2_2(hv[2], hv[3]);
    }
    return __builtin_bit_cast(half8, r9vx_u32x4{o[0], o[1], o[2], o[3]});
}

/* Direct global->LDS copy of one K step of A (256 rows x 64 fp16, already in
 * group order): 4 instructions per lane; instruction i of wave w fills LDS
 * rows 8(4w + i) .. +8, lane l row 8(4w+i) + l/8, slot l%8, which holds group
 * (l%8) ^ swz(row).  src[i] points at the lane's group of step 0.  M0 holds
 * the wave's LDS destination. */
__device__ __forceinline__ void dma_a_step(uint8_t *stage, const _Float16 *const (&src)[4], uint32_t kt,
                                           uint32_t wave) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const _Float16 *g = src[i] + (uint64_t)kt * 64;
        const uint32_t l = __builtin_amdgcn_readfirstlane(
            (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)(stage + (wave * 4 + i) * 1024));
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(l)
                     : "memory", "m0");
    }
}

/* Workgroup barrier that the compiler does not move memory operations across
 * and that adds no waits of its own: the caller has waited for what other
 * waves will read. */
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

/* Waits until at most N vector-memory loads of this wave are outstanding
 * (loads complete in order), leaving LDS and scalar counters alone. */
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

/* MFMAs of one K step (sub-block pair KS of its super-block) from A stage
 * `st` and the lane's decoded weights. */
template <int SCHEME, int KS>
__device__ __forceinline__ void m2_step(const uint8_t *st, const BRaw &b, uint32_t lane, const float *lutf,
                                        r9vx_f32x16 (&acc)[8]) {
    const uint32_t h = lane >> 5, r32 = lane & 31;
    const BScale sc = braw_scale<SCHEME, KS>(b, h);
    /* The 32 MFMAs of the step in order i = 8s + t (slice s, row tile t); the
     * A operand of MFMA i + kAhead is read from LDS just before MFMA i, into
     * a ring of kAhead + 1 registers.  Rows 32t + r32 share one swizzle
     * (swz(32t + r32) = swz(r32)). */
    constexpr int kAhead = 4;
    half8 af[kAhead + 1];
    auto read_a = [&](int i) {
        const int s = i >> 3, t = i & 7;
        const uint32_t q = 4 * h + (uint32_t)s;
        af[i % (kAhead + 1)] =
            *reinterpret_cast<const half8 *>(st + r32 * 128 + ((q ^ m2_swz(r32)) << 4) + 4096 * t);
    };
#pragma unroll
    for (int i = 0; i < kAhead; ++i) read_a(i);
    half8 bf = decode_bfrag<SCHEME>(b, sc, 0, lutf);
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        if (i + kAhead < 32) read_a(i + kAhead);
        if ((i & 7) == 0 && i > 0) bf = decode_bfrag<SCHEME>(b, sc, i >> 3, lutf);
        acc[i & 7] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i % (kAhead + 1)], bf, acc[i & 7], 0, 0, 0);
    }
    /* Issue order: the first reads, then each MFMA with one read ahead of it
     * and a share of the decode VALU work. */
    __builtin_amdgcn_sched_group_barrier(0x100, kAhead, 0); /* DS read */
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); /* DS read */
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); /* MFMA */
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0); /* VALU */
    }
}

}  // namespace r9vx

#endif
