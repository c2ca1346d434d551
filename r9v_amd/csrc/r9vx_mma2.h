/*
 * r9vx_mma2.h -- dequant-GEMM main loop with the weights decoded straight
 * into MFMA operand registers, shared by the dense prefill GEMM and the two
 * grouped MoE GEMMs.
 *
 * Shape (template MT, NWN): a workgroup of MT waves computes a tile of
 * 32*MT rows; wave w owns NWN 32-column tiles and all rows: MT x NWN
 * v_mfma_f32_32x32x16_f16 accumulators (MT * NWN * 16 registers).  Dense:
 * MT = 8, NWN = 1 (256 x 256 tile, 512 threads, one workgroup per CU, two
 * waves per SIMD).  MoE: MT = 4, NWN = 2 (128 x 256 tile, 256 threads, two
 * workgroups per CU).  Two waves per SIMD keep the matrix pipe near peak;
 * one leaves it idle between MFMAs.
 *
 * K runs in steps of 64 (one Q4_K sub-block pair / two IQ4_XS sub-blocks:
 * 32 payload bytes per weight row).  Within a step the eight 16-byte "groups"
 * q = 0..7 of a row hold the 8 K positions that 4 payload bytes decode to
 * (their 4 low nibbles, then their 4 high nibbles):
 *   Q4_K   (crates/r9v-format/src/ggml.rs:744-790): bytes 4q..4q+3 ->
 *          k = 4q..4q+3 and 32+4q..32+4q+3
 *   IQ4_XS (crates/r9v-format/src/iq.rs:274-293):  bytes 4q..4q+3 ->
 *          k = 32(q/4) + 4(q%4) + {0..3} and the same + 16
 * Lane l (column l%32 of each of its column tiles, half h = l/32) loads the 16
 * payload bytes of groups 4h..4h+3 and, for MFMA slice s, decodes group
 * q = 4h + s into its 8-fp16 B operand with the exact f32 formula, rounded
 * once to fp16.  The activations are stored in the same group order (by
 * x_to_f16 / the h conversion), so the A operand of slice s is group 4h + s
 * of the row: one 16-byte LDS read.  A K-permutation applied to both operands
 * leaves every dot product unchanged.
 *
 * Activations reach LDS by direct global->LDS loads (no registers) into a
 * 4-stage ring, three steps ahead; the weight payload is loaded two steps
 * ahead into registers, the block headers one super-block ahead.  The main
 * loop is unrolled by the 4 steps of a super-block, so stage, register set
 * and sub-block index are compile-time constants and the body has no
 * branches.  LDS rows are 128 bytes of eight 16-byte groups stored at slot
 * group ^ swz(row), swz(row) = (row >> 1) & 7: with 64 four-byte LDS banks a
 * 128-byte row covers half the banks, so the 16 rows one LDS read cycle
 * serves (8 even, 8 odd) use 8 distinct slots per parity: conflict-free.
 */
#ifndef R9VX_MMA2_H
#define R9VX_MMA2_H

#include "r9vx_mfma.h"
#include "r9vx_x16.h"

namespace r9vx {

constexpr int kM2Stages = 4;

/* LDS slot swizzle of a 128-byte A row. */
__host__ __device__ constexpr uint32_t m2_swz(uint32_t row) { return (row >> 1) & 7u; }


/*
 * The main loop issues its loads as inline assembly and waits for them itself
 * (wait_vm before each step's barrier).  The compiler's automatic waits cannot
 * tell a copy into one LDS stage from reads of another and count only the
 * loads they know of, so with compiler-visible loads every step would stall
 * on the prefetches of later steps.  touch() marks the point after that wait
 * from which the registers hold the loaded data.  Each load's destination is
 * tied in and out ("+v") and nothing is built from it before the wait, so
 * the register the load writes is the one later read, also for a value
 * carried across the loop back-edge.
 */
template <int SCHEME>
__device__ __forceinline__ void load_bpay(const uint8_t *row, uint32_t kt, uint32_t h, r9vx_u32x4 &p) {
    const uint32_t blk = kt >> 2, ks = kt & 3;
    const uint8_t *pp = SCHEME == R9VX_SCHEME_Q4_K ? row + (uint64_t)blk * R9VX_Q4K_BYTES + 16 + 32 * ks + 16 * h
                                                   : row + (uint64_t)blk * R9VX_IQ4XS_BYTES + 8 + 32 * ks + 16 * h;
    asm volatile("global_load_dwordx4 %0, %1, off" : "+v"(p) : "v"(pp) : "memory");
}

template <int SCHEME>
__device__ __forceinline__ void load_bhdr(const uint8_t *row, uint32_t blk, r9vx_u32x4 &hd) {
    /* Q4_K: the 16-byte header; IQ4_XS: the block's first 16 bytes (its
     * 8-byte header and 8 payload bytes, inside the 136-byte block), of which
     * .x / .y are used */
    const uint8_t *bp = row + (uint64_t)blk * (SCHEME == R9VX_SCHEME_Q4_K ? R9VX_Q4K_BYTES : R9VX_IQ4XS_BYTES);
    asm volatile("global_load_dwordx4 %0, %1, off" : "+v"(hd) : "v"(bp) : "memory");
}

template <int SCHEME>
__device__ __forceinline__ void touch_hdr(r9vx_u32x4 &hd) {
    if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
        asm volatile("" : "+v"(hd));
    } else {
        r9vx_u32x2 hh{hd.x, hd.y};
        asm volatile("" : "+v"(hh));
        hd = r9vx_u32x4{hh.x, hh.y, 0u, 0u};
    }
}
__device__ __forceinline__ void touch_pay(r9vx_u32x4 &p) { asm volatile("" : "+v"(p)); }

/* Direct global->LDS copy of one K step of A (32*MT rows x 64 fp16, already in
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

/* The group of A row `r` (0 .. 32*MT-1) that this lane copies: the row and the
 * global group index for dma_a_step's lane mapping. */
__device__ __forceinline__ uint32_t dma_row(uint32_t wave, int i, uint32_t lane) {
    return (wave * 4 + (uint32_t)i) * 8 + (lane >> 3);
}
__device__ __forceinline__ uint32_t dma_group(uint32_t row, uint32_t lane) { return (lane & 7u) ^ m2_swz(row); }

/* Workgroup barrier that the compiler does not move memory operations across.
 * It first waits for this wave's own LDS reads: the compiler is free to sink
 * the last MFMAs of a step (and the waits for their operands) below the
 * barrier, and a read still in flight there would race with the copy that
 * another wave starts into the same stage once the barrier opens.  The
 * caller has already waited for the loads that other waves will read. */
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

/* Waits until at most N vector-memory loads of this wave are outstanding
 * (loads complete in order), leaving LDS and scalar counters alone.  Written
 * as inline assembly so that it stays ordered with the loads and touch()es
 * around it. */
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N < 64, "vmcnt");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

/* Per-step scale terms of one column. */
struct BScale {
    float dl0, nml0, dl1, nml1; /* Q4_K: low nibbles (sub-block 2ks), high (2ks+1); IQ4_XS: dl0 */
    float c0, c1;               /* Q4_K: nml - 1024 dl, the addend for fp16 operands 1024 + q */
};

template <int SCHEME, int KS>
__device__ __forceinline__ BScale bscale(const r9vx_u32x4 &hd, uint32_t h, uint32_t hd2 = 0u) {
    BScale s;
    if constexpr (SCHEME == R9VX_SCHEME_IQ3_S) {
        /* hd: the block's side word; group 2 KS + h: db = d (1 + 2 s) with
         * s its scale nibble (crates/r9v-format/src/iq.rs:698-722) */
        const float d = r9vx_f16_to_f32((uint16_t)(hd.w & 0xFFFF));
        s.dl0 = d * (float)(1u + 2u * ((hd.z >> (4 * (2 * KS + h))) & 0xFu));
        s.c0 = -1152.f * s.dl0; /* exact: db has at most 16 significant bits */
        s.nml0 = s.dl1 = s.nml1 = s.c1 = 0.f;
        return s;
    }
    if constexpr (SCHEME == R9VX_SCHEME_Q6_K) {
        /* hd: the block's 16 int8 scales, hd2: its f16 d.  Step KS (span n =
         * KS / 2, part j = KS % 2), half h: the low nibbles' columns take
         * scale 8 n + 2 j + h, the high nibbles' 8 n + 4 + 2 j + h (one per
         * 16 columns, crates/r9v-format/src/ggml.rs:817-850) */
        const uint32_t lw = (KS >> 1) == 0 ? hd.x : hd.z, hw = (KS >> 1) == 0 ? hd.y : hd.w;
        const uint32_t sh = 8 * (2 * (KS & 1) + h);
        const float d = r9vx_f16_to_f32((uint16_t)hd2);
        s.dl0 = d * (float)(int8_t)(lw >> sh);
        s.dl1 = d * (float)(int8_t)(hw >> sh);
        s.c0 = -1056.f * s.dl0; /* exact: dl has at most 18 significant bits, 1056 = 33 * 2^5 */
        s.c1 = -1056.f * s.dl1;
        s.nml0 = s.nml1 = 0.f;
        return s;
    }
    if constexpr (SCHEME == R9VX_SCHEME_Q8_0) {
        /* hd: the f16 d of the eight 32-weight blocks of a 256-weight block;
         * step KS, half h is block 2 KS + h */
        const uint32_t dw = KS == 0 ? hd.x : KS == 1 ? hd.y : KS == 2 ? hd.z : hd.w;
        s.dl0 = r9vx_f16_to_f32((uint16_t)(dw >> (16 * h)));
        s.c0 = -1152.f * s.dl0; /* exact: 1152 = 9 * 2^7 */
        s.nml0 = s.dl1 = s.nml1 = s.c1 = 0.f;
        return s;
    }
    const float d = r9vx_f16_to_f32((uint16_t)(hd.x & 0xFFFF));
    if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
        const float dmin = r9vx_f16_to_f32((uint16_t)(hd.x >> 16));
        uint32_t sc[2], mn[2];
        r9vx_q4k_scale_pair(hd, KS, sc, mn); /* KS constant: no branches */
        s.dl0 = d * (float)sc[0];
        s.nml0 = -(dmin * (float)mn[0]);
        s.dl1 = d * (float)sc[1];
        s.nml1 = -(dmin * (float)mn[1]);
        s.c0 = fmaf(-1024.f, s.dl0, s.nml0);
        s.c1 = fmaf(-1024.f, s.dl1, s.nml1);
    } else {
        s.dl0 = d * r9vx_iq4xs_scale(r9vx_u32x2{hd.x, hd.y}, 2 * KS + h);
        s.nml0 = s.dl1 = s.nml1 = s.c0 = s.c1 = 0.f;
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

/* B operand of slice s: group 4h + s = payload dword s. */
template <int SCHEME>
__device__ __forceinline__ half8 decode_bfrag(const r9vx_u32x4 &p, const BScale &sc, int s, const float *lutf) {
    const uint32_t dw = s == 0 ? p.x : s == 1 ? p.y : s == 2 ? p.z : p.w;
    float l[4], hv[4];
    if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
        const uint32_t l4 = dw & 0x0F0F0F0Fu, h4 = (dw >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            l[j] = fmaf(sc.dl0, (float)((l4 >> (8 * j)) & 0xFFu), sc.nml0);
            hv[j] = fmaf(sc.dl1, (float)((h4 >> (8 * j)) & 0xFFu), sc.nml1);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float *e = lutf + 2 * ((dw >> (8 * j)) & 0xFFu);
            l[j] = sc.dl0 * e[0];
            hv[j] = sc.dl0 * e[1];
        }
    }
    return __builtin_bit_cast(half8, r9vx_u32x4{cvt_pk_h2_2(l[0], l[1]), cvt_pk_h2_2(l[2], l[3]),
                                                cvt_pk_h2_2(hv[0], hv[1]), cvt_pk_h2_2(hv[2], hv[3])});
}

/* MFMAs of one K step (sub-block pair KS of its super-block) from A stage
 * `st`.  MFMA order i = MT*s + t (slice s, row tile t), each feeding all NWN
 * column tiles; the A operand of index i + kAhead is read from LDS just before
 * index i, into a ring of kAhead + 1 registers.  Rows 32t + r32 share one
 * swizzle (swz(32t + r32) = swz(r32)). */
template <int SCHEME, int KS, int MT, int NWN>
__device__ __forceinline__ void m2_step(const uint8_t *st, const r9vx_u32x4 (&p)[NWN], const r9vx_u32x4 (&hd)[NWN],
                                        uint32_t lane, const float *lutf, r9vx_f32x16 (&acc)[MT][NWN]) {
    const uint32_t h = lane >> 5, r32 = lane & 31;
    BScale sc[NWN];
#pragma unroll
    for (int j = 0; j < NWN; ++j) sc[j] = bscale<SCHEME, KS>(hd[j], h);
    constexpr int kAhead = 4 / NWN, kN = 4 * MT; /* about 4 MFMAs of read-ahead */
    half8 af[kAhead + 1];
    auto read_a = [&](int i) {
        const int s = i / MT, t = i % MT;
        const uint32_t q = 4 * h + (uint32_t)s;
        af[i % (kAhead + 1)] =
            *reinterpret_cast<const half8 *>(st + r32 * 128 + ((q ^ m2_swz(r32)) << 4) + 4096 * t);
    };
#pragma unroll
    for (int i = 0; i < kAhead; ++i) read_a(i);
    half8 bf[NWN];
#pragma unroll
    for (int i = 0; i < kN; ++i) {
        if (i + kAhead < kN) read_a(i + kAhead);
        if (i % MT == 0) {
#pragma unroll
            for (int j = 0; j < NWN; ++j) bf[j] = decode_bfrag<SCHEME>(p[j], sc[j], i / MT, lutf);
        }
#pragma unroll
        for (int j = 0; j < NWN; ++j)
            acc[i % MT][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i % (kAhead + 1)], bf[j], acc[i % MT][j], 0, 0, 0);
    }
    /* Issue order: the first reads, then each group of NWN MFMAs with one read
     * ahead of it and a share of the decode VALU work. */
    __builtin_amdgcn_sched_group_barrier(0x100, kAhead, 0); /* DS read */
#pragma unroll
    for (int i = 0; i < kN; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);       /* DS read */
        __builtin_amdgcn_sched_group_barrier(0x008, NWN, 0);     /* MFMA */
        __builtin_amdgcn_sched_group_barrier(0x002, 3 * NWN, 0); /* VALU */
    }
}

/*
 * The main loop over nk K steps (nk a multiple of 4).  Per step the loads are,
 * in order: the A copy of step +3 (4 instructions), the payload of step +2
 * (NWN), and at the first step of a super-block the headers of the next
 * super-block (NWN).  Before step k only the loads issued during step k - 1
 * may still be in flight, which wait_vm's count states exactly.
 *   stages: 4 LDS stages of 32*MT*128 bytes; asrc: dma sources; wrow: the
 *   lane's weight row per column tile.
 */
template <int SCHEME, int MT, int NWN>
__device__ __forceinline__ void m2_mainloop(uint8_t *const (&stages)[4], const _Float16 *const (&asrc)[4],
                                            const uint8_t *const (&wrow)[NWN], uint32_t nk, uint32_t wave,
                                            uint32_t lane, const float *lutf, r9vx_f32x16 (&acc)[MT][NWN]) {
    const uint32_t h = lane >> 5;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NWN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    r9vx_u32x4 pay[4][NWN], hcur[NWN], hnext[NWN];
#pragma unroll
    for (int j = 0; j < NWN; ++j) {
#pragma unroll
        for (int q = 0; q < 4; ++q) pay[q][j] = r9vx_u32x4{0u, 0u, 0u, 0u};
        hnext[j] = r9vx_u32x4{0u, 0u, 0u, 0u};
    }
    /* prologue in the steady-state order: A0 A1 H(blk 0) P0 | A2 P1 */
    dma_a_step(stages[0], asrc, 0, wave);
    dma_a_step(stages[1], asrc, 1, wave);
#pragma unroll
    for (int j = 0; j < NWN; ++j) load_bhdr<SCHEME>(wrow[j], 0, hnext[j]);
#pragma unroll
    for (int j = 0; j < NWN; ++j) load_bpay<SCHEME>(wrow[j], 0, h, pay[0][j]);
    dma_a_step(stages[2], asrc, 2, wave);
#pragma unroll
    for (int j = 0; j < NWN; ++j) load_bpay<SCHEME>(wrow[j], 1, h, pay[1][j]);

    const uint32_t nblk = nk / 4;
    for (uint32_t blk = 0; blk < nblk; ++blk) {
        /* At the first step of a super-block its headers (loaded one block
         * earlier into hnext) become hcur, and hnext takes the next block's. */
#define R9VX_M2_STEP(J)                                                                              \
    {                                                                                                \
        const uint32_t k = blk * 4 + J;                                                              \
        wait_vm<(J == 1 ? 4 + 2 * NWN : 4 + NWN)>(); /* step k's A copy, payload and headers */      \
        _Pragma("unroll") for (int j = 0; j < NWN; ++j) {                                            \
            touch_pay(pay[J][j]);                                                                    \
            if (J == 0) {                                                                            \
                touch_hdr<SCHEME>(hnext[j]);                                                         \
                hcur[j] = hnext[j];                                                                  \
            }                                                                                        \
        }                                                                                            \
        lds_barrier(); /* and every wave's A copy */                                                 \
        const uint32_t ka = k + 3 < nk ? k + 3 : nk - 1;                                             \
        const uint32_t kb = k + 2 < nk ? k + 2 : nk - 1;                                             \
        dma_a_step(stages[(J + 3) & 3], asrc, ka, wave);                                             \
        _Pragma("unroll") for (int j = 0; j < NWN; ++j) load_bpay<SCHEME>(wrow[j], kb, h, pay[(J + 2) & 3][j]); \
        if (J == 0) {                                                                                \
            const uint32_t nb = blk + 1 < nblk ? blk + 1 : nblk - 1;                                 \
            _Pragma("unroll") for (int j = 0; j < NWN; ++j) load_bhdr<SCHEME>(wrow[j], nb, hnext[j]); \
        }                                                                                            \
        m2_step<SCHEME, J, MT, NWN>(stages[J], pay[J], hcur, lane, lutf, acc);                       \
    }
        R9VX_M2_STEP(0)
        R9VX_M2_STEP(1)
        R9VX_M2_STEP(2)
        R9VX_M2_STEP(3)
#undef R9VX_M2_STEP
    }
    /* The last steps' loads (of steps past the end) are still in flight and
     * their registers are dead to the compiler, which could hand them to the
     * caller's epilogue: wait, then touch them so that they stay reserved up
     * to here. */
    wait_vm<0>();
#pragma unroll
    for (int j = 0; j < NWN; ++j) {
#pragma unroll
        for (int q = 0; q < 4; ++q) touch_pay(pay[q][j]);
        touch_hdr<SCHEME>(hnext[j]);
    }
}

}  // namespace r9vx

#endif
