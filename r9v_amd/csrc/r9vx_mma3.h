/*
 * r9vx_mma3.h -- dequant-GEMM main loop with the weight tile decoded once per
 * workgroup into LDS, shared by the grouped MoE GEMMs and the dense GEMM.
 *
 * Tile: 256 rows x 256 columns, K steps of 64, 512 threads (8 waves, two per
 * SIMD, one workgroup per CU).  LDS: two A stages and two B tiles (128 KiB).
 *   B (weights): thread t decodes half hh = t & 1 of weight row m3_brow(t)
 *     for the next K step while the MFMAs of the current one run: its 16
 *     payload bytes (groups 4hh .. 4hh+3 of the step in the scheme's K
 *     order, r9vx_x16.h order_pos; Q8_0 / Q6_K / IQ3_S: two loads) become 32 fp16 by the
 *     exact f32 formula and one rounding, and each 16-byte granule goes to
 *     the other B tile as soon as it is whole.  Every weight is decoded once
 *     per 256 output rows.
 *   A (activations, fp16 in the same group order): direct global->LDS copies
 *     into the other A stage, one step ahead (tiles of at most 128 rows:
 *     m3_mainloop_half's ring of four 128-row slots, three steps ahead).
 *   MFMA: wave w owns rows 128 (w >> 2) .. +128 (four 32-row tiles, of which
 *     the first NR hold rows of this tile) and two 32-column tiles of B; per
 *     16-K slice it reads 2 B and NR A fragments for 2 NR MFMAs
 *     (v_mfma_f32_32x32x16_f16), fragments two MFMA pairs ahead.
 * Per K step: one barrier (B(k) and A(k) complete; step k - 1's tile and
 * stage free), the A(k + 1) copy and the payload load of step k + 4 issued
 * (into the buffer of payload k, whose B was decoded in step k - 1),
 * then the MFMAs of step k interleaved with the decode and writes of
 * B(k + 1), then a wait for the A(k + 1) copy.
 *
 * Loads are inline assembly waited by count (wait_vm); their registers are
 * tied in and out of the load ("+v") so that a value crossing the loop
 * back-edge keeps one register, and the kernels that use this loop are
 * checked spill-free at build time.
 */
#ifndef R9VX_MMA3_H
#define R9VX_MMA3_H

#include <stddef.h>

#include "r9vx_mfma.h"
#include "r9vx_x16.h"

namespace r9vx {

/* LDS rows are 128 bytes of eight 16-byte groups, group q of row r stored at
 * slot q ^ m2_swz(r): with 64 four-byte LDS banks a 128-byte row covers half
 * the banks, so the 16 rows one LDS read cycle serves (8 even, 8 odd) use 8
 * distinct slots per parity: conflict-free. */
__host__ __device__ constexpr uint32_t m2_swz(uint32_t row) { return (row >> 1) & 7u; }

/*
 * The main loop issues its loads as inline assembly and waits for them itself
 * (wait_vm before each step's barrier).  The compiler's automatic waits cannot
 * tell a copy into one LDS stage from reads of another and count only the
 * loads they know of, so with compiler-visible loads every step would stall
 * on the prefetches of later steps.  touch_pay() marks the point after that
 * wait from which the registers hold the loaded data.  Each load's
 * destination is tied in and out ("+v") and nothing is built from it before
 * the wait, so the register the load writes is the one later read, also for
 * a value carried across the loop back-edge.
 */
__device__ __forceinline__ void touch_pay(r9vx_u32x4 &p) { asm volatile("" : "+v"(p)); }


/* The A row (0..255) that instruction i of wave `wave` copies for this lane
 * (m3_dma_a), and the group of that row the lane copies. */
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

constexpr uint32_t kM3Rows = 256;          /* output rows per tile */
constexpr uint32_t kM3Cols = 256;          /* output columns per tile */
constexpr uint32_t kM3Stage = 256u * 128u; /* one A stage or the B tile: 256 rows of 64 fp16 */
constexpr int kM3AStages = 2;
constexpr int kM3BStages = 2;

/* The IQ4_XS codebook-pair table comes first, so that its LDS address fits
 * the 16-bit offset of ds_read (the byte index, shifted by one SDWA
 * instruction, is the whole address computation of a lookup). */
struct M3Lds {
    uint32_t lut[256];
    uint8_t a[kM3AStages][kM3Stage];
    uint8_t b[kM3BStages][kM3Stage];
};
static_assert(offsetof(M3Lds, b) == offsetof(M3Lds, a) + kM3AStages * kM3Stage, "a and b are contiguous");

/* After the main loop: a and b as one 256 x 512-byte staging tile (an epilogue
 * may stage a 256 x 256 fp16 output tile there). */
__device__ __forceinline__ uint8_t *m3_out_tile(M3Lds &sm) { return reinterpret_cast<uint8_t *>(&sm) + offsetof(M3Lds, a); }

__device__ __forceinline__ uint32_t pack_h2h(_Float16 a, _Float16 b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

/* Byte address of an LDS object, for M0. */
__device__ __forceinline__ uint32_t m3_lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)p;
}

/* Weight row of the decoding thread: a uniform base plus a 32-bit offset
 * (row offset; the step's block / payload offsets are added per load); the
 * split layout (Q8_0) keeps the row's f16 d values at sbase + soff. */
struct M3WRow {
    const uint8_t *base; /* uniform */
    uint32_t off;        /* this thread's row */
    const uint8_t *sbase = nullptr; /* uniform */
    uint32_t soff = 0;
};

/* Q8_0: a thread's half of a K step is one whole block, 32 int8 quants;
 * Q6_K: 16 ql bytes and the 16 qh bytes holding their high bit pairs.  Two
 * 16-byte loads either way, so the payload ring holds two steps in the
 * registers the 4-bit schemes use for four. */
constexpr bool m3_wide(int s) {
    return s == R9VX_SCHEME_Q8_0 || s == R9VX_SCHEME_Q6_K || s == R9VX_SCHEME_IQ3_S;
}
/* Schemes whose decode reads an LDS table (IQ4_XS: codebook pairs; IQ3_S:
 * the signed grid, m3_init_iq3s_lut), ahead of the MFMA pair that uses it. */
constexpr bool m3_table(int s) { return s == R9VX_SCHEME_IQ4_XS || s == R9VX_SCHEME_IQ3_S; }

/* A pointer the caller knows to be wave-uniform, moved to scalar registers
 * (the loads take it as their SGPR base whatever the compiler's divergence
 * analysis concludes). */
__device__ __forceinline__ const uint8_t *m3_uniform(const uint8_t *p) {
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<const uint8_t *>((uintptr_t)(((uint64_t)hi << 32) | lo));
}

/* Payload / header loads with the destination tied in and out. */
template <int SCHEME>
__device__ __forceinline__ void m3_load_pay(const M3WRow &w, uint32_t kt, uint32_t hh, r9vx_u32x4 &p) {
    const uint32_t blk = kt >> 2, ks = kt & 3;
    const uint32_t off = SCHEME == R9VX_SCHEME_Q4_K ? w.off + blk * R9VX_Q4K_BYTES + 16 + 32 * ks + 16 * hh
                                                    : w.off + blk * R9VX_IQ4XS_BYTES + 8 + 32 * ks + 16 * hh;
    asm volatile("global_load_dwordx4 %0, %1, %2" : "+v"(p) : "v"(off), "s"(w.base) : "memory");
}

/* The m3_wide payload of step kt.  Q8_0: block 2 kt + hh, quants 0-15 into
 * p0 and 16-31 into p1.  Q6_K (208-byte body blocks: ql 0-127, qh 128-191,
 * scales 192-207): step s = kt % 4 of block kt / 4 is span n = s / 2, part
 * j = s % 2; p0 = ql bytes 64 n + 32 j + 16 hh .. + 15 (low nibbles: columns
 * 128 n + 32 j + 16 hh + i, high: the same + 64), p1 = qh bytes 32 n + 16 hh
 * .. + 15 (bit pairs j and 2 + j of those columns;
 * crates/r9v-format/src/ggml.rs:817-850).  IQ3_S (112-byte device blocks:
 * grid index bytes 0-63, sign words 64-95, side word 96-111): step s is
 * groups 2 s (hh = 0) and 2 s + 1 (hh = 1) of 32 columns; p0 = their index
 * bytes 16 s .. + 15 (8 per group), p1 = bytes 64 + 8 s .. + 15 (their sign
 * words in .x / .y; .z / .w unused). */
template <int SCHEME>
__device__ __forceinline__ void m3_load_pay2(const M3WRow &w, uint32_t kt, uint32_t hh, r9vx_u32x4 &p0,
                                             r9vx_u32x4 &p1) {
    if constexpr (SCHEME == R9VX_SCHEME_IQ3_S) {
        const uint32_t b = w.off + (kt >> 2) * R9VX_IQ3S_DEV_BYTES, s = kt & 3;
        const uint32_t qs = b + 16 * s, sg = b + 64 + 8 * s;
        asm volatile("global_load_dwordx4 %0, %2, %4\n\tglobal_load_dwordx4 %1, %3, %4"
                     : "+v"(p0), "+v"(p1)
                     : "v"(qs), "v"(sg), "s"(w.base)
                     : "memory");
    } else if constexpr (SCHEME == R9VX_SCHEME_Q6_K) {
        const uint32_t s = kt & 3, b = w.off + (kt >> 2) * R9VX_Q6K_BODY + 16 * hh;
        const uint32_t ql = b + 64 * (s >> 1) + 32 * (s & 1), qh = b + 128 + 32 * (s >> 1);
        asm volatile("global_load_dwordx4 %0, %2, %4\n\tglobal_load_dwordx4 %1, %3, %4"
                     : "+v"(p0), "+v"(p1)
                     : "v"(ql), "v"(qh), "s"(w.base)
                     : "memory");
    } else {
        const uint32_t off = w.off + 64 * kt + 32 * hh;
        asm volatile("global_load_dwordx4 %0, %2, %3\n\tglobal_load_dwordx4 %1, %2, %3 offset:16"
                     : "+v"(p0), "+v"(p1)
                     : "v"(off), "s"(w.base)
                     : "memory");
    }
}

/* Q4_K: the 16-byte header; IQ4_XS: the block's first 16 bytes (its 8-byte
 * header and 8 payload bytes, inside the 136-byte block), of which .x/.y are
 * used; Q8_0: the f16 d values of the eight 32-weight blocks of 256-weight
 * block blk; Q6_K: the block's 16 int8 scales (its d: m3_load_hdr2); IQ3_S:
 * the block's side word (qh bytes of groups 0-3 in .x, 4-7 in .y, the
 * groups' scale nibbles in .z, d in the low half of .w). */
template <int SCHEME>
__device__ __forceinline__ void m3_load_hdr(const M3WRow &w, uint32_t blk, r9vx_u32x4 &hd) {
    if constexpr (SCHEME == R9VX_SCHEME_IQ3_S) {
        const uint32_t off = w.off + blk * R9VX_IQ3S_DEV_BYTES + 96;
        asm volatile("global_load_dwordx4 %0, %1, %2" : "+v"(hd) : "v"(off), "s"(w.base) : "memory");
    } else if constexpr (SCHEME == R9VX_SCHEME_Q8_0) {
        const uint32_t off = w.soff + 16 * blk;
        asm volatile("global_load_dwordx4 %0, %1, %2" : "+v"(hd) : "v"(off), "s"(w.sbase) : "memory");
    } else if constexpr (SCHEME == R9VX_SCHEME_Q6_K) {
        const uint32_t off = w.off + blk * R9VX_Q6K_BODY + 192;
        asm volatile("global_load_dwordx4 %0, %1, %2" : "+v"(hd) : "v"(off), "s"(w.base) : "memory");
    } else {
        const uint32_t off = w.off + blk * (SCHEME == R9VX_SCHEME_Q4_K ? R9VX_Q4K_BYTES : R9VX_IQ4XS_BYTES);
        asm volatile("global_load_dwordx4 %0, %1, %2" : "+v"(hd) : "v"(off), "s"(w.base) : "memory");
    }
}

/* Header loads per block (m3_load_hdr, and m3_load_hdr2 for Q6_K). */
constexpr int m3_hdr_loads(int s) { return s == R9VX_SCHEME_Q6_K ? 2 : 1; }

/* Q6_K: block blk's f16 d from the split layout's d row (zero-extended). */
template <int SCHEME>
__device__ __forceinline__ void m3_load_hdr2(const M3WRow &w, uint32_t blk, uint32_t &d) {
    if constexpr (SCHEME == R9VX_SCHEME_Q6_K) {
        const uint32_t off = w.soff + 2 * blk;
        asm volatile("global_load_ushort %0, %1, %2" : "+v"(d) : "v"(off), "s"(w.sbase) : "memory");
    }
}

/* Direct global->LDS copy of one K step of A (256 rows x 64 fp16, group
 * order): instruction i of wave w fills LDS rows 8(4w + i) .. +8 (1 KiB, lane
 * l at row 8(4w+i) + l/8, slot l%8); aoff[i] is the lane's byte offset from
 * the uniform base `abase` at step 0 (dma_row / dma_group). */
__device__ __forceinline__ void m3_dma_a(uint32_t stage_lds, const _Float16 *abase, const uint32_t (&aoff)[4],
                                         uint32_t kt, uint32_t wave) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t m0 = stage_lds + (wave * 4 + (uint32_t)i) * 1024u;
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(aoff[i] + kt * 128u),
                     "s"(abase), "s"(m0)
                     : "memory", "m0");
    }
}

/* The B row (0..255) that thread tid decodes and writes, two threads per
 * row (tid & 1 picks the 32-element half).  Rows are permuted inside each
 * aligned group of 8 so that the 8 lanes a 128-bit LDS write serves per
 * pass hold 4 rows with distinct swizzles (m2_swz pairs rows 2i, 2i + 1):
 * lanes of threads 2j, 2j + 1, j = 8g .. 8g + 7, take rows 8g + {0, 2, 4, 6,
 * 1, 3, 5, 7}.  With tid >> 1 as the row every write conflicted two ways. */
__device__ __forceinline__ uint32_t m3_brow(uint32_t tid) {
    const uint32_t j = tid >> 1;
    return (j & ~7u) | ((j & 3u) << 1) | ((j >> 2) & 1u);
}

/* IQ4_XS codebook pairs as fp16: entry b = {kv[b & 15], kv[b >> 4]} (1 KiB,
 * exact: the values are integers below 128). */
__device__ __forceinline__ void m3_init_iq4_lut(uint32_t *lut, uint32_t tid, uint32_t nthreads) {
    for (uint32_t b = tid; b < 256; b += nthreads) {
        const _Float16 lo = (_Float16)(float)r9vx_iq4_kvalue(b & 15), hi = (_Float16)(float)r9vx_iq4_kvalue(b >> 4);
        lut[b] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
    }
}

/* IQ3_S: the signed grid as fp16 pairs.  Word (e << 3) | (h << 2) | s (e the
 * 9-bit grid index, h a half of the entry, s two sign bits) holds the fp16
 * 1152 + v0 and 1152 + v1 for values 2h and 2h + 1 of entry e (odd, 1..15),
 * each negated first when its sign bit is set (crates/r9v-format/src/
 * iq.rs:698-722): 16 KiB, so that a lookup of two signed weights is one LDS
 * read. */
constexpr uint32_t kM3Iq3Words = 512 * 8;
__device__ __forceinline__ void m3_init_iq3s_lut(uint32_t *lut, uint32_t tid, uint32_t nthreads) {
    for (uint32_t i = tid; i < kM3Iq3Words; i += nthreads) {
        const uint32_t gw = kIq3sGrid[i >> 3], h = (i >> 2) & 1u, s = i & 3u;
        const uint32_t v0 = (gw >> (16 * h)) & 0xFFu, v1 = (gw >> (16 * h + 8)) & 0xFFu;
        const uint32_t b0 = (s & 1u) ? 128u - v0 : 128u + v0, b1 = (s & 2u) ? 128u - v1 : 128u + v1;
        lut[i] = (0x6400u | b0) | ((0x6400u | b1) << 16);
    }
}

/* Decode unit u (0..7) of a step: payload bytes 2u, 2u + 1 (bytes 4q + 2m,
 * 4q + 2m + 1 of dword q = u / 2, m = u % 2), whose low nibbles are elements
 * 2m, 2m + 1 and high nibbles elements 4 + 2m, 4 + 2m + 1 of group q.  Each
 * weight is the f32 formula (crates/r9v-format/src/ggml.rs:1131-1150,
 * iq.rs:578-598) evaluated in one fused operation and rounded once to fp16
 * (Q4_K: up to the f32 rounding of the precomputed addend, below).
 * Returns the two packed dwords {low pair, high pair}.  IQ4_XS: kv0 / kv1
 * are the bytes' codebook pairs {kv[low], kv[high]}.  Q8_0: the low pair is
 * quants 4q + 2m, +1 (bytes 2m, 2m + 1 of dword q of the first 16 quants,
 * dw), the high pair the same bytes of the second 16 (dw2).  Q6_K: dw the
 * ql dword, dw2 the qh dword; low pair = columns of the low nibbles (bit
 * pair j = KS % 2), high pair = the high nibbles' (bit pair 2 + j).  IQ3_S:
 * kv0 / kv1 are the signed grid pairs (m3_init_iq3s_lut) of the low and high
 * pair. */
template <int SCHEME, int KS = 0>
__device__ __forceinline__ void m3_dec_unit(uint32_t dw, uint32_t dw2, int m, const BScale &sc, uint32_t kv0,
                                            uint32_t kv1, uint32_t &lo2, uint32_t &hi2) {
    if constexpr (SCHEME == R9VX_SCHEME_IQ3_S) {
        /* w = db (1152 +- v) - 1152 db, fused: db v is exact in f32 (db = d
         * (1 + 2 s) has at most 16 significant bits, v 4), as is 1152 db */
        uint32_t a, b;
        asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[0,1,0]" : "=v"(a) : "v"(sc.dl0), "v"(kv0), "v"(sc.c0));
        asm("v_fma_mixhi_f16 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]"
            : "+v"(a) : "v"(sc.dl0), "v"(kv0), "v"(sc.c0));
        asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[0,1,0]" : "=v"(b) : "v"(sc.dl0), "v"(kv1), "v"(sc.c0));
        asm("v_fma_mixhi_f16 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]"
            : "+v"(b) : "v"(sc.dl0), "v"(kv1), "v"(sc.c0));
        lo2 = a;
        hi2 = b;
        asm volatile("" : "+v"(lo2), "+v"(hi2));
    } else if constexpr (SCHEME == R9VX_SCHEME_Q6_K) {
        /* the 6-bit values q (nibble | bit pair << 4) under a 0x64 byte read
         * as the fp16 1024 + q; w = dl (1024 + q) - 1056 dl, fused: dl q -
         * 32 dl with dl = d sc (exact in f32, as is 1056 dl), rounded once */
        constexpr uint32_t j = KS & 1;
        const uint32_t lowq = r9vx_and_or(dw, 0x0F0F0F0Fu, (dw2 << (4 - 2 * j)) & 0x30303030u);
        const uint32_t highq = r9vx_and_or(dw >> 4, 0x0F0F0F0Fu, (dw2 >> (2 * j)) & 0x30303030u);
        const uint32_t sel = m ? 0x04030402u : 0x04010400u;
        const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, lowq, sel);
        const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, highq, sel);
        uint32_t a, b;
        asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[0,1,0]" : "=v"(a) : "v"(sc.dl0), "v"(lo), "v"(sc.c0));
        asm("v_fma_mixhi_f16 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]"
            : "+v"(a) : "v"(sc.dl0), "v"(lo), "v"(sc.c0));
        asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[0,1,0]" : "=v"(b) : "v"(sc.dl1), "v"(hi), "v"(sc.c1));
        asm("v_fma_mixhi_f16 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]"
            : "+v"(b) : "v"(sc.dl1), "v"(hi), "v"(sc.c1));
        lo2 = a;
        hi2 = b;
        asm volatile("" : "+v"(lo2), "+v"(hi2));
    } else if constexpr (SCHEME == R9VX_SCHEME_Q8_0) {
        /* q + 128 (the byte XOR 0x80) under a 0x64 byte reads as the fp16
         * 1152 + q; w = d (1152 + q) - 1152 d, fused: d q is exact in f32
         * (11 + 8 significant bits) and -1152 d too, so the one rounding is
         * fp16(d q), the f32 value rounded once. */
        const uint32_t sel = m ? 0x04030402u : 0x04010400u;
        const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, dw ^ 0x80808080u, sel);
        const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, dw2 ^ 0x80808080u, sel);
        uint32_t a, b;
        asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[0,1,0]" : "=v"(a) : "v"(sc.dl0), "v"(lo), "v"(sc.c0));
        asm("v_fma_mixhi_f16 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]"
            : "+v"(a) : "v"(sc.dl0), "v"(lo), "v"(sc.c0));
        asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[0,1,0]" : "=v"(b) : "v"(sc.dl0), "v"(hi), "v"(sc.c0));
        asm("v_fma_mixhi_f16 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]"
            : "+v"(b) : "v"(sc.dl0), "v"(hi), "v"(sc.c0));
        lo2 = a;
        hi2 = b;
        asm volatile("" : "+v"(lo2), "+v"(hi2));
    } else if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
        /* bytes 2m, 2m + 1 each under a 0x64 byte (v_perm), so that their
         * nibbles read as the fp16 pairs {1024 + lo(2m), 1024 + lo(2m+1)}
         * and {1024 + hi(2m), 1024 + hi(2m+1)}; then w = dl (1024 + q) + c
         * with c = -dmin m - 1024 dl, fused and rounded once to fp16 -- the
         * f32 value dl q - dmin m up to c's own f32 rounding. */
        const uint32_t t = __builtin_amdgcn_perm(0x64646464u, dw, m ? 0x04030402u : 0x04010400u);
        const uint32_t lo = t & 0x640F640Fu, hi = ((t >> 4) & 0x000F000Fu) | 0x64006400u;
        uint32_t a, b;
        asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[0,1,0]" : "=v"(a) : "v"(sc.dl0), "v"(lo), "v"(sc.c0));
        asm("v_fma_mixhi_f16 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]"
            : "+v"(a) : "v"(sc.dl0), "v"(lo), "v"(sc.c0));
        asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[0,1,0]" : "=v"(b) : "v"(sc.dl1), "v"(hi), "v"(sc.c1));
        asm("v_fma_mixhi_f16 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]"
            : "+v"(b) : "v"(sc.dl1), "v"(hi), "v"(sc.c1));
        lo2 = a;
        hi2 = b;
        asm volatile("" : "+v"(lo2), "+v"(hi2));
    } else {
        /* dl * kv is exact in f32 (dl = d * s has 17 significant bits, kv
         * 8), so v_fma_mix with the fp16 codebook value as its operand and
         * 0 as the addend rounds exactly that product to fp16 -- the value
         * of the f32 multiply followed by one fp16 rounding.  mixlo / mixhi
         * write the low / high half of the destination (op_sel picks the
         * codebook half, op_sel_hi marks it as fp16). */
        uint32_t a, b; /* mixlo writes the low half (the high half is then written by mixhi) */
        asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel_hi:[0,1,0]" : "=v"(a) : "v"(sc.dl0), "v"(kv0));
        asm("v_fma_mixhi_f16 %0, %1, %2, 0 op_sel_hi:[0,1,0]" : "+v"(a) : "v"(sc.dl0), "v"(kv1));
        asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(b) : "v"(sc.dl0), "v"(kv0));
        asm("v_fma_mixhi_f16 %0, %1, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "+v"(b) : "v"(sc.dl0), "v"(kv1));
        lo2 = a;
        hi2 = b;
        /* keep the computation here: its only use is at the end of the step,
         * where the compiler's IR passes would otherwise sink it */
        asm volatile("" : "+v"(lo2), "+v"(hi2));
    }
}

/*
 * One K step's compute: the MFMAs of this step (A rows arow0 + 32t for t <
 * NR, B rows bc0 / bc1; the bases are multiples of 32, so a fragment row's
 * swizzle is that of lane % 32) and the decode of the next step's B, whose
 * granules go to bdst (this thread's row of the other B tile, swizzle bsw).
 * Scheduled by hand, each stage fenced so the compiler keeps it: per MFMA
 * pair the fragment and codebook reads that run ahead, the pair, and the
 * decode of one or more payload bytes with the writes it completes.
 */
template <int SCHEME, int KS, int NR, bool TR, bool BSTEP = false>
__device__ __forceinline__ void m3_compute(const uint8_t *ast, const uint8_t *bsm, uint32_t lane, uint32_t arow0,
                                           uint32_t bc0, uint32_t bc1, r9vx_f32x16 (&acc)[4][2],
                                           const r9vx_u32x4 &pay, const r9vx_u32x4 &pay2, const r9vx_u32x4 &hd,
                                           uint32_t hd2, uint32_t hh, const uint32_t *lut, uint8_t *bdst,
                                           uint32_t bsw, uint32_t bsd = 0u) {
    constexpr bool kIq3 = SCHEME == R9VX_SCHEME_IQ3_S;
    constexpr int P = 4 * NR; /* MFMA pairs */
    const uint32_t h = lane >> 5, r32 = lane & 31, sw = m2_swz(r32);
    const uint8_t *arow = ast + (arow0 + r32) * 128u;
    const uint8_t *brow0 = bsm + (bc0 + r32) * 128u, *brow1 = bsm + (bc1 + r32) * 128u;
    auto goff = [&](int s) { return ((4u * h + (uint32_t)s) ^ sw) << 4; };
    const uint32_t dws[4] = {pay.x, pay.y, pay.z, pay.w};
    /* Q8_0: the block's second 16 quants (unused by the 4-bit schemes) */
    const uint32_t dws2[4] = {pay2.x, pay2.y, pay2.z, pay2.w};
    /* IQ4_XS codebook pairs of unit u are read kLead pairs before the pair
     * that decodes it (pair dec_pair(u)), so that their LDS latency and bank
     * conflicts overlap MFMAs; those due before pair 0 are read up front. */
    constexpr int kLead = 2;
    /* the pair after whose MFMAs unit u is decoded */
    auto dec_pair = [](int u) { return ((u + 1) * P + 7) / 8 - 1; };
    uint32_t kv[16];
    const uint8_t *lutb = reinterpret_cast<const uint8_t *>(lut);
    /* IQ3_S: the thread's group 2 KS + hh -- its 8 index bytes (payload
     * dwords 2 hh, 2 hh + 1), sign word and qh byte */
    uint32_t i3d0 = 0u, i3d1 = 0u, i3sg = 0u, i3qh = 0u;
    if constexpr (kIq3) {
        i3d0 = hh ? pay.z : pay.x;
        i3d1 = hh ? pay.w : pay.y;
        i3sg = hh ? pay2.y : pay2.x;
        i3qh = ((KS < 2 ? hd.x : hd.y) >> (8 * (2 * (KS & 1) + hh))) & 0xFFu;
    }
    /* byte address of the grid entry of index i of the group in the signed
     * table: (9-bit entry << 5) = index byte << 5 (one SDWA shift) | qh bit
     * i << 13 */
    auto i3_base = [&](int i) {
        const uint32_t dw = i < 4 ? i3d0 : i3d1;
        uint32_t b5;
        switch (i & 3) {
        case 0:
            asm("v_lshlrev_b32_sdwa %0, 5, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
                : "=v"(b5) : "v"(dw));
            break;
        case 1:
            asm("v_lshlrev_b32_sdwa %0, 5, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1"
                : "=v"(b5) : "v"(dw));
            break;
        case 2:
            asm("v_lshlrev_b32_sdwa %0, 5, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2"
                : "=v"(b5) : "v"(dw));
            break;
        default:
            asm("v_lshlrev_b32_sdwa %0, 5, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
                : "=v"(b5) : "v"(dw));
            break;
        }
        return r9vx_and_or(i3qh << (13 - i), 0x2000u, b5);
    };
    /* sign bits p, p + 1 of the group as the table word's s, times 4 */
    auto i3_sgn = [&](int p) { return p >= 2 ? (i3sg >> (p - 2)) & 0xCu : (i3sg << 2) & 0xCu; };
    auto read_kv = [&](int u) {
        if constexpr (kIq3) {
            /* unit (q, m): values 2m, 2m + 1 of indices 2q (low pair) and
             * 2q + 1 (high pair), signs 8q + 2m and 8q + 4 + 2m */
            const int q = u >> 1, m = u & 1;
            const uint32_t a0 = i3_base(2 * q) | (uint32_t)(16 * m) | i3_sgn(8 * q + 2 * m);
            const uint32_t a1 = i3_base(2 * q + 1) | (uint32_t)(16 * m) | i3_sgn(8 * q + 4 + 2 * m);
            kv[2 * u] = *reinterpret_cast<const uint32_t *>(lutb + a0);
            kv[2 * u + 1] = *reinterpret_cast<const uint32_t *>(lutb + a1);
            return;
        }
        uint32_t o0, o1; /* 4 x bytes 2m, 2m + 1 of the dword, one SDWA shift each */
        if (u & 1) {
            asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2"
                : "=v"(o0) : "v"(dws[u >> 1]));
            asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
                : "=v"(o1) : "v"(dws[u >> 1]));
        } else {
            asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
                : "=v"(o0) : "v"(dws[u >> 1]));
            asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1"
                : "=v"(o1) : "v"(dws[u >> 1]));
        }
        kv[2 * u] = *reinterpret_cast<const uint32_t *>(lutb + o0);
        kv[2 * u + 1] = *reinterpret_cast<const uint32_t *>(lutb + o1);
    };
#pragma unroll
    for (int b = 0; b < 16; ++b) kv[b] = 0u;
    if constexpr (m3_table(SCHEME)) {
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (P == 0 || dec_pair(u) - kLead < 0) read_kv(u);
    }
    const BScale sc = bscale<SCHEME, KS>(hd, hh, hd2);
    uint32_t o[4][4]; /* granule q of the decoded half row */
    /* Fragments are read kAhead pairs before their MFMAs (two when the
     * wave has several row tiles: B of a slice then lands after the slice
     * two back has used its buffer; one otherwise), so that the LDS latency
     * overlaps this wave's earlier MFMAs. */
    constexpr int kAhead = NR >= 2 ? 2 : 1;
    half8 a[kAhead + 1], b[2][2];
    auto read_frags = [&](int j) {
        const int sj = j / NR, tj = j % NR;
        if (tj == 0) {
            b[sj & 1][0] = *reinterpret_cast<const half8 *>(brow0 + goff(sj));
            b[sj & 1][1] = *reinterpret_cast<const half8 *>(brow1 + goff(sj));
        }
        a[j % (kAhead + 1)] = *reinterpret_cast<const half8 *>(arow + 4096u * tj + goff(sj));
    };
#pragma unroll
    for (int j = 0; j < kAhead; ++j)
        if (j < P) read_frags(j);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const int s = i / NR, t = i % NR;
        if (i + kAhead < P) read_frags(i + kAhead);
        if constexpr (m3_table(SCHEME)) {
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (dec_pair(u) - kLead == i) read_kv(u);
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (BSTEP) {
            /* a new 128-K block of A rows: tile t's accumulators (lane: one
             * A row) times 2^(signed byte t of bsd), before its first MFMA of
             * the step */
            if (i < NR) {
                const int d = (int)(int8_t)(uint8_t)(bsd >> (8 * i));
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_amdgcn_ldexpf(acc[i][j][r], d);
            }
        }
        if constexpr (TR) { /* operands swapped: the tile of B . A^T */
            acc[t][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b[s & 1][0], a[i % (kAhead + 1)], acc[t][0], 0, 0, 0);
            acc[t][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b[s & 1][1], a[i % (kAhead + 1)], acc[t][1], 0, 0, 0);
        } else {
            acc[t][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i % (kAhead + 1)], b[s & 1][0], acc[t][0], 0, 0, 0);
            acc[t][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i % (kAhead + 1)], b[s & 1][1], acc[t][1], 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (dec_pair(u) == i) m3_dec_unit<SCHEME, KS>(dws[u >> 1], dws2[u >> 1], u & 1, sc, kv[2 * u], kv[2 * u + 1], o[u >> 1][u & 1], o[u >> 1][2 + (u & 1)]);
        /* granule q of the row is whole once unit 2q + 1 is decoded */
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (dec_pair(2 * q + 1) == i)
                *reinterpret_cast<r9vx_u32x4 *>(bdst + (((4u * hh + q) ^ bsw) << 4)) =
                    r9vx_u32x4{o[q][0], o[q][1], o[q][2], o[q][3]};
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (P == 0) {
#pragma unroll
        for (int u = 0; u < 8; ++u)
            m3_dec_unit<SCHEME, KS>(dws[u >> 1], dws2[u >> 1], u & 1, sc, kv[2 * u], kv[2 * u + 1], o[u >> 1][u & 1], o[u >> 1][2 + (u & 1)]);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            *reinterpret_cast<r9vx_u32x4 *>(bdst + (((4u * hh + q) ^ bsw) << 4)) =
                r9vx_u32x4{o[q][0], o[q][1], o[q][2], o[q][3]};
    }
}

/* Block-scale steps (BS): A rows whose 128-K blocks carry their own
 * power-of-two scales.  bst (LDS) holds, for block b >= 1 and A-row half
 * rh = arow0 / 128, one word per lane & 31 whose byte t is the exponent
 * step e(b - 1) - e(b) of A row 128 rh + 32 t + (lane & 31); at the first
 * step of block b (k = 2b) each tile's accumulators are multiplied by 2^that
 * before the block's MFMAs, so that after the last block they hold the
 * product at the last block's scale.  Block 0's words are 0 (no step). */
constexpr uint32_t kM3MaxBlk = 8; /* blocks with their own words; later blocks read block 0's (no step) */
template <bool ON>
__device__ __forceinline__ uint32_t m3_bsd(const uint32_t *bst, uint32_t k, uint32_t arow0, uint32_t lane) {
    if constexpr (!ON) {
        return 0u;
    } else {
        const uint32_t b = k >> 1;
        return bst[(b < kM3MaxBlk ? b : 0u) * 64u + (arow0 >> 2) + (lane & 31u)];
    }
}

/*
 * The main loop over nk K steps (nk a multiple of 4), with two B tiles and
 * two A stages: one barrier per step.  abase / aoff: the A copy sources
 * (m3_dma_a); w: the decoding thread's weight row; wave: the uniform wave
 * index.  acc must be zero on entry; rows of tiles t >= NR are not computed.
 * The decode of step k + 1's B needs the next super-block's header when
 * J == 3; it is loaded at J == 1 into hnext and copied to hcur at J == 3.
 * Step k: barrier (B(k) and A(k) are complete and visible, and every wave is
 * done with step k - 1's A stage and B tile), the copy of A(k + 1) into the
 * other A stage and the payload load of step k + 4 into the buffer of
 * payload k (plus the next block header when J == 1), then the MFMAs of step k interleaved with the decode
 * of B(k + 1), each of whose four 16-byte granules is written into the other
 * B tile as soon as it is whole, then a wait for the A(k + 1) copy.
 */
/* The first prologue loads of the main loop -- payload 0 and the first
 * block header, in the prologue's order -- issued ahead by a caller that
 * still has LDS work to do (an epilogue); m3_run_pre then runs the loop from
 * them.  Stores the caller issues in between are waited for with them. */
template <int SCHEME>
__device__ __forceinline__ void m3_issue_head(const M3WRow &w, uint32_t tid, r9vx_u32x4 (&pay)[4], r9vx_u32x4 &hnext) {
    const uint32_t hh = tid & 1;
    pay[0] = hnext = r9vx_u32x4{0u, 0u, 0u, 0u};
    m3_load_pay<SCHEME>(w, 0, hh, pay[0]);
    m3_load_hdr<SCHEME>(w, 0, hnext);
}

/* PRE: the caller issued P0 H0 (m3_issue_head), and perhaps stores after
 * them; the prologue then issues what the plain one issues after them (the
 * A(0) copy, payloads 1-3) and goes on with the same counted waits. */
template <int SCHEME, int NR, bool TR, bool BS, bool PRE, class Hook>
__device__ __forceinline__ void m3_mainloop_core(M3Lds &sm, const _Float16 *abase, const uint32_t (&aoff)[4],
                                                 const M3WRow &w, uint32_t nk, uint32_t tid, uint32_t wave,
                                                 const uint32_t *lut, uint32_t arow0, uint32_t bc0, uint32_t bc1,
                                                 r9vx_f32x16 (&acc)[4][2], const uint32_t *bst, Hook &hook,
                                                 r9vx_u32x4 (&pay)[4], r9vx_u32x4 &hnext) {
    const uint32_t lane = tid & 63, c = m3_brow(tid), hh = tid & 1, bsw = m2_swz(c);
    const uint32_t a_lds = m3_lds_addr(&sm.a[0][0]);
    r9vx_u32x4 hcur;
    /* prologue: P0 H0 | A0 | P1 P2 P3; B(0) decoded into B tile 0 */
    if constexpr (!PRE) {
        pay[0] = hnext = r9vx_u32x4{0u, 0u, 0u, 0u};
        m3_load_pay<SCHEME>(w, 0, hh, pay[0]);
        m3_load_hdr<SCHEME>(w, 0, hnext);
    }
    pay[1] = pay[2] = pay[3] = r9vx_u32x4{0u, 0u, 0u, 0u};
    m3_dma_a(a_lds, abase, aoff, 0, wave);
    m3_load_pay<SCHEME>(w, 1, hh, pay[1]);
    m3_load_pay<SCHEME>(w, 2, hh, pay[2]);
    m3_load_pay<SCHEME>(w, 3 < nk ? 3 : nk - 1, hh, pay[3]);
    wait_vm<7>(); /* P0, H0 (and the loads and stores issued before) */
    touch_pay(pay[0]);
    touch_pay(hnext);
    hcur = hnext;
    hook();
    m3_compute<SCHEME, 0, 0, TR>(nullptr, nullptr, lane, 0, 0, 0, acc, pay[0], pay[0], hcur, 0u, hh, lut, sm.b[0] + c * 128u,
                                 bsw);
    wait_vm<2>(); /* A0, P1 */
    touch_pay(pay[1]);

    for (uint32_t k0 = 0; k0 < nk; k0 += 4) {
#define R9VX_M3_STEP_DB(J)                                                                                   \
    {                                                                                                        \
        const uint32_t k = k0 + J;                                                                           \
        lds_barrier(); /* B(k), A(k) visible; step k - 1's tile and stage are free */                        \
        m3_dma_a(a_lds + ((k + 1) & 1u) * kM3Stage, abase, aoff, k + 1 < nk ? k + 1 : nk - 1, wave);          \
        m3_load_pay<SCHEME>(w, k + 4 < nk ? k + 4 : nk - 1, hh, pay[J & 3]);                                  \
        if (J == 1) {                                                                                        \
            const uint32_t blk = (k + 3) / 4 < nk / 4 ? (k + 3) / 4 : nk / 4 - 1;                             \
            m3_load_hdr<SCHEME>(w, blk, hnext);                                                              \
        }                                                                                                    \
        if (J == 3) {                                                                                        \
            touch_pay(hnext);                                                                                \
            hcur = hnext;                                                                                    \
        }                                                                                                    \
        m3_compute<SCHEME, (J + 1) & 3, NR, TR, BS && (J & 1) == 0>(                                          \
            sm.a[k & 1u], sm.b[k & 1u], lane, arow0, bc0, bc1, acc, pay[(J + 1) & 3], pay[(J + 1) & 3], hcur, 0u, hh, lut,           \
            sm.b[(k + 1) & 1u] + c * 128u, bsw, m3_bsd<BS && (J & 1) == 0>(bst, k, arow0, lane));              \
        __builtin_amdgcn_sched_barrier(0);                                                                   \
        wait_vm<(J == 1 ? 2 : 1)>(); /* A(k + 1) copied; payload k + 2 (and the header) arrived */           \
        touch_pay(pay[(J + 2) & 3]);                                                                         \
    }
        R9VX_M3_STEP_DB(0)
        R9VX_M3_STEP_DB(1)
        R9VX_M3_STEP_DB(2)
        R9VX_M3_STEP_DB(3)
#undef R9VX_M3_STEP_DB
    }
    wait_vm<0>();
#pragma unroll
    for (int i = 0; i < 4; ++i) touch_pay(pay[i]);
    touch_pay(hnext);
}

template <int SCHEME, int NR, bool TR, bool BS, class Hook>
__device__ __forceinline__ void m3_mainloop(M3Lds &sm, const _Float16 *abase, const uint32_t (&aoff)[4],
                                            const M3WRow &w, uint32_t nk, uint32_t tid, uint32_t wave,
                                            const uint32_t *lut, uint32_t arow0, uint32_t bc0, uint32_t bc1,
                                            r9vx_f32x16 (&acc)[4][2], const uint32_t *bst, Hook &hook) {
    r9vx_u32x4 pay[4], hnext;
    m3_mainloop_core<SCHEME, NR, TR, BS, false>(sm, abase, aoff, w, nk, tid, wave, lut, arow0, bc0, bc1, acc, bst,
                                                hook, pay, hnext);
}

/*
 * The main loop for the m3_wide schemes (every tile size): a step's payload
 * is the pair pay[2 (k & 1)], pay[2 (k & 1) + 1], loaded two steps ahead.
 * Step k: barrier, the A(k + 1) copy and payload k + 2 (plus the next block's
 * d values when J == 1) issued, the MFMAs of step k with the decode of
 * B(k + 1), then a wait for A(k + 1) and payload k + 2 (the plain loop's
 * wait for A(k + 1) already holds its payload loads to the same step and a
 * half).
 */
template <int SCHEME, int NR, bool TR, bool BS, class Hook>
__device__ __forceinline__ void m3_mainloop_wide(M3Lds &sm, const _Float16 *abase, const uint32_t (&aoff)[4],
                                                 const M3WRow &w, uint32_t nk, uint32_t tid, uint32_t wave,
                                                 const uint32_t *lut, uint32_t arow0, uint32_t bc0, uint32_t bc1,
                                                 r9vx_f32x16 (&acc)[4][2], const uint32_t *bst, Hook &hook) {
    static_assert(m3_wide(SCHEME), "two-load payload schemes only");
    constexpr int kH = m3_hdr_loads(SCHEME);
    const uint32_t lane = tid & 63, c = m3_brow(tid), hh = tid & 1, bsw = m2_swz(c);
    const uint32_t a_lds = m3_lds_addr(&sm.a[0][0]);
    r9vx_u32x4 pay[4], hnext, hcur;
    uint32_t h2next = 0u, h2cur; /* Q6_K: the block's d */
#pragma unroll
    for (int i = 0; i < 4; ++i) pay[i] = r9vx_u32x4{0u, 0u, 0u, 0u};
    hnext = r9vx_u32x4{0u, 0u, 0u, 0u};
    /* prologue: P0 H0 | A0 | P1; B(0) decoded into B tile 0 */
    m3_load_pay2<SCHEME>(w, 0, hh, pay[0], pay[1]);
    m3_load_hdr<SCHEME>(w, 0, hnext);
    m3_load_hdr2<SCHEME>(w, 0, h2next);
    m3_dma_a(a_lds, abase, aoff, 0, wave);
    m3_load_pay2<SCHEME>(w, 1 < nk ? 1 : nk - 1, hh, pay[2], pay[3]);
    wait_vm<6>(); /* P0, H0 (and the loads issued before) */
    touch_pay(pay[0]);
    touch_pay(pay[1]);
    touch_pay(hnext);
    asm volatile("" : "+v"(h2next));
    hcur = hnext;
    h2cur = h2next;
    hook();
    m3_compute<SCHEME, 0, 0, TR>(nullptr, nullptr, lane, 0, 0, 0, acc, pay[0], pay[1], hcur, h2cur, hh, lut,
                                 sm.b[0] + c * 128u, bsw);
    wait_vm<0>(); /* A0, P1 */
    touch_pay(pay[2]);
    touch_pay(pay[3]);

    for (uint32_t k0 = 0; k0 < nk; k0 += 4) {
#define R9VX_M3W_STEP(J)                                                                                     \
    {                                                                                                        \
        const uint32_t k = k0 + J;                                                                           \
        lds_barrier(); /* B(k), A(k) visible; step k - 1's tile and stage are free */                        \
        m3_dma_a(a_lds + ((k + 1) & 1u) * kM3Stage, abase, aoff, k + 1 < nk ? k + 1 : nk - 1, wave);          \
        m3_load_pay2<SCHEME>(w, k + 2 < nk ? k + 2 : nk - 1, hh, pay[2 * (J & 1)], pay[2 * (J & 1) + 1]);     \
        if (J == 1) {                                                                                        \
            const uint32_t blk = (k + 3) / 4 < nk / 4 ? (k + 3) / 4 : nk / 4 - 1;                             \
            m3_load_hdr<SCHEME>(w, blk, hnext);                                                              \
            m3_load_hdr2<SCHEME>(w, blk, h2next);                                                            \
        }                                                                                                    \
        if (J == 3) {                                                                                        \
            touch_pay(hnext);                                                                                \
            asm volatile("" : "+v"(h2next));                                                                 \
            hcur = hnext;                                                                                    \
            h2cur = h2next;                                                                                  \
        }                                                                                                    \
        m3_compute<SCHEME, (J + 1) & 3, NR, TR, BS && (J & 1) == 0>(                                          \
            sm.a[k & 1u], sm.b[k & 1u], lane, arow0, bc0, bc1, acc, pay[2 * ((J + 1) & 1)],                   \
            pay[2 * ((J + 1) & 1) + 1], hcur, h2cur, hh, lut, sm.b[(k + 1) & 1u] + c * 128u, bsw,             \
            m3_bsd<BS && (J & 1) == 0>(bst, k, arow0, lane));                                                \
        __builtin_amdgcn_sched_barrier(0);                                                                   \
        wait_vm<(J == 1 ? kH : 0)>(); /* A(k + 1) copied; payload k + 2 arrived */                           \
        touch_pay(pay[2 * (J & 1)]);                                                                         \
        touch_pay(pay[2 * (J & 1) + 1]);                                                                     \
    }
        R9VX_M3W_STEP(0)
        R9VX_M3W_STEP(1)
        R9VX_M3W_STEP(2)
        R9VX_M3W_STEP(3)
#undef R9VX_M3W_STEP
    }
    wait_vm<0>();
#pragma unroll
    for (int i = 0; i < 4; ++i) touch_pay(pay[i]);
    touch_pay(hnext);
    asm volatile("" : "+v"(h2next));
}

/*
 * The main loop for tiles of at most 128 rows (only waves 0-3 own rows: a
 * wave of rows 128-255 decodes and runs no MFMA).  A step of such a tile has
 * little MFMA work to hide the copy of the next A step behind, so A goes
 * through a ring of four 128-row slots (16 KiB each, the two A stages' space):
 * waves 0-3 copy A(k + 3) at step k into the slot A(k - 1) left, and the
 * other waves copy nothing.  Per step the loads are issued in the order
 * [next block header when J == 0], A(k + 3) (waves 0-3), payload k + 4; the
 * wait at the end of step k is for A(k + 1) and payload k + 2, both issued
 * in step k - 2, so the loads of steps k - 1 and k may stay in flight.  The
 * prologue issues A(1) P(2) and A(2) P(3) as steps -2 and -1 would have.  The
 * block header is loaded at J == 0 and used from J == 3 on (the wait at the
 * end of J == 2 covers it).
 */
template <int SCHEME, int NR, bool TR, bool BS, class Hook>
__device__ __forceinline__ void m3_mainloop_half(M3Lds &sm, const _Float16 *abase, const uint32_t (&aoff)[4],
                                                 const M3WRow &w, uint32_t nk, uint32_t tid, uint32_t wave,
                                                 const uint32_t *lut, uint32_t arow0, uint32_t bc0, uint32_t bc1,
                                                 r9vx_f32x16 (&acc)[4][2], const uint32_t *bst, Hook &hook) {
    constexpr uint32_t kSlot = kM3Stage / 2;
    const uint32_t lane = tid & 63, c = m3_brow(tid), hh = tid & 1, bsw = m2_swz(c);
    const uint32_t a_lds = m3_lds_addr(&sm.a[0][0]);
    const bool dma = wave < 4; /* uniform */
    r9vx_u32x4 pay[4], hnext, hcur;
#pragma unroll
    for (int i = 0; i < 4; ++i) pay[i] = r9vx_u32x4{0u, 0u, 0u, 0u};
    hnext = r9vx_u32x4{0u, 0u, 0u, 0u};
    /* prologue: P0 H0 A0 P1 | A1 P2 | A2 P3; B(0) decoded into B tile 0 */
    m3_load_pay<SCHEME>(w, 0, hh, pay[0]);
    m3_load_hdr<SCHEME>(w, 0, hnext);
    if (dma) m3_dma_a(a_lds, abase, aoff, 0, wave);
    m3_load_pay<SCHEME>(w, 1, hh, pay[1]);
    if (dma) m3_dma_a(a_lds + kSlot, abase, aoff, 1, wave);
    m3_load_pay<SCHEME>(w, 2, hh, pay[2]);
    if (dma) m3_dma_a(a_lds + 2 * kSlot, abase, aoff, 2, wave);
    m3_load_pay<SCHEME>(w, 3, hh, pay[3]);
    if (dma)
        wait_vm<15>(); /* P0, H0 (and the caller's loads issued before) */
    else
        wait_vm<3>();
    touch_pay(pay[0]);
    touch_pay(hnext);
    hcur = hnext;
    hook();
    m3_compute<SCHEME, 0, 0, TR>(nullptr, nullptr, lane, 0, 0, 0, acc, pay[0], pay[0], hcur, 0u, hh, lut, sm.b[0] + c * 128u,
                                 bsw);
    if (dma)
        wait_vm<10>(); /* A0, P1 */
    else
        wait_vm<2>();
    touch_pay(pay[1]);

    for (uint32_t k0 = 0; k0 < nk; k0 += 4) {
#define R9VX_M3H_STEP(J)                                                                                     \
    {                                                                                                        \
        const uint32_t k = k0 + J;                                                                           \
        lds_barrier(); /* B(k), A(k) visible; step k - 1's tile and slot are free */                         \
        if (J == 0) {                                                                                        \
            const uint32_t blk = (k + 4) / 4 < nk / 4 ? (k + 4) / 4 : nk / 4 - 1;                             \
            m3_load_hdr<SCHEME>(w, blk, hnext);                                                              \
        }                                                                                                    \
        if (dma) m3_dma_a(a_lds + ((J + 3) & 3) * kSlot, abase, aoff, k + 3 < nk ? k + 3 : nk - 1, wave);     \
        m3_load_pay<SCHEME>(w, k + 4 < nk ? k + 4 : nk - 1, hh, pay[J & 3]);                                  \
        if (J == 3) {                                                                                        \
            touch_pay(hnext);                                                                                \
            hcur = hnext;                                                                                    \
        }                                                                                                    \
        m3_compute<SCHEME, (J + 1) & 3, NR, TR, BS && (J & 1) == 0>(                                          \
            sm.a[0] + J * kSlot, sm.b[k & 1u], lane, arow0, bc0, bc1, acc, pay[(J + 1) & 3], pay[(J + 1) & 3], hcur, 0u, hh, lut,    \
            sm.b[(k + 1) & 1u] + c * 128u, bsw, m3_bsd<BS && (J & 1) == 0>(bst, k, arow0, lane));              \
        __builtin_amdgcn_sched_barrier(0);                                                                   \
        /* A(k + 1) and payload k + 2 (steps k - 1 and k may stay in flight) */                              \
        if (dma)                                                                                             \
            wait_vm<(J <= 1 ? 11 : 10)>();                                                                   \
        else                                                                                                 \
            wait_vm<(J <= 1 ? 3 : 2)>();                                                                     \
        touch_pay(pay[(J + 2) & 3]);                                                                         \
    }
        R9VX_M3H_STEP(0)
        R9VX_M3H_STEP(1)
        R9VX_M3H_STEP(2)
        R9VX_M3H_STEP(3)
#undef R9VX_M3H_STEP
    }
    wait_vm<0>();
#pragma unroll
    for (int i = 0; i < 4; ++i) touch_pay(pay[i]);
    touch_pay(hnext);
}

/* Number of 32-row tiles of rows [row0, row0 + 128) that hold rows < rows. */
__device__ __forceinline__ uint32_t m3_active_tiles(uint32_t rows, uint32_t row0) {
    if (rows <= row0) return 0;
    const uint32_t n = (rows - row0 + 31) / 32;
    return n < 4 ? n : 4;
}

/* Runs the main loop with the wave's active row-tile count as a constant;
 * half (tiles of at most 128 rows) takes m3_mainloop_half.
 * TR: acc[t][j] holds the transposed tile (B rows bc_j.. as its rows, A rows
 * arow0 + 32 t.. as its columns): lane l then holds A row arow0 + 32 t +
 * (l & 31) and B rows bc_j + 8 (r >> 2) + 4 (l >> 5) + (r & 3). */
struct M3NoHook {
    __device__ void operator()() const {}
};

template <int SCHEME, bool TR = false, bool BS = false, class Hook = M3NoHook>
__device__ __forceinline__ void m3_run(uint32_t nr, bool half, M3Lds &sm, const _Float16 *abase,
                                       const uint32_t (&aoff)[4], const M3WRow &w, uint32_t nk, uint32_t tid,
                                       uint32_t wave, const uint32_t *lut, uint32_t arow0, uint32_t bc0, uint32_t bc1,
                                       r9vx_f32x16 (&acc)[4][2], const uint32_t *bst = nullptr, Hook &&hook = Hook{}) {

#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[t][j][r] = 0.f;
#define R9VX_M3_CASE(LOOP, N) \
    case N: LOOP<SCHEME, N, TR, BS>(sm, abase, aoff, w, nk, tid, wave, lut, arow0, bc0, bc1, acc, bst, hook); break;
    if constexpr (m3_wide(SCHEME)) { /* one loop for every tile size */
        switch (nr) {
            R9VX_M3_CASE(m3_mainloop_wide, 4)
            R9VX_M3_CASE(m3_mainloop_wide, 3)
            R9VX_M3_CASE(m3_mainloop_wide, 2)
            R9VX_M3_CASE(m3_mainloop_wide, 1)
        default: m3_mainloop_wide<SCHEME, 0, TR, BS>(sm, abase, aoff, w, nk, tid, wave, lut, arow0, bc0, bc1, acc, bst, hook); break;
        }
    } else {
        if (half) { /* the tile's rows fit waves 0-3 (uniform over the workgroup) */
            switch (nr) {
                R9VX_M3_CASE(m3_mainloop_half, 4)
                R9VX_M3_CASE(m3_mainloop_half, 3)
                R9VX_M3_CASE(m3_mainloop_half, 2)
                R9VX_M3_CASE(m3_mainloop_half, 1)
            default: m3_mainloop_half<SCHEME, 0, TR, BS>(sm, abase, aoff, w, nk, tid, wave, lut, arow0, bc0, bc1, acc, bst, hook); break;
            }
            return;
        }
        switch (nr) {
            R9VX_M3_CASE(m3_mainloop, 4)
            R9VX_M3_CASE(m3_mainloop, 3)
            R9VX_M3_CASE(m3_mainloop, 2)
            R9VX_M3_CASE(m3_mainloop, 1)
        default: m3_mainloop<SCHEME, 0, TR, BS>(sm, abase, aoff, w, nk, tid, wave, lut, arow0, bc0, bc1, acc, bst, hook); break;
        }
    }
#undef R9VX_M3_CASE
}

/* m3_run's full-tile loop (more than 128 rows) from loads m3_issue_head
 * issued; no hook. */
template <int SCHEME, bool TR = false, bool BS = false>
__device__ __forceinline__ void m3_run_pre(uint32_t nr, M3Lds &sm, const _Float16 *abase, const uint32_t (&aoff)[4],
                                           const M3WRow &w, uint32_t nk, uint32_t tid, uint32_t wave,
                                           const uint32_t *lut, uint32_t arow0, uint32_t bc0, uint32_t bc1,
                                           r9vx_f32x16 (&acc)[4][2], const uint32_t *bst, r9vx_u32x4 (&pay)[4],
                                           r9vx_u32x4 &hnext) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[t][j][r] = 0.f;
    M3NoHook hook;
#define R9VX_M3P_CASE(N)                                                                                          \
    case N:                                                                                                       \
        m3_mainloop_core<SCHEME, N, TR, BS, true>(sm, abase, aoff, w, nk, tid, wave, lut, arow0, bc0, bc1, acc,   \
                                                  bst, hook, pay, hnext);                                         \
        break;
    switch (nr) {
        R9VX_M3P_CASE(4)
        R9VX_M3P_CASE(3)
        R9VX_M3P_CASE(2)
        R9VX_M3P_CASE(1)
    default:
        m3_mainloop_core<SCHEME, 0, TR, BS, true>(sm, abase, aoff, w, nk, tid, wave, lut, arow0, bc0, bc1, acc, bst,
                                                  hook, pay, hnext);
        break;
    }
#undef R9VX_M3P_CASE
}

}  // namespace r9vx

#endif
