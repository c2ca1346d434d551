/*
 * r9vx_mma3.h -- dequant-GEMM main loop with the weight tile decoded once per
 * workgroup into LDS, shared by the grouped MoE GEMMs.
 *
 * Tile: 256 rows x 256 columns, K steps of 64, 512 threads (8 waves, two per
 * SIMD, one workgroup per CU).
 *   B (weights): thread t decodes half hh = t & 1 of weight row c = t >> 1 for
 *     the next K step while the MFMAs of the current one run: its 16 payload
 *     bytes (groups 4hh .. 4hh+3 of the step, r9vx_mma2.h's K group order)
 *     become 32 fp16 by the exact f32 formula and one rounding, held in
 *     registers, and are written to the single LDS B tile after the step's
 *     first barrier.  Every weight is decoded once per 256 output rows.
 *   A (activations, fp16 in the same group order): direct global->LDS copies
 *     into 3 stages, two steps ahead.
 *   MFMA: wave w owns rows 128 (w >> 2) .. +128 (four 32-row tiles, of which
 *     the first NR hold rows of this tile) and two 32-column tiles of B; per
 *     16-K slice it reads 2 B and NR A fragments for 2 NR MFMAs
 *     (v_mfma_f32_32x32x16_f16).
 * Per K step: barrier (every wave is done reading B and the oldest A stage),
 * B written, this step's loads issued (payload 3 steps ahead, block header
 * with the first payload of its super-block, A copy 2 steps ahead), wait for
 * this step's A copy and the next step's payload, barrier, MFMAs of this step
 * interleaved with the decode of the next.
 *
 * Loads are inline assembly waited by count, as in r9vx_mma2.h; their
 * registers are tied in and out of the load ("+v") so that a value crossing
 * the loop back-edge keeps one register, and the kernels that use this loop
 * are checked spill-free at build time.
 */
#ifndef R9VX_MMA3_H
#define R9VX_MMA3_H

#include "r9vx_mma2.h"

namespace r9vx {

constexpr uint32_t kM3Rows = 256;          /* output rows per tile */
constexpr uint32_t kM3Cols = 256;          /* output columns per tile */
constexpr uint32_t kM3Stage = 256u * 128u; /* one A stage or the B tile: 256 rows of 64 fp16 */
constexpr int kM3AStages = 3;

struct M3Lds {
    uint8_t a[kM3AStages][kM3Stage];
    uint8_t b[kM3Stage];
};

__device__ __forceinline__ uint32_t pack_h2h(_Float16 a, _Float16 b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

/* Byte address of an LDS object, for M0. */
__device__ __forceinline__ uint32_t m3_lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)p;
}

/* Weight row of the decoding thread: a uniform base plus a 32-bit offset
 * (row offset; the step's block / payload offsets are added per load). */
struct M3WRow {
    const uint8_t *base; /* uniform */
    uint32_t off;        /* this thread's row */
};

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

/* Q4_K: the 16-byte header; IQ4_XS: the block's first 16 bytes (its 8-byte
 * header and 8 payload bytes, inside the 136-byte block), of which .x/.y are
 * used. */
template <int SCHEME>
__device__ __forceinline__ void m3_load_hdr(const M3WRow &w, uint32_t blk, r9vx_u32x4 &hd) {
    const uint32_t off = w.off + blk * (SCHEME == R9VX_SCHEME_Q4_K ? R9VX_Q4K_BYTES : R9VX_IQ4XS_BYTES);
    asm volatile("global_load_dwordx4 %0, %1, %2" : "+v"(hd) : "v"(off), "s"(w.base) : "memory");
}

/* Direct global->LDS copy of one K step of A (256 rows x 64 fp16, group
 * order): instruction i of wave w fills LDS rows 8(4w + i) .. +8 (1 KiB, lane
 * l at row 8(4w+i) + l/8, slot l%8); aoff[i] is the lane's byte offset from
 * the uniform base `abase` at step 0 (r9vx_mma2.h dma_row / dma_group). */
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

__device__ __forceinline__ void m3_write_b(uint8_t *b, uint32_t c, uint32_t hh, const r9vx_u32x4 (&v)[4]) {
    uint8_t *row = b + c * 128u;
    const uint32_t sw = m2_swz(c);
#pragma unroll
    for (int s = 0; s < 4; ++s) *reinterpret_cast<r9vx_u32x4 *>(row + (((4u * hh + s) ^ sw) << 4)) = v[s];
}

/* IQ4_XS codebook pairs as fp16: entry b = {kv[b & 15], kv[b >> 4]} (1 KiB,
 * exact: the values are integers below 128). */
__device__ __forceinline__ void m3_init_iq4_lut(uint32_t *lut, uint32_t tid, uint32_t nthreads) {
    for (uint32_t b = tid; b < 256; b += nthreads) {
        const _Float16 lo = (_Float16)(float)r9vx_iq4_kvalue(b & 15), hi = (_Float16)(float)r9vx_iq4_kvalue(b >> 4);
        lut[b] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
    }
}

/* Decode unit u (0..7) of a step: payload bytes 2u, 2u + 1 (bytes 4q + 2m,
 * 4q + 2m + 1 of dword q = u / 2, m = u % 2), whose low nibbles are elements
 * 2m, 2m + 1 and high nibbles elements 4 + 2m, 4 + 2m + 1 of group q.  Each
 * weight is the exact f32 formula rounded once to fp16
 * (crates/r9v-format/src/ggml.rs:1131-1150, iq.rs:578-598).  Returns the two
 * packed dwords {low pair, high pair}.  IQ4_XS: kv0 / kv1 are the bytes'
 * codebook pairs {kv[low], kv[high]}. */
typedef _Float16 m3_h2 __attribute__((ext_vector_type(2)));
template <int SCHEME>
__device__ __forceinline__ void m3_dec_unit(uint32_t dw, int m, const BScale &sc, uint32_t kv0, uint32_t kv1,
                                            uint32_t &lo2, uint32_t &hi2) {
    m3_h2 l, h;
    if constexpr (SCHEME == R9VX_SCHEME_Q4_K) {
        uint32_t l4 = dw & 0x0F0F0F0Fu, h4 = (dw >> 4) & 0x0F0F0F0Fu;
        /* hide the masks' known-zero bits, so that each nibble becomes one
         * byte-select conversion (v_cvt_f32_ubyteN) */
        asm volatile("" : "+v"(l4), "+v"(h4));
        l.x = (_Float16)fmaf(sc.dl0, (float)((l4 >> (16 * m)) & 0xFFu), sc.nml0);
        l.y = (_Float16)fmaf(sc.dl0, (float)((l4 >> (16 * m + 8)) & 0xFFu), sc.nml0);
        h.x = (_Float16)fmaf(sc.dl1, (float)((h4 >> (16 * m)) & 0xFFu), sc.nml1);
        h.y = (_Float16)fmaf(sc.dl1, (float)((h4 >> (16 * m + 8)) & 0xFFu), sc.nml1);
    } else {
        /* dl * kv is exact in f32 (dl = d * s has 17 significant bits, kv
         * 8), so v_fma_mix with the fp16 codebook value as its operand and
         * 0 as the addend rounds exactly that product to fp16 -- the value
         * of the f32 multiply followed by one fp16 rounding.  mixlo / mixhi
         * write the low / high half of the destination (op_sel picks the
         * codebook half, op_sel_hi marks it as fp16). */
        uint32_t a = 0, b = 0;
        asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel_hi:[0,1,0]" : "+v"(a) : "v"(sc.dl0), "v"(kv0));
        asm("v_fma_mixhi_f16 %0, %1, %2, 0 op_sel_hi:[0,1,0]" : "+v"(a) : "v"(sc.dl0), "v"(kv1));
        asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "+v"(b) : "v"(sc.dl0), "v"(kv0));
        asm("v_fma_mixhi_f16 %0, %1, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "+v"(b) : "v"(sc.dl0), "v"(kv1));
        lo2 = a;
        hi2 = b;
        asm volatile("" : "+v"(lo2), "+v"(hi2));
        return;
    }
    lo2 = __builtin_bit_cast(uint32_t, l);
    hi2 = __builtin_bit_cast(uint32_t, h);
    /* keep the computation here: its only use is at the end of the step,
     * where the compiler's IR passes would otherwise sink it */
    asm volatile("" : "+v"(lo2), "+v"(hi2));
}

/*
 * One K step's compute: the MFMAs of this step (A rows arow0 + 32t for t <
 * NR, B rows bc0 / bc1; the bases are multiples of 32, so a fragment row's
 * swizzle is that of lane % 32) and the decode of the next step's B into
 * `out`.  Scheduled by hand, each stage fenced so the compiler keeps it:
 * the step's 16 codebook reads (IQ4_XS) and first fragments, then per MFMA
 * pair the fragment reads of the next pair (B of a slice with the last A of
 * the previous one), the pair, and the decode of one or more payload bytes.
 */
template <int SCHEME, int KS, int NR, bool TR>
__device__ __forceinline__ void m3_compute(const uint8_t *ast, const uint8_t *bsm, uint32_t lane, uint32_t arow0,
                                           uint32_t bc0, uint32_t bc1, r9vx_f32x16 (&acc)[4][2],
                                           const r9vx_u32x4 &pay, const r9vx_u32x4 &hd, uint32_t hh,
                                           const uint32_t *lut, r9vx_u32x4 (&out)[4]) {
    constexpr bool kIq4 = SCHEME == R9VX_SCHEME_IQ4_XS;
    constexpr int P = 4 * NR; /* MFMA pairs */
    const uint32_t h = lane >> 5, r32 = lane & 31, sw = m2_swz(r32);
    const uint8_t *arow = ast + (arow0 + r32) * 128u;
    const uint8_t *brow0 = bsm + (bc0 + r32) * 128u, *brow1 = bsm + (bc1 + r32) * 128u;
    auto goff = [&](int s) { return ((4u * h + (uint32_t)s) ^ sw) << 4; };
    const uint32_t dws[4] = {pay.x, pay.y, pay.z, pay.w};
    uint32_t kv[16];
    if constexpr (kIq4) {
#pragma unroll
        for (int b = 0; b < 16; ++b) kv[b] = lut[(dws[b >> 2] >> (8 * (b & 3))) & 0xFFu];
    } else {
#pragma unroll
        for (int b = 0; b < 16; ++b) kv[b] = 0u;
    }
    const BScale sc = bscale<SCHEME, KS>(hd, hh);
    uint32_t o[4][4]; /* out[q] words */
    half8 a[2], b[2][2];
    if constexpr (P > 0) {
        b[0][0] = *reinterpret_cast<const half8 *>(brow0 + goff(0));
        b[0][1] = *reinterpret_cast<const half8 *>(brow1 + goff(0));
        a[0] = *reinterpret_cast<const half8 *>(arow + goff(0));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const int s = i / NR, t = i % NR;
        if (i + 1 < P) { /* the next pair's fragments, a whole pair ahead of their use */
            const int s1 = (i + 1) / NR, t1 = (i + 1) % NR;
            if (t1 == 0) {
                b[s1 & 1][0] = *reinterpret_cast<const half8 *>(brow0 + goff(s1));
                b[s1 & 1][1] = *reinterpret_cast<const half8 *>(brow1 + goff(s1));
            }
            a[(i + 1) & 1] = *reinterpret_cast<const half8 *>(arow + 4096u * t1 + goff(s1));
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (TR) { /* operands swapped: the tile of B . A^T */
            acc[t][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b[s & 1][0], a[i & 1], acc[t][0], 0, 0, 0);
            acc[t][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b[s & 1][1], a[i & 1], acc[t][1], 0, 0, 0);
        } else {
            acc[t][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i & 1], b[s & 1][0], acc[t][0], 0, 0, 0);
            acc[t][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i & 1], b[s & 1][1], acc[t][1], 0, 0, 0);
        }
        /* decode units [8 i / P, 8 (i + 1) / P) */
#pragma unroll
        for (int u = 8 * i / P; u < 8 * (i + 1) / P; ++u)
            m3_dec_unit<SCHEME>(dws[u >> 1], u & 1, sc, kv[2 * u], kv[2 * u + 1], o[u >> 1][u & 1], o[u >> 1][2 + (u & 1)]);
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (P == 0) {
#pragma unroll
        for (int u = 0; u < 8; ++u)
            m3_dec_unit<SCHEME>(dws[u >> 1], u & 1, sc, kv[2 * u], kv[2 * u + 1], o[u >> 1][u & 1], o[u >> 1][2 + (u & 1)]);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) out[q] = r9vx_u32x4{o[q][0], o[q][1], o[q][2], o[q][3]};
}

/* Loads in flight after step J's issue that may still be outstanding when
 * step J waits (those of steps J-1 and J; a step issues 5, 6 when it also
 * loads the next block header, which step J == 1 of a super-block does). */
template <int J>
constexpr int m3_allowed() {
    return (J == 1 || J == 2) ? 11 : 10;
}

/*
 * The main loop over nk K steps (nk a multiple of 4).  abase / aoff: the A
 * copy sources (m3_dma_a); w: the decoding thread's weight row; wave: the
 * uniform wave index.  acc must be zero on entry; rows of tiles t >= NR are
 * not computed.  Step J of a super-block decodes the next step's B, which
 * is in the next super-block when J == 3; that block's header arrives in
 * hnext (loaded at J == 1) and is copied to hcur once it has arrived.
 */
template <int SCHEME, int NR, bool TR>
__device__ __forceinline__ void m3_mainloop(M3Lds &sm, const _Float16 *abase, const uint32_t (&aoff)[4],
                                            const M3WRow &w, uint32_t nk, uint32_t tid, uint32_t wave,
                                            const uint32_t *lut, uint32_t arow0, uint32_t bc0, uint32_t bc1,
                                            r9vx_f32x16 (&acc)[4][2]) {
    const uint32_t lane = tid & 63, c = tid >> 1, hh = tid & 1;
    const uint32_t a_lds = m3_lds_addr(&sm.a[0][0]);
    r9vx_u32x4 pay[4], hnext, hcur, bdec[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) pay[i] = r9vx_u32x4{0u, 0u, 0u, 0u};
    hnext = r9vx_u32x4{0u, 0u, 0u, 0u};
    /* prologue in the steady-state order: P0 H0 | P1 A0 | P2 A1 */
    m3_load_pay<SCHEME>(w, 0, hh, pay[0]);
    m3_load_hdr<SCHEME>(w, 0, hnext);
    m3_load_pay<SCHEME>(w, 1, hh, pay[1]);
    m3_dma_a(a_lds, abase, aoff, 0, wave);
    m3_load_pay<SCHEME>(w, 2, hh, pay[2]);
    m3_dma_a(a_lds + kM3Stage, abase, aoff, 1, wave);
    wait_vm<10>();
    touch_pay(pay[0]);
    touch_pay(hnext);
    hcur = hnext;
    m3_compute<SCHEME, 0, 0, TR>(nullptr, nullptr, lane, 0, 0, 0, acc, pay[0], hcur, hh, lut, bdec);

    uint32_t s_cur = 0; /* A stage of step k; step k + 2 copies into (s_cur + 2) % 3 */
    for (uint32_t k0 = 0; k0 < nk; k0 += 4) {
#define R9VX_M3_STEP(J)                                                                                      \
    {                                                                                                        \
        const uint32_t k = k0 + J;                                                                           \
        lds_barrier(); /* every wave is done with B(k-1) and A stage (k-1) % 3 */                            \
        m3_write_b(sm.b, c, hh, bdec);                                                                       \
        m3_load_pay<SCHEME>(w, k + 3 < nk ? k + 3 : nk - 1, hh, pay[(J + 3) & 3]);                            \
        if (J == 1) {                                                                                        \
            const uint32_t blk = (k + 3) / 4 < nk / 4 ? (k + 3) / 4 : nk / 4 - 1;                             \
            m3_load_hdr<SCHEME>(w, blk, hnext);                                                              \
        }                                                                                                    \
        const uint32_t s_next2 = s_cur == 0 ? 2u : s_cur - 1; /* (s_cur + 2) % 3 */                          \
        m3_dma_a(a_lds + s_next2 * kM3Stage, abase, aoff, k + 2 < nk ? k + 2 : nk - 1, wave);                 \
        wait_vm<m3_allowed<J>()>(); /* A(k) copied, payload (and header) of k + 1 here */                   \
        touch_pay(pay[(J + 1) & 3]);                                                                         \
        if (J == 3) {                                                                                        \
            touch_pay(hnext);                                                                                \
            hcur = hnext;                                                                                    \
        }                                                                                                    \
        lds_barrier(); /* every wave's A(k) copy and B(k) */                                                 \
        m3_compute<SCHEME, (J + 1) & 3, NR, TR>(sm.a[s_cur], sm.b, lane, arow0, bc0, bc1, acc, pay[(J + 1) & 3],  \
                                            hcur, hh, lut, bdec);                                            \
        __builtin_amdgcn_sched_barrier(0);                                                                   \
        s_cur = s_cur == 2 ? 0u : s_cur + 1;                                                                 \
    }
        R9VX_M3_STEP(0)
        R9VX_M3_STEP(1)
        R9VX_M3_STEP(2)
        R9VX_M3_STEP(3)
#undef R9VX_M3_STEP
    }
    /* The clamped loads of the last steps are still in flight into registers
     * the compiler sees as dead and LDS stages the caller may reuse: wait,
     * and keep the registers reserved up to here. */
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

/* Runs the main loop with the wave's active row-tile count as a constant.
 * TR: acc[t][j] holds the transposed tile (B rows bc_j.. as its rows, A rows
 * arow0 + 32 t.. as its columns): lane l then holds A row arow0 + 32 t +
 * (l & 31) and B rows bc_j + 8 (r >> 2) + 4 (l >> 5) + (r & 3). */
template <int SCHEME, bool TR = false>
__device__ __forceinline__ void m3_run(uint32_t nr, M3Lds &sm, const _Float16 *abase, const uint32_t (&aoff)[4],
                                       const M3WRow &w, uint32_t nk, uint32_t tid, uint32_t wave, const uint32_t *lut,
                                       uint32_t arow0, uint32_t bc0, uint32_t bc1, r9vx_f32x16 (&acc)[4][2]) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[t][j][r] = 0.f;
    switch (nr) {
    case 4: m3_mainloop<SCHEME, 4, TR>(sm, abase, aoff, w, nk, tid, wave, lut, arow0, bc0, bc1, acc); break;
    case 3: m3_mainloop<SCHEME, 3, TR>(sm, abase, aoff, w, nk, tid, wave, lut, arow0, bc0, bc1, acc); break;
    case 2: m3_mainloop<SCHEME, 2, TR>(sm, abase, aoff, w, nk, tid, wave, lut, arow0, bc0, bc1, acc); break;
    case 1: m3_mainloop<SCHEME, 1, TR>(sm, abase, aoff, w, nk, tid, wave, lut, arow0, bc0, bc1, acc); break;
    default: m3_mainloop<SCHEME, 0, TR>(sm, abase, aoff, w, nk, tid, wave, lut, arow0, bc0, bc1, acc); break;
    }
}

}  // namespace r9vx

#endif
