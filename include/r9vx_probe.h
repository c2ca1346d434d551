/*
 * r9vx_probe.h -- measured-ceiling probes of libr9vx (diagnostics; no
 * counterpart in the reference's op surface -- the reference measured its
 * ceilings with stand-alone spikes, spikes/dot4-gemv and spikes/wmma-l1).
 */
#ifndef R9VX_PROBE_H
#define R9VX_PROBE_H

#include <stddef.h>
#include <stdint.h>

#include "r9vx.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Streams `bytes` (a multiple of 16) from `src` with 128-bit loads; `sink`
 * (>= r9vx_probe_stream_blocks() u32) is written only if a workgroup's
 * checksum equals a sentinel the caller's fill pattern avoids, so a launch
 * reads and does not write.  Duration / bytes is the measured HBM read
 * ceiling. */
int r9vx_probe_stream_launch(const void *src, uint64_t bytes, uint32_t *sink, r9vx_stream_t stream);
uint32_t r9vx_probe_stream_blocks(uint64_t bytes);
/* Runs `iters` dependent rounds of 16 independent v_mfma_f32_32x32x16_f16
 * per wave on every CU (256 threads x `blocks` workgroups); writes one f32
 * per thread to `sink`.  FLOPs = blocks * 4 waves * iters * 16 * 32768. */
int r9vx_probe_mfma_launch(uint32_t blocks, uint32_t iters, float *sink, r9vx_stream_t stream);

/* Checks the device's routing exp (r9vx_expf.h, all three forms the routing
 * kernels use) on the f32 inputs whose bit patterns are first_bits ..
 * first_bits + n - 1 against want[0..n) (the host libm expf of the same
 * inputs): bad[0..3) (device u32, caller-zeroed) receive the per-form count
 * of outputs with other bits. */
int r9vx_probe_expf_check_launch(uint32_t first_bits, uint32_t n, const float *want, uint32_t *bad,
                                 r9vx_stream_t stream);

/* Relaunches one stage of the grouped (t_bucket > 8) moe_ffn path on a workspace
 * that a completed r9vx_moe_ffn_launch with the same static and args left
 * behind, so a stage's kernel can be timed on its own: stage 1 = the gate/up
 * GEMM (writes the h rows), 2 = the down GEMM (writes the expert output
 * rows), 3 = the weighted combine (writes y).  Each stage reads only what the
 * full launch wrote, so repeating it reproduces the same outputs.  Refused
 * for t_bucket <= 8 (the decode path) and for unknown stages. */
int r9vx_probe_moe_stage_launch(const r9vx_moe_ffn_static *st, const r9vx_moe_ffn_args *args, uint32_t stage,
                                r9vx_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif
