/* Measurement aids of librsllm_hip.so, for the benchmark (bench.py): the
 * ceilings the HBM-bound kernels and the matrix-core GEMMs are compared
 * with. Not part of the drop-in boundary (rsllm_hip.h): no rsLLM caller
 * uses them, and they have no counterpart in the reference. */
#ifndef RSLLM_HIP_PROBE_H
#define RSLLM_HIP_PROBE_H

#include "rsllm_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* No counterpart in the reference: a pure streaming read of `bytes` bytes at
 * device pointer p (16-byte aligned, a multiple of 16, below 4 GiB), the
 * ceiling the HBM-bound kernels are compared with. n_wg workgroups of
 * `threads` threads (a multiple of 64, at most 1024), each lane with
 * `unroll` (1, 2, 4, 8, 16) 16-byte loads in flight; contiguous != 0: each
 * workgroup reads one contiguous share, else a grid-wide stride. `sink`
 * (device, n_wg * threads words) is written only in the practically
 * impossible case that a lane's xor of its words equals a fixed constant.
 * Enqueued on `stream`. */
int rsllm_hip_stream_read_dev(const uint8_t *p, size_t bytes, uint32_t *sink, size_t sink_len,
                              int n_wg, int threads, int unroll, int contiguous,
                              rsllm_hip_stream_t stream);

/* No counterpart in the reference: the matrix-core issue ceiling the MFMA
 * GEMMs are compared with. n_wg workgroups of 4 wavefronts (one per CU, or
 * two with two_per_cu != 0), each wavefront running `iters` (1..100000)
 * rounds of 32 groups of four independent v_mfma_f32_16x16x32_f16 with
 * valu_per_group (0, 4, 8, 16) independent packed-f16 FMAs after each group:
 * 128 * iters MFMAs of 16384 flops per wavefront. `sink` (device, n_wg * 256
 * words) is written only when a lane's folded result equals a fixed
 * constant. Enqueued on `stream`. */
int rsllm_hip_mfma_issue_dev(uint32_t *sink, size_t sink_len, int n_wg, int iters,
                             int valu_per_group, int two_per_cu, rsllm_hip_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* RSLLM_HIP_PROBE_H */
