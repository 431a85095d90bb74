/*
 * musc_measure.h -- HBM measurement probes (libmusc_measure.so).
 *
 * Working tools, not part of the product library libmusc_hip.so or its header: they
 * replay memory access patterns with no arithmetic so that the rates the part reaches
 * can be stated beside the kernels' rooflines.  No counterpart in the reference.
 * Return codes are those of musc_hip.h (MUSC_OK, MUSC_ERR_*); launches are asynchronous
 * on `stream`.
 */
#ifndef MUSC_MEASURE_H
#define MUSC_MEASURE_H

#include <hip/hip_runtime.h>

#ifdef __cplusplus
extern "C" {
#endif

/* mode 0 reads `bytes` of src (nontemporal loads), 1 writes `bytes` of dst, 2 copies
 * src -> dst; one 16-byte vector per thread in a one-shot grid, the most HBM-friendly
 * pattern (the achievable rate of the part).  16-byte aligned buffers. */
int musc_measure_hbm_stream(int mode, const void* src, void* dst, long long bytes, hipStream_t stream);

/* The global access pattern of the LNAMD streaming kernel (tokens (layers, n,
 * tokens_per_image, c) fp32 read once, n_radii writes of (n_radii, layers, n, P, c) fp32)
 * with no arithmetic: the rate the pattern allows.  mode 0 replays reads and writes,
 * 1 only the writes, 2 only the reads.  c a multiple of 64; 16-byte aligned buffers. */
int musc_measure_lnamd_pattern(const float* tokens, float* out, int n, int layers, int tokens_per_image,
                               int c, int n_radii, int mode, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MUSC_MEASURE_H */
