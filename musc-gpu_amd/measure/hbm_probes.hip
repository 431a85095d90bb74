// HBM measurement probes (libmusc_measure.so, declared in musc_measure.h): working
// tools that replay memory access patterns, kept out of the product library
// libmusc_hip.so.  musc_hip/kernels_bench.py (the `hbm` command) loads them to measure
// the rates the part reaches for one-shot streams and for the LNAMD stream kernel's
// own access pattern, the ceilings its roofline discussion cites.
#include "../csrc/common.hpp"
#include "musc_measure.h"

// ---------------------------------------------------------------------------
// HBM probes (measurement aids, no counterpart in the reference).
//
// hbm_stream_kernel: one float4 per thread, one-shot grid (no grid-stride loop),
// so the resident workgroups always cover one compact, advancing address window:
// the best-case pattern for HBM on this part.  mode 0 reads (nontemporal loads),
// 1 writes, 2 copies.
//
// lnamd_pattern_kernel: the exact global access pattern of the LNAMD stream kernel
// (workgroup per (image, layer, 64-channel slice), thread (column, 4 channels)
// sweeping the rows, one float4 read per input row and n_radii float4 writes per
// output row into the (R, L, N, P, C) pools) with no arithmetic, LDS or barriers:
// the rate that access pattern itself allows.  kMode 0 replays reads and writes,
// 1 only the writes, 2 only the reads, so the cost of interleaving the two on HBM
// is the difference between mode 0 and the sum of modes 1 and 2.
// ---------------------------------------------------------------------------
namespace musc {
namespace cal {

typedef float cal_f4 __attribute__((ext_vector_type(4)));

template <int kMode>
__global__ __launch_bounds__(1024) void hbm_stream_kernel(const cal_f4* __restrict__ src, cal_f4* __restrict__ dst,
                                                         long long n4) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n4) return;
  if constexpr (kMode == 0) {
    const cal_f4 v = __builtin_nontemporal_load(src + i);
    if (v.x == 1234.5f && v.y == -1234.5f) dst[0] = v;  // keeps the load; never true for the fill used
  } else if constexpr (kMode == 1) {
    const float f = (float)(i & 1023);
    dst[i] = cal_f4{f, f + 1.f, f + 2.f, f + 3.f};
  } else {
    dst[i] = src[i];
  }
}

constexpr int kPatCg = 16;

template <int kMode>
__global__ __launch_bounds__(1024) void lnamd_pattern_kernel(const cal_f4* __restrict__ tokens,
                                                             cal_f4* __restrict__ out, int n, int layers, int tpi,
                                                             int c, int side, int n_radii) {
  const int slices = c / 4 / kPatCg;
  const int unit = blockIdx.x / slices, slice = blockIdx.x % slices;
  const int b = unit / layers, l = unit % layers;
  const int w = threadIdx.x / kPatCg, g = slice * kPatCg + threadIdx.x % kPatCg;
  if (w >= side) return;
  const long long P = (long long)side * side, c4 = c / 4;
  const long long in0 = ((long long)l * n * tpi + (long long)b * tpi + 1) * c4 + (long long)w * c4 + g;
  cal_f4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int h = 0; h < side; ++h) {
    if constexpr (kMode != 1) acc += __builtin_nontemporal_load(tokens + in0 + (long long)h * side * c4);
    const long long p = (long long)h * side + w;
    if constexpr (kMode != 2) {
      for (int k = 0; k < n_radii; ++k) {
        const long long o = ((((long long)k * layers + l) * n + b) * P + p) * c4 + g;
        __builtin_nontemporal_store(acc, out + o);
      }
    }
  }
  if constexpr (kMode == 2) {
    if (acc.x == 1234.5f && acc.y == -1234.5f) out[0] = acc;  // keeps the loads; never true for the fill used
  }
}

}  // namespace cal
}  // namespace musc

using namespace musc;

extern "C" int musc_measure_hbm_stream(int mode, const void* src, void* dst, long long bytes, hipStream_t stream) {
  if (mode < 0 || mode > 2 || bytes < 16 || bytes % 16 || !dst || (mode != 1 && !src)) return MUSC_ERR_INVALID_ARG;
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) % 16) return MUSC_ERR_INVALID_ARG;
  const long long n4 = bytes / 16;
  const long long blocks = (n4 + 255) / 256;
  if (blocks > 0x7fffffffLL) return MUSC_ERR_UNSUPPORTED;
  const auto* s = static_cast<const cal::cal_f4*>(src);
  auto* d = static_cast<cal::cal_f4*>(dst);
  if (mode == 0)  // reads: 1024-thread workgroups measured fastest (writes and copies: 256)
    hipLaunchKernelGGL(cal::hbm_stream_kernel<0>, dim3((unsigned)((n4 + 1023) / 1024)), dim3(1024), 0, stream, s, d,
                       n4);
  else if (mode == 1)
    hipLaunchKernelGGL(cal::hbm_stream_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, stream, s, d, n4);
  else
    hipLaunchKernelGGL(cal::hbm_stream_kernel<2>, dim3((unsigned)blocks), dim3(256), 0, stream, s, d, n4);
  return check_launch();
}

extern "C" int musc_measure_lnamd_pattern(const float* tokens, float* out, int n, int layers, int tokens_per_image,
                                            int c, int n_radii, int mode, hipStream_t stream) {
  if (!tokens || !out || n < 1 || layers < 1 || n_radii < 1 || c < 4 * cal::kPatCg) return MUSC_ERR_INVALID_ARG;
  if (mode < 0 || mode > 2) return MUSC_ERR_INVALID_ARG;
  if (c % (4 * cal::kPatCg)) return MUSC_ERR_UNSUPPORTED;
  int side = 0;
  while ((side + 1) * (side + 1) <= tokens_per_image - 1) ++side;
  if (side * side != tokens_per_image - 1 || side * cal::kPatCg > 1024) return MUSC_ERR_INVALID_ARG;
  if ((reinterpret_cast<uintptr_t>(tokens) | reinterpret_cast<uintptr_t>(out)) % 16) return MUSC_ERR_INVALID_ARG;
  const long long grid = (long long)n * layers * (c / 4 / cal::kPatCg);
  const auto* tk = reinterpret_cast<const cal::cal_f4*>(tokens);
  auto* o = reinterpret_cast<cal::cal_f4*>(out);
  const dim3 g((unsigned)grid), blk(side * cal::kPatCg);
  if (mode == 0)
    hipLaunchKernelGGL(cal::lnamd_pattern_kernel<0>, g, blk, 0, stream, tk, o, n, layers, tokens_per_image, c, side,
                       n_radii);
  else if (mode == 1)
    hipLaunchKernelGGL(cal::lnamd_pattern_kernel<1>, g, blk, 0, stream, tk, o, n, layers, tokens_per_image, c, side,
                       n_radii);
  else
    hipLaunchKernelGGL(cal::lnamd_pattern_kernel<2>, g, blk, 0, stream, tk, o, n, layers, tokens_per_image, c, side,
                       n_radii);
  return check_launch();
}
