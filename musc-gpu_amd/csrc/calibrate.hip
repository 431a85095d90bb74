// Calibration kernel: the sustained fp32 MFMA rate of this device with no memory
// traffic in the loop (each wave issues independent v_mfma_f32_32x32x2f32 on eight
// accumulators back to back).  Used to state how far the hot kernels are from
// what the part delivers under full MFMA load, next to the datasheet peak.  Eight
// chains, not four: with four per wave and every workgroup of the grid resident at
// once (the kernel needs few registers) the loop measured 12 % below the rate that
// one to four waves per SIMD reach with either chain count.
#include "common.hpp"

namespace musc {
namespace cal {

typedef float floatx16 __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256, 2) void mfma_f32_loop(float* __restrict__ out, int iters, float seed) {
  floatx16 acc[8];
#pragma unroll
  for (int b = 0; b < 8; ++b)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[b][v] = 0.f;
  const float a = seed + threadIdx.x * 1e-3f, c = seed - threadIdx.x * 1e-3f;
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int b = 0; b < 8; ++b)   // 64 MFMAs per iteration
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32((b & 1) ? a : c, (b & 2) ? c : a, acc[b], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int b = 0; b < 8; ++b)
#pragma unroll
    for (int v = 0; v < 16; ++v) s += acc[b][v];
  out[(long long)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// fp16 counterpart: independent v_mfma_f32_32x32x16_f16 on eight accumulators (the
// instruction of the split MSM engine).
typedef _Float16 cal_half8 __attribute__((ext_vector_type(8)));

__global__ __launch_bounds__(256, 2) void mfma_f16_loop(float* __restrict__ out, int iters, float seed) {
  floatx16 acc[8];
#pragma unroll
  for (int b = 0; b < 8; ++b)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[b][v] = 0.f;
  cal_half8 a, c;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = (_Float16)(seed + threadIdx.x * 1e-3f + i * 1e-2f);
    c[i] = (_Float16)(seed - threadIdx.x * 1e-3f - i * 1e-2f);
  }
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int b = 0; b < 8; ++b)   // 64 MFMAs per iteration
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16((b & 1) ? a : c, (b & 2) ? c : a, acc[b], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int b = 0; b < 8; ++b)
#pragma unroll
    for (int v = 0; v < 16; ++v) s += acc[b][v];
  out[(long long)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

}  // namespace cal
}  // namespace musc

using namespace musc;

extern "C" int musc_calibrate_mfma_f16(float* out, int blocks, int iters, double* flop, hipStream_t stream) {
  if (!out || blocks < 1 || iters < 1) return MUSC_ERR_INVALID_ARG;
  if (flop) *flop = (double)blocks * 4 /* waves */ * iters * 64 /* MFMAs */ * 32768.0;
  hipLaunchKernelGGL(cal::mfma_f16_loop, dim3(blocks), dim3(256), 0, stream, out, iters, 1.0f);
  return check_launch();
}

extern "C" int musc_calibrate_mfma_f32(float* out, int blocks, int iters, double* flop, hipStream_t stream) {
  if (!out || blocks < 1 || iters < 1) return MUSC_ERR_INVALID_ARG;
  if (flop) *flop = (double)blocks * 4 /* waves */ * iters * 64 /* MFMAs */ * 4096.0;
  hipLaunchKernelGGL(cal::mfma_f32_loop, dim3(blocks), dim3(256), 0, stream, out, iters, 1.0f);
  return check_launch();
}
