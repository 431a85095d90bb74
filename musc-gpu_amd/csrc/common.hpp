// Shared helpers for the libmusc_hip kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/musc_hip.h"

namespace musc {

constexpr int kWave = 64;
// Number of XCDs on MI355X: consecutive workgroup ids are dispatched round-robin
// over them, and each has its own L2.
constexpr int kXcds = 8;

__host__ __device__ inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Remap a linear workgroup id so that each XCD receives one contiguous run of
// logical ids (grid must be padded to a multiple of kXcds).  Logical neighbours
// then share an L2.
__device__ inline long long xcd_logical_id(long long wg, long long grid) {
  const long long per = grid / kXcds;
  return (wg % kXcds) * per + wg / kXcds;
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ inline double wave_sum(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Fill `count` 32-bit words with `value` (used instead of hipMemsetAsync so the
// entry points stay correct under HIP graph capture).  Template so that every
// translation unit carries its own instance.
template <int kUnused = 0>
__global__ void fill_u32_kernel(uint32_t* __restrict__ dst, size_t count, uint32_t value) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < count; i += stride) dst[i] = value;
}

inline void launch_fill_u32(uint32_t* dst, size_t count, uint32_t value, hipStream_t s) {
  if (count == 0) return;
  size_t blocks = (count + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(fill_u32_kernel<0>, dim3((unsigned)blocks), dim3(256), 0, s, dst, count, value);
}

inline int check_launch() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? MUSC_OK : static_cast<int>(e);
}

}  // namespace musc
