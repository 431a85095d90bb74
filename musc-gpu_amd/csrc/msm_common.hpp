// Pieces shared by the two MSM pair-minima engines (msm.hip: fp32 MFMA;
// msm_split.hip: fp32 products from three fp16 MFMA products): the
// upper-triangular tile enumeration, the row squared norm, the transposing
// min-butterfly of the register epilogues and the workspace layout.
#pragma once

#include <type_traits>

#include "common.hpp"

namespace musc {
namespace msm {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BAND = 8;  // tile rows per band of the tile enumeration
constexpr uint32_t kInfBits = 0x7f800000u;

// ---------------------------------------------------------------------------
// NaN semantics.  The reference's minima come from torch.min over cdist rows
// (models/modules/_MSM.py:16-17), which propagates NaN: a patch whose distance to
// any patch of image j is NaN (a row with a NaN, a zero row that the 0/0 of
// models/musc.py:238 turned into NaN, the inf - inf of the expanded form) has a
// NaN minimum for j.  So the epilogues reduce with the IEEE-754-2019 `minimum`
// (v_minimum3_f32 on gfx950: one instruction, like fminf), never with fminf,
// which drops NaN.
//
// The per-(row, image) minima are merged across tiles with an unsigned atomicMin
// on a key in which NaN orders first: key(x) = 0 for NaN, else bits(max(x, 0)) + 1
// (non-negative floats order like their bits; the +1 makes room for NaN; the
// clamp at 0 is torch.cdist's clamp_min(0) of the squared distance, applied once
// to the tile minimum since max(., 0) commutes with min).  The fill value is
// key(+inf).  Readers subtract 1: NaN becomes 0xffffffff, which orders after
// every number (torch.topk ranks NaN last, _MSM.py:27).
// ---------------------------------------------------------------------------
constexpr uint32_t kMinFill = kInfBits + 1u;  // key(+inf): "no pair seen yet"

__device__ inline float nmin(float a, float b) { return __builtin_elementwise_minimum(a, b); }

__device__ inline uint32_t min_key(float x) {
  return x > 0.f ? __float_as_uint(x) + 1u : (x == x ? 1u : 0u);
}

// key - 1: the squared distance's bits, 0xffffffff for NaN.
__device__ inline uint32_t key_bits(uint32_t key) { return key - 1u; }

// ---------------------------------------------------------------------------
// Tile enumeration.  Tiles (I, J), I <= J < T, are numbered band by band (BAND
// tile rows per band); inside a band the triangle (J < I0 + h) comes first,
// then the rectangle in column-major order, so that the workgroups one XCD runs
// at the same time share a few A and B panels.
// ---------------------------------------------------------------------------
template <int kBand = BAND>
__host__ __device__ inline long long band_prefix(long long s, long long T) {
  // tiles in bands 0..s-1, all of which are full (kBand rows; row i holds T - i tiles)
  return s * kBand * T - (long long)kBand * kBand * s * (s - 1) / 2 - s * (long long)kBand * (kBand - 1) / 2;
}

__host__ __device__ inline long long total_tiles(long long T) { return T * (T + 1) / 2; }

template <int kBand = BAND>
__device__ inline int2 decode_tile(long long w, long long T) {
  const long long nb = (T + kBand - 1) / kBand;
  long long lo = 0, hi = nb - 1;  // largest s with band_prefix(s) <= w
  while (lo < hi) {
    long long mid = (lo + hi + 1) >> 1;
    if (band_prefix<kBand>(mid, T) <= w) lo = mid; else hi = mid - 1;
  }
  const long long s = lo;
  const long long I0 = s * kBand;
  const long long h = (T - I0) < kBand ? (T - I0) : kBand;
  long long q = w - band_prefix<kBand>(s, T);
  const long long tri = h * (h + 1) / 2;
  if (q < tri) {
    long long jl = (long long)((sqrt(8.0 * (double)q + 1.0) - 1.0) * 0.5);
    while ((jl + 1) * (jl + 2) / 2 <= q) ++jl;
    while (jl * (jl + 1) / 2 > q) --jl;
    const long long il = q - jl * (jl + 1) / 2;
    return make_int2((int)(I0 + il), (int)(I0 + jl));
  }
  q -= tri;
  return make_int2((int)(I0 + q % h), (int)(I0 + h + q / h));
}

// Sum of squares of one row in fp64, reduced over the wave (result in every lane).
__device__ inline double row_sumsq(const float* __restrict__ src, int c, int lane) {
  double acc = 0.0;
  if ((c & 3) == 0) {
    const float4* s4 = reinterpret_cast<const float4*>(src);
    for (int k = lane; k < c / 4; k += kWave) {
      float4 v = s4[k];
      acc += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
    }
  } else {
    for (int k = lane; k < c; k += kWave) acc += (double)src[k] * src[k];
  }
  return wave_sum(acc);
}

// Partner value for stage `half` of the transposing min-butterfly over the 32 lanes
// of a half-wave.  Stages 8, 4, 2, 1 use DPP within 16-lane rows (row_ror:8 = lane
// ^ 8; row_half_mirror = lane ^ 7, which flips bit 2 like lane ^ 4 and is an
// equally valid pairing: a lane keeps the half of its items selected by the bit
// being resolved, its partner holds the complementary half of the same item set,
// and the partners met over the five stages still span all 32 lanes); stage 16 is
// the permlane16 swap of transpose_min32.
template <int kHalf>
__device__ inline float butterfly_partner(float v) {
  const int x = __builtin_bit_cast(int, v);
  if constexpr (kHalf == 1) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0xb1, 0xf, 0xf, false));
  if constexpr (kHalf == 2) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x4e, 0xf, 0xf, false));
  if constexpr (kHalf == 4) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x141, 0xf, 0xf, false));
  if constexpr (kHalf == 8) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x128, 0xf, 0xf, false));
  return __shfl_xor(v, kHalf, kWave);
}

// Minimum across the two 32-lane halves of a wave: the lower half receives the
// minimum of its and its partner's item0, the upper half that of item1
// (v_permlane32_swap exchanges VDST's upper half with SRC0's lower half, leaving each
// lane its own kept item in one register and the partner's in the other).
__device__ inline float halves_min2(float item0, float item1) {
  // (__uint_as_float on the elements: clang folds __builtin_bit_cast of the second
  // element of the returned pair to the first)
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(item0), __float_as_uint(item1), false, false);
  return nmin(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// rv[0] of lane lr ends with min over the 32 lanes of item k = lr (items = 32
// values per lane).  The first stage (lane ^ 16, 16 exchanges) uses
// v_permlane16_swap: with rv[q] as VDST and rv[q + 16] as SRC0, the swap of VDST's
// odd 16-lane rows with SRC0's even rows leaves each lane its own kept item in one
// register and its partner's copy of that item in the other, so one swap and one
// minimum replace the select / exchange / select of a shuffle.
__device__ inline float transpose_min32(float (&rv)[32], int lr) {
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(rv[q]), __float_as_uint(rv[q + 16]), false, false);
    rv[q] = nmin(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  auto stage = [&](auto half_c) {
    constexpr int half = decltype(half_c)::value;
    const bool up = (lr & half) != 0;
#pragma unroll
    for (int q = 0; q < half; ++q) {
      const float send = up ? rv[q] : rv[q + half];
      const float keep = up ? rv[q + half] : rv[q];
      rv[q] = nmin(keep, butterfly_partner<half>(send));
    }
  };
  stage(std::integral_constant<int, 8>{});
  stage(std::integral_constant<int, 4>{});
  stage(std::integral_constant<int, 2>{});
  stage(std::integral_constant<int, 1>{});
  return rv[0];
}

// Row index (within a 64-row wave sub-tile) whose minimum transpose_min32 leaves in
// lane (lr, lh): value index k = lr of the 32 values (mb, v) = (k / 16, k % 16).
__device__ inline int transposed_row(int lr, int lh) {
  return (lr >> 4) * 32 + ((lr & 15) >> 2) * 8 + lh * 4 + (lr & 3);
}

// Workspace: norms (n*p fp32) | epilogue row scales (n*p fp32) | minima keys (n*p x n
// uint32, see min_key) | exact-distance row scales (n*p fp32: 1 / ||z_row|| when the
// rows are normalised, else 1) | per-image maximum of norms (n fp32 bits).  The last
// two serve the cancellation refinement (msm_refine_kernel), the same for both engines.
struct Workspace {
  float* norms;
  float* inv;
  uint32_t* minbits;
  float* scale;
  uint32_t* imgmax;
};

inline size_t workspace_bytes(long long n, long long p) {
  const long long rows = n * p;
  return 3 * align_up((size_t)rows * 4, 256) + align_up((size_t)rows * n * 4, 256) + align_up((size_t)n * 4, 256);
}

inline Workspace carve(void* ws, long long n, long long p) {
  const long long rows = n * p;
  const size_t vec = align_up((size_t)rows * 4, 256);
  char* base = static_cast<char*>(ws);
  Workspace w;
  w.norms = reinterpret_cast<float*>(base);
  w.inv = reinterpret_cast<float*>(base + vec);
  w.minbits = reinterpret_cast<uint32_t*>(base + 2 * vec);
  w.scale = reinterpret_cast<float*>(base + 2 * vec + align_up((size_t)rows * n * 4, 256));
  w.imgmax = reinterpret_cast<uint32_t*>(base + 3 * vec + align_up((size_t)rows * n * 4, 256));
  return w;
}

// imgmax[i] = the bits of the largest finite norms[] of image i's p rows (finite only,
// so that one NaN or infinite row does not disable the refinement of its image's
// pairs): one workgroup per image, no atomics.
template <int kUnused = 0>
__global__ __launch_bounds__(256) void image_max_kernel(const float* __restrict__ norms, int p,
                                                        uint32_t* __restrict__ imgmax) {
  __shared__ float part[256 / kWave];
  const float* src = norms + (long long)blockIdx.x * p;
  float m = 0.f;
  for (int q = threadIdx.x; q < p; q += 256) {
    const float v = src[q];
    if (v <= 3.402823466e38f) m = fmaxf(m, v);
  }
  m = wave_max(m);
  if (threadIdx.x % kWave == 0) part[threadIdx.x / kWave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 256 / kWave; ++w) m = fmaxf(m, part[w]);
    imgmax[blockIdx.x] = __float_as_uint(m);
  }
}

inline void launch_image_max(const float* norms, int n, int p, uint32_t* imgmax, hipStream_t s) {
  hipLaunchKernelGGL(image_max_kernel<0>, dim3((unsigned)n), dim3(256), 0, s, norms, p, imgmax);
}

// The fp32 MFMA pair-minima kernel (msm_pair.hip): leaves the squared minima keys.
int run_pairs(const float* z, int n, int p, int c, const Workspace& w, hipStream_t s);

// Trimmed rank means over the minima (defined in msm.hip, shared by both engines).
int run_rank(int n, int p, int a, int b, double* scores, const Workspace& w, hipStream_t s);

// Exact distances for the minima the expanded form cannot resolve (defined in
// msm.hip, shared by both engines; runs after either pair kernel).
int run_refine(const float* z, int n, int p, int c, const Workspace& w, hipStream_t s);

}  // namespace msm
}  // namespace musc
