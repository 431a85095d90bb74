// Elementwise and row-normalisation layers of the ViT encoder blocks, fused.
//
// Reference: models/backbone/open_clip/transformer.py
//   :23-29   LayerNorm that casts back to the input dtype (under fp16 autocast torch
//            casts the input to fp32, normalises, and the module casts back:
//            three passes over the activations),
//   :32-35   QuickGELU x * sigmoid(1.702 x) (three elementwise passes in fp16),
//   :236-248 ResidualAttentionBlock.forward: x = q_x + attn(ln_1(q_x));
//            x = x + mlp(ln_2(x)), mlp = c_fc -> act -> c_proj,
//   model.py:84-87 act = QuickGELU for OpenAI weights, else nn.GELU.
//
// MI355X design
//   layernorm_rows_kernel  one wave per row (width <= 64 * 8 * kMaxChunks halves);
//                          the row stays in registers between the mean pass, the
//                          variance pass (two-pass, fp32) and the write.  With a
//                          residual it first forms s = x + r rounded to the
//                          storage dtype (exactly torch's fp16 add), writes s and
//                          normalises s: the residual add and ln_2 are one pass.
//   activation_kernel      QuickGELU or erf-GELU on 16-byte vectors.  fp16 keeps
//                          torch's roundings: QuickGELU rounds 1.702 x, then the
//                          sigmoid, then the product to fp16, as the three
//                          separate torch ops do; GELU rounds once.  The fp16
//                          sigmoid is formed from the hardware exp2 and reciprocal:
//                          rounded to fp16 it equals torch's expf-and-divide
//                          sigmoid for every fp16 input (an elementwise function
//                          of a 16-bit input, checked over all of them).
#include <hip/hip_fp16.h>

#include "common.hpp"

namespace musc {
namespace enc {

constexpr int kMaxChunks = 4;   // 16-byte chunks per lane: width <= 2048 (fp16), 1024 (fp32)
constexpr int kRowsPerBlock = 4;

template <int kDtype>
struct Vec;
template <>
struct Vec<MUSC_DTYPE_F32> {
  static constexpr int N = 4;
};
template <>
struct Vec<MUSC_DTYPE_F16> {
  static constexpr int N = 8;
};

typedef _Float16 half8 __attribute__((ext_vector_type(8)));

template <int kDtype>
__device__ inline void load_vec(const void* base, long long idx, float (&v)[Vec<kDtype>::N]) {
  if constexpr (kDtype == MUSC_DTYPE_F32) {
    const float4 x = reinterpret_cast<const float4*>(base)[idx];
    v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
  } else {
    const half8 x = reinterpret_cast<const half8*>(base)[idx];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (float)x[j];
  }
}

// Rounds to the storage dtype.
template <int kDtype>
__device__ inline void store_vec(void* base, long long idx, const float (&v)[Vec<kDtype>::N]) {
  if constexpr (kDtype == MUSC_DTYPE_F32) {
    reinterpret_cast<float4*>(base)[idx] = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    half8 x;
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = (_Float16)v[j];
    reinterpret_cast<half8*>(base)[idx] = x;
  }
}

// The fp32 value as a register operand: the backend otherwise folds an fp32 multiply
// and the fp16 conversion of its result into one mixed-precision instruction that
// rounds once (v_fma_mixlo_f16), where torch rounds to fp32 and then to fp16.
__device__ inline float as_fp32(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

template <int kDtype>
__device__ inline float round_to(float v) {
  if constexpr (kDtype == MUSC_DTYPE_F32) return v;
  return (float)(_Float16)v;
}

// grid ceil(rows / kRowsPerBlock), block 256.  A row is width / N vectors; lane
// handles vectors lane + 64 c for c < kC (the last chunk may be partial).  All
// loads of a row (x, residual, weight, bias) are issued before the first use, from
// clamped indices, so a wave waits for memory once.
template <int kDtype, bool kAdd, int kC>
__global__ __launch_bounds__(kRowsPerBlock * kWave) void layernorm_rows_kernel(
    const void* x, const void* r, void* sum_out,  // sum_out may alias x or r (same element read, then written)
    const float* __restrict__ w, const float* __restrict__ b, int rows, int width, float eps,
    void* __restrict__ y) {
  // no contraction: every fp32 result is formed, then rounded to fp16 (a fused
  // multiply-and-convert would round once and differ from torch at ties)
#pragma clang fp contract(off)
  constexpr int N = Vec<kDtype>::N;
  const int lane = threadIdx.x % kWave;
  const long long row = (long long)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave;
  if (row >= rows) return;
  const int vrow = width / N;
  const long long row_vec = (long long)row * vrow;
  float v[kC][N], rv[kC][N], wv[kC][N], bv[kC][N];
  bool ok[kC];
#pragma unroll
  for (int c = 0; c < kC; ++c) {
    const int col = c * kWave + lane;
    ok[c] = col < vrow;
    const int cc = ok[c] ? col : vrow - 1;
    load_vec<kDtype>(x, row_vec + cc, v[c]);
    if constexpr (kAdd) load_vec<kDtype>(r, row_vec + cc, rv[c]);
    if (w) {
      load_vec<MUSC_DTYPE_F32>(w + (long long)cc * N, 0, *reinterpret_cast<float(*)[4]>(&wv[c][0]));
      if constexpr (N == 8) load_vec<MUSC_DTYPE_F32>(w + (long long)cc * N + 4, 0, *reinterpret_cast<float(*)[4]>(&wv[c][4]));
    } else {
#pragma unroll
      for (int j = 0; j < N; ++j) wv[c][j] = 1.f;
    }
    if (b) {
      load_vec<MUSC_DTYPE_F32>(b + (long long)cc * N, 0, *reinterpret_cast<float(*)[4]>(&bv[c][0]));
      if constexpr (N == 8) load_vec<MUSC_DTYPE_F32>(b + (long long)cc * N + 4, 0, *reinterpret_cast<float(*)[4]>(&bv[c][4]));
    } else {
#pragma unroll
      for (int j = 0; j < N; ++j) bv[c][j] = 0.f;
    }
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < kC; ++c) {
    if constexpr (kAdd) {
#pragma unroll
      for (int j = 0; j < N; ++j) v[c][j] = round_to<kDtype>(v[c][j] + rv[c][j]);
      if (ok[c]) store_vec<kDtype>(sum_out, row_vec + c * kWave + lane, v[c]);
    }
#pragma unroll
    for (int j = 0; j < N; ++j) s += ok[c] ? v[c][j] : 0.f;
  }
  const float mean = wave_sum(s) / (float)width;
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < kC; ++c)
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const float d = v[c][j] - mean;
      q += ok[c] ? d * d : 0.f;
    }
  const float rstd = 1.f / sqrtf(wave_sum(q) / (float)width + eps);
#pragma unroll
  for (int c = 0; c < kC; ++c) {
    float o[N];
#pragma unroll
    for (int j = 0; j < N; ++j) o[j] = as_fp32((v[c][j] - mean) * rstd * wv[c][j] + bv[c][j]);
    if (ok[c]) store_vec<kDtype>(y, row_vec + c * kWave + lane, o);
  }
}

// e^-t from the hardware exp2 (about 1 ulp, plus the rounding of t log2 e)
__device__ inline float exp_neg(float t) { return __builtin_amdgcn_exp2f(-t * 1.4426950408889634f); }

// 1 / d for d >= 1 or d = +inf: the hardware reciprocal refined by one Newton step
__device__ inline float recip_ge1(float d) {
  float r = __builtin_amdgcn_rcpf(d);
  const float err = fmaf(-d, r, 1.f);
  r = fmaf(err, r, r);
  return d < INFINITY ? r : 0.f;
}

// n / N vectors, grid-stride.  mode 0: QuickGELU, mode 1: GELU (erf).
template <int kDtype, int kMode>
__global__ __launch_bounds__(256) void activation_kernel(const void* __restrict__ x, void* __restrict__ y,
                                                         long long nvec) {
  // no contraction: 1.702 x is formed in fp32 and then rounded to fp16, as torch's
  // separate multiply does (a fused multiply-and-convert rounds once and differs at ties)
#pragma clang fp contract(off)
  constexpr int N = Vec<kDtype>::N;
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < nvec; i += stride) {
    float v[N];
    load_vec<kDtype>(x, i, v);
#pragma unroll
    for (int j = 0; j < N; ++j) {
      if constexpr (kMode == 0) {
        const float t = round_to<kDtype>(as_fp32(1.702f * v[j]));
        // fp16: exp2 and reciprocal in hardware (one Newton step); fp32: expf and IEEE division
        const float sg = round_to<kDtype>(
            as_fp32(kDtype == MUSC_DTYPE_F16 ? recip_ge1(1.f + exp_neg(t)) : 1.f / (1.f + expf(-t))));
        v[j] = as_fp32(v[j] * sg);
      } else {
        v[j] = as_fp32(0.5f * v[j] * (1.f + erff(v[j] * 0.70710678118654752f)));
      }
    }
    store_vec<kDtype>(y, i, v);
  }
}

}  // namespace enc
}  // namespace musc

using namespace musc;

extern "C" int musc_layernorm_rows(const void* x, const void* residual, void* sum_out, const float* weight,
                                   const float* bias, int dtype, int rows, int width, float eps, void* y,
                                   hipStream_t stream) {
  if (!x || !y || rows < 0 || width < 1 || !(eps >= 0.f)) return MUSC_ERR_INVALID_ARG;
  if (dtype != MUSC_DTYPE_F32 && dtype != MUSC_DTYPE_F16) return MUSC_ERR_INVALID_ARG;
  if (residual && !sum_out) return MUSC_ERR_INVALID_ARG;
  const int n = dtype == MUSC_DTYPE_F32 ? 4 : 8;
  if (width % n != 0 || (width / n + kWave - 1) / kWave > enc::kMaxChunks) return MUSC_ERR_UNSUPPORTED;
  const uintptr_t addr = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y) |
                         reinterpret_cast<uintptr_t>(residual) | reinterpret_cast<uintptr_t>(sum_out) |
                         reinterpret_cast<uintptr_t>(weight) | reinterpret_cast<uintptr_t>(bias);
  if (addr % 16) return MUSC_ERR_INVALID_ARG;
  if (rows == 0) return MUSC_OK;
  const int chunks = (width / n + kWave - 1) / kWave;
  const dim3 grid((unsigned)((rows + enc::kRowsPerBlock - 1) / enc::kRowsPerBlock)), block(enc::kRowsPerBlock * kWave);
#define MUSC_LN_LAUNCH(DT, ADD, C)                                                                               \
  hipLaunchKernelGGL((enc::layernorm_rows_kernel<DT, ADD, C>), grid, block, 0, stream, x, residual, sum_out, weight, \
                     bias, rows, width, eps, y)
#define MUSC_LN_CHUNKS(DT, ADD)                                                                                  \
  switch (chunks) {                                                                                              \
    case 1: MUSC_LN_LAUNCH(DT, ADD, 1); break;                                                                   \
    case 2: MUSC_LN_LAUNCH(DT, ADD, 2); break;                                                                   \
    case 3: MUSC_LN_LAUNCH(DT, ADD, 3); break;                                                                   \
    default: MUSC_LN_LAUNCH(DT, ADD, 4); break;                                                                  \
  }
  if (dtype == MUSC_DTYPE_F32) {
    if (residual) { MUSC_LN_CHUNKS(MUSC_DTYPE_F32, true) } else { MUSC_LN_CHUNKS(MUSC_DTYPE_F32, false) }
  } else {
    if (residual) { MUSC_LN_CHUNKS(MUSC_DTYPE_F16, true) } else { MUSC_LN_CHUNKS(MUSC_DTYPE_F16, false) }
  }
#undef MUSC_LN_CHUNKS
#undef MUSC_LN_LAUNCH
  return check_launch();
}

extern "C" int musc_activation(const void* x, void* y, int dtype, int mode, long long n, hipStream_t stream) {
  if (!x || !y || n < 0) return MUSC_ERR_INVALID_ARG;
  if (dtype != MUSC_DTYPE_F32 && dtype != MUSC_DTYPE_F16) return MUSC_ERR_INVALID_ARG;
  if (mode != MUSC_ACT_QUICK_GELU && mode != MUSC_ACT_GELU) return MUSC_ERR_INVALID_ARG;
  const int vec = dtype == MUSC_DTYPE_F32 ? 4 : 8;
  if (n % vec != 0) return MUSC_ERR_UNSUPPORTED;
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) % 16) return MUSC_ERR_INVALID_ARG;
  if (n == 0) return MUSC_OK;
  const long long nvec = n / vec;
  const long long want = (nvec + 255) / 256;
  const unsigned grid = (unsigned)(want < 65536 ? want : 65536);
#define MUSC_ACT_LAUNCH(DT, MODE)                                                                            \
  hipLaunchKernelGGL((enc::activation_kernel<DT, MODE>), dim3(grid), dim3(256), 0, stream, x, y, nvec)
  if (dtype == MUSC_DTYPE_F32) {
    if (mode == MUSC_ACT_QUICK_GELU) MUSC_ACT_LAUNCH(MUSC_DTYPE_F32, 0); else MUSC_ACT_LAUNCH(MUSC_DTYPE_F32, 1);
  } else {
    if (mode == MUSC_ACT_QUICK_GELU) MUSC_ACT_LAUNCH(MUSC_DTYPE_F16, 0); else MUSC_ACT_LAUNCH(MUSC_DTYPE_F16, 1);
  }
#undef MUSC_ACT_LAUNCH
  return check_launch();
}
