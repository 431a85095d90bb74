// LNAMD neighbourhood aggregation for gfx950 (HBM-bound).
//
// Reference semantics (models/modules/_LNAMD.py:72-129; the identity used by
// models/modules/_encoder_gpu.py:14-42): per image and layer, LayerNorm over all
// C*side*side values (biased variance, eps, unit weight, zero bias), then an r x r
// box mean with zero padding r//2 and divisor r*r (count_include_pad), for every
// requested radius; models/musc.py:238 then divides each patch by its L2 norm.
//
// MI355X design
//   lnamd_stats_kernel     per (image, layer): kChunks workgroups stream disjoint
//                          slices and write shifted fp64 partial sums.
//   lnamd_finalize_kernel  per (image, layer): mean and 1/sqrt(var + eps).
//   lnamd_pool_kernel      one workgroup per (image, layer, output row); each
//                          thread owns 4 channels.  It sweeps the row's columns,
//                          reading the 2*hmax+1 input rows once per column, keeps
//                          vertical sums for every radius in a small register
//                          window, and emits all radii of one column from that one
//                          read.  Optional fused L2 normalisation reduces each
//                          patch's squared norm across the workgroup, batched over
//                          kColBatch columns per barrier.  Consecutive rows of one
//                          image are mapped to one XCD so the 2*hmax+1-fold row
//                          reuse is served by that XCD's L2.
#include <hip/hip_fp16.h>

#include "common.hpp"

namespace musc {
namespace lnamd {

constexpr int kChunks = 16;       // stats workgroups per (image, layer)
constexpr int kMaxRadii = 4;
constexpr int kMaxHalo = 4;       // radius <= 9
constexpr int kColBatch = 4;      // columns per normalisation barrier

struct Radii {
  int r[kMaxRadii];
  int n;
};

struct TokenPtrs {
  const void* p[16];
};
constexpr int kMaxLayers = 16;

template <int kDtype>
__device__ inline float4 load4(const void* base, long long idx4) {
  if (kDtype == MUSC_DTYPE_F32) {
    return reinterpret_cast<const float4*>(base)[idx4];
  } else {
    const uint2 raw = reinterpret_cast<const uint2*>(base)[idx4];
    const __half2 lo = *reinterpret_cast<const __half2*>(&raw.x);
    const __half2 hi = *reinterpret_cast<const __half2*>(&raw.y);
    const float2 a = __half22float2(lo), b = __half22float2(hi);
    return make_float4(a.x, a.y, b.x, b.y);
  }
}

template <int kDtype>
__device__ inline float load1(const void* base, long long idx) {
  if (kDtype == MUSC_DTYPE_F32) return reinterpret_cast<const float*>(base)[idx];
  return __half2float(reinterpret_cast<const __half*>(base)[idx]);
}

// grid: units * kChunks, block 256.  unit = b * n_layers + l.
template <int kDtype>
__global__ __launch_bounds__(256) void lnamd_stats_kernel(TokenPtrs tokens, int n_layers, int batch,
                                                          int tokens_per_image, int c, int has_cls,
                                                          double* __restrict__ partials) {
  const int unit = blockIdx.x / kChunks, chunk = blockIdx.x % kChunks;
  const int b = unit / n_layers, l = unit % n_layers;
  const void* base = tokens.p[l];
  const long long grid_vals = (long long)(tokens_per_image - has_cls) * c;
  const long long first = ((long long)b * tokens_per_image + has_cls) * c;  // element index
  const float shift = load1<kDtype>(base, first);
  const long long n4 = grid_vals / 4;  // c % 4 == 0
  const long long per = (n4 + kChunks - 1) / kChunks;
  const long long lo = chunk * per, hi = lo + per < n4 ? lo + per : n4;
  double s = 0.0, ss = 0.0;
  for (long long i = lo + threadIdx.x; i < hi; i += blockDim.x) {
    const float4 v = load4<kDtype>(base, first / 4 + i);
    const float d0 = v.x - shift, d1 = v.y - shift, d2 = v.z - shift, d3 = v.w - shift;
    s += (double)d0 + (double)d1 + (double)d2 + (double)d3;
    ss += (double)d0 * d0 + (double)d1 * d1 + (double)d2 * d2 + (double)d3 * d3;
  }
  s = wave_sum(s);
  ss = wave_sum(ss);
  __shared__ double red[2][4];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (lane == 0) {
    red[0][wave] = s;
    red[1][wave] = ss;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double a = 0.0, q = 0.0;
    for (int w = 0; w < (int)(blockDim.x / kWave); ++w) {
      a += red[0][w];
      q += red[1][w];
    }
    partials[(size_t)blockIdx.x * 2 + 0] = a;
    partials[(size_t)blockIdx.x * 2 + 1] = q;
  }
}

// stats[unit] = {mean, rstd}
template <int kDtype>
__global__ void lnamd_finalize_kernel(TokenPtrs tokens, int n_layers, int units, int tokens_per_image, int c,
                                      int has_cls, float eps, const double* __restrict__ partials,
                                      double* __restrict__ stats) {
  const int unit = blockIdx.x * blockDim.x + threadIdx.x;
  if (unit >= units) return;
  const int b = unit / n_layers, l = unit % n_layers;
  const long long first = ((long long)b * tokens_per_image + has_cls) * c;
  const double shift = (double)load1<kDtype>(tokens.p[l], first);
  double s = 0.0, ss = 0.0;
  for (int k = 0; k < kChunks; ++k) {
    s += partials[((size_t)unit * kChunks + k) * 2 + 0];
    ss += partials[((size_t)unit * kChunks + k) * 2 + 1];
  }
  const double count = (double)(tokens_per_image - has_cls) * c;
  const double dm = s / count;
  double var = ss / count - dm * dm;
  if (var < 0.0) var = 0.0;
  stats[unit * 2 + 0] = shift + dm;
  stats[unit * 2 + 1] = 1.0 / sqrt(var + (double)eps);
}

__device__ inline float4 f4add(float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); }
__device__ inline float4 f4scale(float4 a, float s) { return make_float4(a.x * s, a.y * s, a.z * s, a.w * s); }
__device__ inline float f4dot(float4 a) { return a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w; }

// grid: xcd-padded units * side; block = c/4 threads rounded up to a wave multiple.
template <int kDtype, int kHalo, int kNR>
__global__ __launch_bounds__(1024) void lnamd_pool_kernel(TokenPtrs tokens, int n_layers, int batch,
                                                          int tokens_per_image, int c, int has_cls, int side,
                                                          Radii radii, int l2norm, int layout,
                                                          const double* __restrict__ stats,
                                                          float* __restrict__ out, long long work) {
  const long long wid = xcd_logical_id(blockIdx.x, gridDim.x);
  if (wid >= work) return;
  const int unit = (int)(wid / side), h = (int)(wid % side);
  const int b = unit / n_layers, l = unit % n_layers;
  const int g = threadIdx.x;  // channel group (4 channels)
  const int groups = c / 4;
  const bool act = g < groups;
  const void* base = tokens.p[l];
  const float mean = (float)stats[unit * 2 + 0];
  const float rstd = (float)stats[unit * 2 + 1];
  const int P = side * side;
  const long long img_base4 = (((long long)b * tokens_per_image + has_cls) * c) / 4;

  __shared__ float red[kNR * kColBatch][16];
  const int nwaves = (blockDim.x + kWave - 1) / kWave;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;

  // vertical sums window: win[k][i] = V_{radius k}(column wo - kHalo + i)
  float4 win[kNR][2 * kHalo + 1];
#pragma unroll
  for (int k = 0; k < kNR; ++k)
#pragma unroll
    for (int i = 0; i < 2 * kHalo + 1; ++i) win[k][i] = make_float4(0.f, 0.f, 0.f, 0.f);

  // Shift the window left by one column and append the vertical sums of input
  // column wi (zero outside the image).
  auto push = [&](int wi) {
#pragma unroll
    for (int k = 0; k < kNR; ++k)
#pragma unroll
      for (int i = 0; i < 2 * kHalo; ++i) win[k][i] = win[k][i + 1];
    float4 vs[kNR];
#pragma unroll
    for (int k = 0; k < kNR; ++k) vs[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (wi < side && act) {
#pragma unroll
      for (int dy = -kHalo; dy <= kHalo; ++dy) {
        const int hh = h + dy;
        if (hh < 0 || hh >= side) continue;
        float4 x = load4<kDtype>(base, img_base4 + ((long long)(hh * side + wi) * c) / 4 + g);
        x = make_float4((x.x - mean) * rstd, (x.y - mean) * rstd, (x.z - mean) * rstd, (x.w - mean) * rstd);
        const int ady = dy < 0 ? -dy : dy;
#pragma unroll
        for (int k = 0; k < kNR; ++k)
          if (ady <= radii.r[k] / 2) vs[k] = f4add(vs[k], x);
      }
    }
#pragma unroll
    for (int k = 0; k < kNR; ++k) win[k][2 * kHalo] = vs[k];
  };

#pragma unroll
  for (int wi = 0; wi < kHalo; ++wi) push(wi);

  for (int wb = 0; wb < side; wb += kColBatch) {
    float4 outs[kColBatch][kNR];
#pragma unroll
    for (int q = 0; q < kColBatch; ++q) {
      const int wo = wb + q;
      push(wo + kHalo);
      // horizontal sums for output column wo (window index kHalo is column wo)
#pragma unroll
      for (int k = 0; k < kNR; ++k) {
        const int hr = radii.r[k] / 2;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int i = 0; i < 2 * kHalo + 1; ++i) {
          const int dx = i - kHalo;
          if ((dx < 0 ? -dx : dx) <= hr) acc = f4add(acc, win[k][i]);
        }
        // the sum of the r*r normalised values (zeros outside), divided by r*r
        outs[q][k] = f4scale(acc, 1.f / (float)(radii.r[k] * radii.r[k]));
      }
    }
    const int nb = side - wb < kColBatch ? side - wb : kColBatch;

    float norm[kColBatch][kNR];  // per-patch L2 norms when l2norm is set
    if (l2norm) {
#pragma unroll
      for (int q = 0; q < kColBatch; ++q)
#pragma unroll
        for (int k = 0; k < kNR; ++k) {
          const float v = wave_sum(act && q < nb ? f4dot(outs[q][k]) : 0.f);
          if (lane == 0) red[q * kNR + k][wave] = v;
        }
      __syncthreads();
#pragma unroll
      for (int q = 0; q < kColBatch; ++q)
#pragma unroll
        for (int k = 0; k < kNR; ++k) {
          float tot = 0.f;
          for (int w = 0; w < nwaves; ++w) tot += red[q * kNR + k][w];
          norm[q][k] = sqrtf(tot);
        }
      __syncthreads();
    }
    if (act) {
#pragma unroll
      for (int q = 0; q < kColBatch; ++q) {
        if (q < nb) {
          const int p = h * side + wb + q;
#pragma unroll
          for (int k = 0; k < kNR; ++k) {
            long long o;
            if (layout == MUSC_LAYOUT_RBPLC)
              o = ((((long long)k * batch + b) * P + p) * n_layers + l) * c;
            else
              o = ((((long long)k * n_layers + l) * batch + b) * P + p) * c;
            float4 v = outs[q][k];
            if (l2norm) {
              const float nrm = norm[q][k];
              v = make_float4(v.x / nrm, v.y / nrm, v.z / nrm, v.w / nrm);
            }
            reinterpret_cast<float4*>(out + o)[g] = v;
          }
        }
      }
    }
  }
}

inline size_t workspace_bytes(long long batch, long long n_layers) {
  const long long units = batch * n_layers;
  return align_up((size_t)units * kChunks * 2 * sizeof(double), 256) + align_up((size_t)units * 2 * sizeof(double), 256);
}

template <int kDtype, int kHalo, int kNR>
void launch_pool(dim3 grid, dim3 block, hipStream_t s, const TokenPtrs& tp, int n_layers, int batch, int tpi, int c,
                 int has_cls, int side, const Radii& radii, int l2norm, int layout, const double* stats, float* out,
                 long long work) {
  hipLaunchKernelGGL((lnamd_pool_kernel<kDtype, kHalo, kNR>), grid, block, 0, s, tp, n_layers, batch, tpi, c, has_cls,
                     side, radii, l2norm, layout, stats, out, work);
}

template <int kDtype, int kHalo>
int dispatch_nr(int nr, dim3 grid, dim3 block, hipStream_t s, const TokenPtrs& tp, int n_layers, int batch, int tpi,
                int c, int has_cls, int side, const Radii& radii, int l2norm, int layout, const double* stats,
                float* out, long long work) {
  switch (nr) {
    case 1: launch_pool<kDtype, kHalo, 1>(grid, block, s, tp, n_layers, batch, tpi, c, has_cls, side, radii, l2norm, layout, stats, out, work); break;
    case 2: launch_pool<kDtype, kHalo, 2>(grid, block, s, tp, n_layers, batch, tpi, c, has_cls, side, radii, l2norm, layout, stats, out, work); break;
    case 3: launch_pool<kDtype, kHalo, 3>(grid, block, s, tp, n_layers, batch, tpi, c, has_cls, side, radii, l2norm, layout, stats, out, work); break;
    case 4: launch_pool<kDtype, kHalo, 4>(grid, block, s, tp, n_layers, batch, tpi, c, has_cls, side, radii, l2norm, layout, stats, out, work); break;
    default: return MUSC_ERR_UNSUPPORTED;
  }
  return MUSC_OK;
}

template <int kDtype>
int dispatch_halo(int halo, int nr, dim3 grid, dim3 block, hipStream_t s, const TokenPtrs& tp, int n_layers,
                  int batch, int tpi, int c, int has_cls, int side, const Radii& radii, int l2norm, int layout,
                  const double* stats, float* out, long long work) {
  switch (halo) {
    case 0: return dispatch_nr<kDtype, 0>(nr, grid, block, s, tp, n_layers, batch, tpi, c, has_cls, side, radii, l2norm, layout, stats, out, work);
    case 1: return dispatch_nr<kDtype, 1>(nr, grid, block, s, tp, n_layers, batch, tpi, c, has_cls, side, radii, l2norm, layout, stats, out, work);
    case 2: return dispatch_nr<kDtype, 2>(nr, grid, block, s, tp, n_layers, batch, tpi, c, has_cls, side, radii, l2norm, layout, stats, out, work);
    case 3: return dispatch_nr<kDtype, 3>(nr, grid, block, s, tp, n_layers, batch, tpi, c, has_cls, side, radii, l2norm, layout, stats, out, work);
    case 4: return dispatch_nr<kDtype, 4>(nr, grid, block, s, tp, n_layers, batch, tpi, c, has_cls, side, radii, l2norm, layout, stats, out, work);
    default: return MUSC_ERR_UNSUPPORTED;
  }
}

}  // namespace lnamd
}  // namespace musc

using namespace musc;

extern "C" int musc_lnamd_workspace_bytes(int batch, int n_layers, size_t* out) {
  if (!out || batch < 1 || n_layers < 1) return MUSC_ERR_INVALID_ARG;
  *out = lnamd::workspace_bytes(batch, n_layers);
  return MUSC_OK;
}

extern "C" int musc_lnamd_f32(const void* const* tokens, int n_layers, int in_dtype, int batch,
                              int tokens_per_image, int c, int has_cls, const int* radii, int n_radii, float eps,
                              int flags, float* out, int out_layout, void* workspace, size_t workspace_bytes,
                              hipStream_t stream) {
  using namespace lnamd;
  if (!tokens || !radii || !out || n_layers < 1 || batch < 1 || c < 4 || n_radii < 1) return MUSC_ERR_INVALID_ARG;
  if (has_cls != 0 && has_cls != 1) return MUSC_ERR_INVALID_ARG;
  if (in_dtype != MUSC_DTYPE_F32 && in_dtype != MUSC_DTYPE_F16) return MUSC_ERR_INVALID_ARG;
  if (out_layout != MUSC_LAYOUT_RBPLC && out_layout != MUSC_LAYOUT_RLBPC) return MUSC_ERR_INVALID_ARG;
  if ((flags & ~(MUSC_LNAMD_L2NORM | MUSC_LNAMD_STATS_READY)) != 0) return MUSC_ERR_INVALID_ARG;
  if (n_layers > kMaxLayers || n_radii > kMaxRadii) return MUSC_ERR_UNSUPPORTED;
  if (c % 4 != 0 || c / 4 > 1024) return MUSC_ERR_UNSUPPORTED;
  const int grid_tokens = tokens_per_image - has_cls;
  int side = 0;
  while ((side + 1) * (side + 1) <= grid_tokens) ++side;
  if (grid_tokens < 1 || side * side != grid_tokens) return MUSC_ERR_INVALID_ARG;
  Radii rr{};
  rr.n = n_radii;
  int halo = 0;
  for (int k = 0; k < n_radii; ++k) {
    const int r = radii[k];
    if (r < 1 || (r & 1) == 0) return MUSC_ERR_INVALID_ARG;
    if (r / 2 > kMaxHalo) return MUSC_ERR_UNSUPPORTED;
    rr.r[k] = r;
    if (r / 2 > halo) halo = r / 2;
  }
  TokenPtrs tp{};
  const size_t align = in_dtype == MUSC_DTYPE_F32 ? 16 : 8;
  for (int l = 0; l < n_layers; ++l) {
    if (!tokens[l] || (reinterpret_cast<uintptr_t>(tokens[l]) % align) != 0) return MUSC_ERR_INVALID_ARG;
    tp.p[l] = tokens[l];
  }
  if ((reinterpret_cast<uintptr_t>(out) & 15) != 0) return MUSC_ERR_INVALID_ARG;
  if (!workspace || workspace_bytes < lnamd::workspace_bytes(batch, n_layers)) return MUSC_ERR_WORKSPACE;

  const int units = batch * n_layers;
  double* partials = static_cast<double*>(workspace);
  double* stats = reinterpret_cast<double*>(static_cast<char*>(workspace) +
                                            align_up((size_t)units * kChunks * 2 * sizeof(double), 256));
  if (flags & MUSC_LNAMD_STATS_READY) {
    // the workspace already holds {mean, rstd} of these tokens from an earlier call
  } else if (in_dtype == MUSC_DTYPE_F32) {
    hipLaunchKernelGGL(lnamd_stats_kernel<MUSC_DTYPE_F32>, dim3(units * kChunks), dim3(256), 0, stream, tp, n_layers,
                       batch, tokens_per_image, c, has_cls, partials);
    hipLaunchKernelGGL(lnamd_finalize_kernel<MUSC_DTYPE_F32>, dim3((units + 255) / 256), dim3(256), 0, stream, tp,
                       n_layers, units, tokens_per_image, c, has_cls, eps, partials, stats);
  } else {
    hipLaunchKernelGGL(lnamd_stats_kernel<MUSC_DTYPE_F16>, dim3(units * kChunks), dim3(256), 0, stream, tp, n_layers,
                       batch, tokens_per_image, c, has_cls, partials);
    hipLaunchKernelGGL(lnamd_finalize_kernel<MUSC_DTYPE_F16>, dim3((units + 255) / 256), dim3(256), 0, stream, tp,
                       n_layers, units, tokens_per_image, c, has_cls, eps, partials, stats);
  }
  const long long work = (long long)units * side;
  const long long grid = (work + kXcds - 1) / kXcds * kXcds;
  const int threads = ((c / 4 + kWave - 1) / kWave) * kWave;
  const int l2 = (flags & MUSC_LNAMD_L2NORM) ? 1 : 0;
  int rc;
  if (in_dtype == MUSC_DTYPE_F32)
    rc = dispatch_halo<MUSC_DTYPE_F32>(halo, n_radii, dim3((unsigned)grid), dim3(threads), stream, tp, n_layers, batch,
                                       tokens_per_image, c, has_cls, side, rr, l2, out_layout, stats, out, work);
  else
    rc = dispatch_halo<MUSC_DTYPE_F16>(halo, n_radii, dim3((unsigned)grid), dim3(threads), stream, tp, n_layers, batch,
                                       tokens_per_image, c, has_cls, side, rr, l2, out_layout, stats, out, work);
  if (rc) return rc;
  return check_launch();
}
