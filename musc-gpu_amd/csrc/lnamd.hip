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
//   lnamd_stream_kernel    default path.  One workgroup per (image, layer, slice of
//                          4*cg channels); thread (column, 4 channels) sweeps the
//                          rows top to bottom with the last 2*hmax+1 rows of its
//                          column in a register ring, puts the nested vertical sums
//                          of each output row in LDS (double-buffered, one barrier
//                          per row) and adds its horizontal neighbours'.  Every
//                          token is read once, every output written once.
//   lnamd_pool_kernel      L2-normalising path.  One workgroup per (image, layer, output row); each
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

// Same as load4 with the nontemporal hint, for tokens a kernel reads exactly once
// (statistics pass, streaming pass): +20 % on the statistics pass, measured.
typedef float nt_load_f4 __attribute__((ext_vector_type(4)));
typedef unsigned int nt_load_u2 __attribute__((ext_vector_type(2)));
template <int kDtype>
__device__ inline float4 load4_once(const void* base, long long idx4) {
  if (kDtype == MUSC_DTYPE_F32) {
    const nt_load_f4 v = __builtin_nontemporal_load(reinterpret_cast<const nt_load_f4*>(base) + idx4);
    return make_float4(v.x, v.y, v.z, v.w);
  } else {
    const nt_load_u2 raw = __builtin_nontemporal_load(reinterpret_cast<const nt_load_u2*>(base) + idx4);
    const unsigned int rx = raw.x, ry = raw.y;
    const float2 a = __half22float2(*reinterpret_cast<const __half2*>(&rx));
    const float2 b = __half22float2(*reinterpret_cast<const __half2*>(&ry));
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
    const float4 v = load4_once<kDtype>(base, first / 4 + i);
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

typedef float nt_float4 __attribute__((ext_vector_type(4)));

__device__ inline float4 f4add(float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); }
__device__ inline float4 f4scale(float4 a, float s) { return make_float4(a.x * s, a.y * s, a.z * s, a.w * s); }
__device__ inline float f4dot(float4 a) { return a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w; }

// Sum of `v` over the 64 lanes of a wave, result in every lane: DPP within rows of
// 16 lanes, then two cross-row exchanges.
__device__ inline float wave_allsum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xb1, 0xf, 0xf, false));  // quad_perm 1,0,3,2
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4e, 0xf, 0xf, false));  // quad_perm 2,3,0,1
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xf, 0xf, false)); // row_half_mirror
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xf, 0xf, false)); // row_mirror
  v += __shfl_xor(v, 16, kWave);
  v += __shfl_xor(v, 32, kWave);
  return v;
}

// grid: xcd-padded units * side; block = c/4 threads rounded up to a wave multiple.
// Radii arrive sorted ascending (the host keeps the caller's order in `slot`), so
// the vertical sums nest: V_k = V_{k-1} + the rows between radius k-1 and k.
template <int kDtype, int kHalo, int kNR, int kMaxThreads>
__global__ __launch_bounds__(kMaxThreads) void lnamd_pool_kernel(TokenPtrs tokens, int n_layers, int batch,
                                                                 int tokens_per_image, int c, int has_cls, int side,
                                                                 Radii radii, Radii slot, int l2norm, int layout,
                                                                 const double* __restrict__ stats,
                                                                 float* __restrict__ out, long long work) {
  const long long wid = xcd_logical_id(blockIdx.x, gridDim.x);
  if (wid >= work) return;
  const int unit = (int)(wid / side), h = (int)(wid % side);
  const int b = unit / n_layers, l = unit % n_layers;
  const int g = threadIdx.x;  // channel group (4 channels)
  const int groups = c / 4;
  const bool act = g < groups;
  const int gl = act ? g : 0;  // inactive lanes read a valid address and discard it
  const void* base = tokens.p[l];
  const float mean = (float)stats[unit * 2 + 0];
  const float rstd = (float)stats[unit * 2 + 1];
  const int P = side * side;
  const long long img_base4 = (((long long)b * tokens_per_image + has_cls) * c) / 4;

  __shared__ float red[kNR * kColBatch][16];
  const int nwaves = (blockDim.x + kWave - 1) / kWave;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;

  // win[k][i]: vertical sum for radius k of column (current - kHalo + i), of x - mean
  float4 win[kNR][2 * kHalo + 1];
#pragma unroll
  for (int k = 0; k < kNR; ++k)
#pragma unroll
    for (int i = 0; i < 2 * kHalo + 1; ++i) win[k][i] = make_float4(0.f, 0.f, 0.f, 0.f);

  // Loads of input column wi, rows h-kHalo..h+kHalo; row and column validity are
  // uniform over the workgroup, so out-of-image rows are skipped, not masked.
  auto load_col = [&](int wi, float4 (&x)[2 * kHalo + 1]) {
#pragma unroll
    for (int dy = -kHalo; dy <= kHalo; ++dy) {
      const int hh = h + dy;
      if (wi < side && hh >= 0 && hh < side) {
        const float4 r = load4<kDtype>(base, img_base4 + ((long long)(hh * side + wi) * c) / 4 + gl);
        x[dy + kHalo] = make_float4(r.x - mean, r.y - mean, r.z - mean, r.w - mean);
      } else {
        x[dy + kHalo] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  };
  auto push = [&](const float4 (&x)[2 * kHalo + 1]) {
#pragma unroll
    for (int k = 0; k < kNR; ++k)
#pragma unroll
      for (int i = 0; i < 2 * kHalo; ++i) win[k][i] = win[k][i + 1];
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    int done = -1;  // rows |dy| <= done are in v
#pragma unroll
    for (int k = 0; k < kNR; ++k) {
      const int hr = radii.r[k] / 2;
#pragma unroll
      for (int a = 0; a <= kHalo; ++a) {
        if (a > done && a <= hr) {
          v = f4add(v, x[kHalo + a]);
          if (a > 0) v = f4add(v, x[kHalo - a]);
        }
      }
      done = hr > done ? hr : done;
      win[k][2 * kHalo] = v;
    }
  };

  {
    float4 pre[kHalo > 0 ? kHalo : 1][2 * kHalo + 1];
#pragma unroll
    for (int wi = 0; wi < kHalo; ++wi) load_col(wi, pre[wi]);
#pragma unroll
    for (int wi = 0; wi < kHalo; ++wi) push(pre[wi]);
  }

  for (int wb = 0; wb < side; wb += kColBatch) {
    float4 xin[kColBatch][2 * kHalo + 1];
#pragma unroll
    for (int q = 0; q < kColBatch; ++q) load_col(wb + q + kHalo, xin[q]);
    float4 outs[kColBatch][kNR];
#pragma unroll
    for (int q = 0; q < kColBatch; ++q) {
      push(xin[q]);
      // horizontal sums for output column wb + q (window index kHalo)
#pragma unroll
      for (int k = 0; k < kNR; ++k) {
        const int hr = radii.r[k] / 2;
        float4 acc = win[k][kHalo];
#pragma unroll
        for (int a = 1; a <= kHalo; ++a)
          if (a <= hr) acc = f4add(f4add(acc, win[k][kHalo - a]), win[k][kHalo + a]);
        outs[q][k] = acc;
      }
    }
    const int nb = side - wb < kColBatch ? side - wb : kColBatch;

    float scale[kColBatch][kNR];
    if (l2norm) {
      // the LayerNorm scale and the 1/r^2 of the box mean cancel in the L2
      // normalisation: out = S / ||S|| with S the window sum of x - mean
#pragma unroll
      for (int q = 0; q < kColBatch; ++q)
#pragma unroll
        for (int k = 0; k < kNR; ++k) {
          const float v = wave_allsum(act && q < nb ? f4dot(outs[q][k]) : 0.f);
          if (lane == 0) red[q * kNR + k][wave] = v;
        }
      __syncthreads();
#pragma unroll
      for (int q = 0; q < kColBatch; ++q)
#pragma unroll
        for (int k = 0; k < kNR; ++k) {
          float tot = 0.f;
          for (int w = 0; w < nwaves; ++w) tot += red[q * kNR + k][w];
          scale[q][k] = 1.f / sqrtf(tot);
        }
      __syncthreads();
    } else {
#pragma unroll
      for (int q = 0; q < kColBatch; ++q)
#pragma unroll
        for (int k = 0; k < kNR; ++k) scale[q][k] = rstd / (float)(radii.r[k] * radii.r[k]);
    }
    if (act) {
#pragma unroll
      for (int q = 0; q < kColBatch; ++q) {
        if (q < nb) {
          const int p = h * side + wb + q;
#pragma unroll
          for (int k = 0; k < kNR; ++k) {
            const int ko = slot.r[k];
            long long o;
            if (layout == MUSC_LAYOUT_RBPLC)
              o = ((((long long)ko * batch + b) * P + p) * n_layers + l) * c;
            else
              o = ((((long long)ko * n_layers + l) * batch + b) * P + p) * c;
            reinterpret_cast<float4*>(out + o)[g] = f4scale(outs[q][k], scale[q][k]);
          }
        }
      }
    }
  }
}

// Streaming variant (no cross-channel reduction).  One workgroup per (image,
// layer, slice of cg channel groups); thread (w, gl) owns column w and channels
// 4*(slice*cg + gl) .. +3 and sweeps the rows top to bottom.  The last 2*kHalo+1
// input rows of its column (x - mean) live in a register ring; the vertical sums
// of each output row go to LDS (double-buffered by row parity, one barrier per
// row) and each thread adds its horizontal neighbours' sums from there.  Every
// input value is read from HBM once and every output written once.  Workgroups
// are XCD-grouped (the slices of one image and layer share an XCD).
//   raw = 0: out = window sum * rstd / r^2   (avg_pool2d of the LayerNorm output)
//   raw = 1: out = window sum of (x - mean)  (unscaled; for consumers that
//            L2-normalise, where the scale cancels)
// kPool: the side x side grid of window sums is adaptively average-pooled to
// pool x pool (F.adaptive_avg_pool2d windows: rows floor(i*side/pool) ..
// ceil((i+1)*side/pool) - 1, likewise columns; the super_fast 37 -> 28 step,
// models/modules/_super_fast.py:17-27) before it is written.  Each finished row of
// window sums goes to LDS, output-column threads sum their columns, and the row
// sums accumulate in two register slots (a source row lies in at most two output
// windows when pool <= side); an output row is written when its last source row
// is done.  raw = 0 divides by r^2 and the window count, raw = 1 writes the plain
// sums.
template <int kDtype, int kHalo, int kNR, bool kPool>
__global__ __launch_bounds__(1024) void lnamd_stream_kernel(TokenPtrs tokens, int n_layers, int batch,
                                                            int tokens_per_image, int c, int has_cls, int side,
                                                            int cg, int slices, Radii radii, Radii slot, int raw,
                                                            int layout, int pool, const double* __restrict__ stats,
                                                            float* __restrict__ out) {
  extern __shared__ float4 vsum[];  // [2][kNR][side * cg], then (kPool) hsum [kNR][side * cg]
  // XCD-grouped order: the slices of one (image, layer) run on one XCD (-3 % time
  // at config 2, measured).  The grid is padded to a multiple of kXcds.
  const long long wid = xcd_logical_id(blockIdx.x, gridDim.x);
  if (wid >= (long long)batch * n_layers * slices) return;
  const int unit = (int)(wid / slices), slice = (int)(wid % slices);
  const int b = unit / n_layers, l = unit % n_layers;
  const int w = threadIdx.x / cg, gl = threadIdx.x % cg;
  const int groups = c / 4;
  const int g = slice * cg + gl;
  const bool act = w < side && g < groups;
  const int wl = act ? w : 0, gg = act ? g : 0;  // inactive threads read a valid address
  const void* base = tokens.p[l];
  const float mean = (float)stats[unit * 2 + 0];
  const float rstd = (float)stats[unit * 2 + 1];
  const int P = kPool ? pool * pool : side * side;
  const int row_len = side * cg;
  float4* hsum = vsum + (size_t)2 * kNR * row_len;
  // pooled-row accumulators of even and odd output rows (named, not indexed by a
  // runtime slot, so they stay in registers)
  float4 pacc_even[kNR], pacc_odd[kNR];
#pragma unroll
  for (int k = 0; k < kNR; ++k) pacc_even[k] = pacc_odd[k] = make_float4(0.f, 0.f, 0.f, 0.f);
  const long long col_base4 = (((long long)b * tokens_per_image + has_cls) * c) / 4 + (long long)wl * (c / 4) + gg;
  const long long row_step4 = (long long)side * (c / 4);

  float4 ring[2 * kHalo + 1];
#pragma unroll
  for (int i = 0; i < 2 * kHalo + 1; ++i) ring[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  float4 next = load4_once<kDtype>(base, col_base4);

  for (int hi = 0; hi < side + kHalo; ++hi) {
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (hi < side) {
      x = make_float4(next.x - mean, next.y - mean, next.z - mean, next.w - mean);
      if (hi + 1 < side) next = load4_once<kDtype>(base, col_base4 + (long long)(hi + 1) * row_step4);
    }
#pragma unroll
    for (int i = 0; i < 2 * kHalo; ++i) ring[i] = ring[i + 1];
    ring[2 * kHalo] = x;
    const int h = hi - kHalo;
    if (h < 0) continue;
    // nested vertical sums of row h (ring index kHalo) for the ascending radii
    float4* buf = vsum + (size_t)(h & 1) * kNR * row_len;
    {
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      int done = -1;
#pragma unroll
      for (int k = 0; k < kNR; ++k) {
        const int hr = radii.r[k] / 2;
#pragma unroll
        for (int a = 0; a <= kHalo; ++a) {
          if (a > done && a <= hr) {
            v = f4add(v, ring[kHalo + a]);
            if (a > 0) v = f4add(v, ring[kHalo - a]);
          }
        }
        done = hr > done ? hr : done;
        buf[k * row_len + threadIdx.x] = v;
      }
    }
    __syncthreads();
    if (act) {
      const int p = h * side + w;
#pragma unroll
      for (int k = 0; k < kNR; ++k) {
        const int hr = radii.r[k] / 2;
        float4 acc = buf[k * row_len + threadIdx.x];
#pragma unroll
        for (int a = 1; a <= kHalo; ++a) {
          if (a <= hr) {
            if (w - a >= 0) acc = f4add(acc, buf[k * row_len + threadIdx.x - a * cg]);
            if (w + a < side) acc = f4add(acc, buf[k * row_len + threadIdx.x + a * cg]);
          }
        }
        if constexpr (kPool) {
          hsum[k * row_len + threadIdx.x] = acc;
        } else {
          const float sc = raw ? 1.f : rstd / (float)(radii.r[k] * radii.r[k]);
          const int ko = slot.r[k];
          long long o;
          if (layout == MUSC_LAYOUT_RBPLC)
            o = ((((long long)ko * batch + b) * P + p) * n_layers + l) * c;
          else
            o = ((((long long)ko * n_layers + l) * batch + b) * P + p) * c;
          // streaming store: the pools are read back only by later kernels
          const float4 r = f4scale(acc, sc);
          const nt_float4 v = {r.x, r.y, r.z, r.w};
          __builtin_nontemporal_store(v, reinterpret_cast<nt_float4*>(out + o) + g);
        }
      }
    }
    if constexpr (kPool) {
      __syncthreads();
      // thread (w, gl) is output column w for the pooling step
      if (w < pool && g < groups) {
        const int x0 = (w * side) / pool, x1 = ((w + 1) * side + pool - 1) / pool;
        float4 hp[kNR];
#pragma unroll
        for (int k = 0; k < kNR; ++k) {
          float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
          for (int x = x0; x < x1; ++x) a = f4add(a, hsum[k * row_len + x * cg + gl]);
          hp[k] = a;
        }
        const int oy0 = (h * pool) / side;  // first output row whose window holds row h
#pragma unroll
        for (int d = 0; d < 2; ++d) {
          const int oy = oy0 + d;
          if (oy >= pool) continue;
          const int y0 = (oy * side) / pool, y1 = ((oy + 1) * side + pool - 1) / pool;
          if (h < y0 || h >= y1) continue;
          auto add_emit = [&](float4 (&pa)[kNR]) {
#pragma unroll
            for (int k = 0; k < kNR; ++k) pa[k] = f4add(pa[k], hp[k]);
            if (h != y1 - 1) return;
            const int po = oy * pool + w;
            const float cnt = (float)((y1 - y0) * (x1 - x0));
#pragma unroll
            for (int k = 0; k < kNR; ++k) {
              const float sc = raw ? 1.f : rstd / ((float)(radii.r[k] * radii.r[k]) * cnt);
              const int ko = slot.r[k];
              long long o;
              if (layout == MUSC_LAYOUT_RBPLC)
                o = ((((long long)ko * batch + b) * P + po) * n_layers + l) * c;
              else
                o = ((((long long)ko * n_layers + l) * batch + b) * P + po) * c;
              const float4 r = f4scale(pa[k], sc);
              const nt_float4 v = {r.x, r.y, r.z, r.w};
              __builtin_nontemporal_store(v, reinterpret_cast<nt_float4*>(out + o) + g);
              pa[k] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
          };
          if (oy & 1) add_emit(pacc_odd); else add_emit(pacc_even);
        }
      }
    }
  }
}

template <int kDtype, int kHalo, bool kPool>
int dispatch_stream_nr(int nr, dim3 grid, dim3 block, size_t smem, hipStream_t s, const TokenPtrs& tp, int n_layers,
                       int batch, int tpi, int c, int has_cls, int side, int cg, int slices, const Radii& radii,
                       const Radii& slot, int raw, int layout, int pool, const double* stats, float* out) {
#define MUSC_STREAM_CASE(NR)                                                                                      \
  case NR:                                                                                                        \
    hipLaunchKernelGGL((lnamd_stream_kernel<kDtype, kHalo, NR, kPool>), grid, block, smem, s, tp, n_layers, batch, \
                       tpi, c, has_cls, side, cg, slices, radii, slot, raw, layout, pool, stats, out);            \
    break;
  switch (nr) {
    MUSC_STREAM_CASE(1)
    MUSC_STREAM_CASE(2)
    MUSC_STREAM_CASE(3)
    MUSC_STREAM_CASE(4)
    default: return MUSC_ERR_UNSUPPORTED;
  }
#undef MUSC_STREAM_CASE
  return MUSC_OK;
}

template <int kDtype, bool kPool>
int dispatch_stream(int halo, int nr, dim3 grid, dim3 block, size_t smem, hipStream_t s, const TokenPtrs& tp,
                    int n_layers, int batch, int tpi, int c, int has_cls, int side, int cg, int slices,
                    const Radii& radii, const Radii& slot, int raw, int layout, int pool, const double* stats,
                    float* out) {
#define MUSC_STREAM_HALO(H)                                                                                      \
  case H:                                                                                                        \
    return dispatch_stream_nr<kDtype, H, kPool>(nr, grid, block, smem, s, tp, n_layers, batch, tpi, c, has_cls,   \
                                                side, cg, slices, radii, slot, raw, layout, pool, stats, out);
  switch (halo) {
    MUSC_STREAM_HALO(0)
    MUSC_STREAM_HALO(1)
    MUSC_STREAM_HALO(2)
    MUSC_STREAM_HALO(3)
    MUSC_STREAM_HALO(4)
    default: return MUSC_ERR_UNSUPPORTED;
  }
#undef MUSC_STREAM_HALO
}

// Adaptive average pooling of a side_in x side_in patch grid to side_out x
// side_out (F.adaptive_avg_pool2d semantics: output cell i averages input rows
// floor(i*in/out) .. ceil((i+1)*in/out)-1, likewise for columns), over
// `batch` grids of shape (side_in^2, ch) -> (side_out^2, ch).  One thread per
// output float4; the window is at most 3 x 3 for 37 -> 28.
__global__ __launch_bounds__(256) void adaptive_pool_kernel(const float* __restrict__ in, int batch, int side_in,
                                                            int ch4, int side_out, float* __restrict__ out) {
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long per_img = (long long)side_out * side_out * ch4;
  if (idx >= per_img * batch) return;
  const int bimg = (int)(idx / per_img);
  const long long rem = idx % per_img;
  const int po = (int)(rem / ch4), g = (int)(rem % ch4);
  const int oy = po / side_out, ox = po % side_out;
  const int y0 = (oy * side_in) / side_out, y1 = ((oy + 1) * side_in + side_out - 1) / side_out;
  const int x0 = (ox * side_in) / side_out, x1 = ((ox + 1) * side_in + side_out - 1) / side_out;
  const float4* src = reinterpret_cast<const float4*>(in) + (long long)bimg * side_in * side_in * ch4 + g;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int y = y0; y < y1; ++y)
    for (int x = x0; x < x1; ++x) acc = f4add(acc, src[(long long)(y * side_in + x) * ch4]);
  const float cnt = (float)((y1 - y0) * (x1 - x0));
  reinterpret_cast<float4*>(out)[idx] = make_float4(acc.x / cnt, acc.y / cnt, acc.z / cnt, acc.w / cnt);
}

inline size_t workspace_bytes(long long batch, long long n_layers) {
  const long long units = batch * n_layers;
  return align_up((size_t)units * kChunks * 2 * sizeof(double), 256) + align_up((size_t)units * 2 * sizeof(double), 256);
}

template <int kDtype, int kHalo, int kNR>
void launch_pool(dim3 grid, dim3 block, hipStream_t s, const TokenPtrs& tp, int n_layers, int batch, int tpi, int c,
                 int has_cls, int side, const Radii& radii, const Radii& slot, int l2norm, int layout,
                 const double* stats, float* out, long long work) {
  // up to 256 threads (C <= 1024): the register budget of 2 waves per SIMD holds the
  // whole column window; wider C uses 1024-thread workgroups
  if (block.x <= 256)
    hipLaunchKernelGGL((lnamd_pool_kernel<kDtype, kHalo, kNR, 256>), grid, block, 0, s, tp, n_layers, batch, tpi, c,
                       has_cls, side, radii, slot, l2norm, layout, stats, out, work);
  else
    hipLaunchKernelGGL((lnamd_pool_kernel<kDtype, kHalo, kNR, 1024>), grid, block, 0, s, tp, n_layers, batch, tpi, c,
                       has_cls, side, radii, slot, l2norm, layout, stats, out, work);
}

template <int kDtype, int kHalo>
int dispatch_nr(int nr, dim3 grid, dim3 block, hipStream_t s, const TokenPtrs& tp, int n_layers, int batch, int tpi,
                int c, int has_cls, int side, const Radii& radii, const Radii& slot, int l2norm, int layout,
                const double* stats, float* out, long long work) {
  switch (nr) {
    case 1: launch_pool<kDtype, kHalo, 1>(grid, block, s, tp, n_layers, batch, tpi, c, has_cls, side, radii, slot, l2norm, layout, stats, out, work); break;
    case 2: launch_pool<kDtype, kHalo, 2>(grid, block, s, tp, n_layers, batch, tpi, c, has_cls, side, radii, slot, l2norm, layout, stats, out, work); break;
    case 3: launch_pool<kDtype, kHalo, 3>(grid, block, s, tp, n_layers, batch, tpi, c, has_cls, side, radii, slot, l2norm, layout, stats, out, work); break;
    case 4: launch_pool<kDtype, kHalo, 4>(grid, block, s, tp, n_layers, batch, tpi, c, has_cls, side, radii, slot, l2norm, layout, stats, out, work); break;
    default: return MUSC_ERR_UNSUPPORTED;
  }
  return MUSC_OK;
}

template <int kDtype>
int dispatch_halo(int halo, int nr, dim3 grid, dim3 block, hipStream_t s, const TokenPtrs& tp, int n_layers,
                  int batch, int tpi, int c, int has_cls, int side, const Radii& radii, const Radii& slot, int l2norm,
                  int layout, const double* stats, float* out, long long work) {
  switch (halo) {
    case 0: return dispatch_nr<kDtype, 0>(nr, grid, block, s, tp, n_layers, batch, tpi, c, has_cls, side, radii, slot, l2norm, layout, stats, out, work);
    case 1: return dispatch_nr<kDtype, 1>(nr, grid, block, s, tp, n_layers, batch, tpi, c, has_cls, side, radii, slot, l2norm, layout, stats, out, work);
    case 2: return dispatch_nr<kDtype, 2>(nr, grid, block, s, tp, n_layers, batch, tpi, c, has_cls, side, radii, slot, l2norm, layout, stats, out, work);
    case 3: return dispatch_nr<kDtype, 3>(nr, grid, block, s, tp, n_layers, batch, tpi, c, has_cls, side, radii, slot, l2norm, layout, stats, out, work);
    case 4: return dispatch_nr<kDtype, 4>(nr, grid, block, s, tp, n_layers, batch, tpi, c, has_cls, side, radii, slot, l2norm, layout, stats, out, work);
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

namespace {

// pool_side == 0: no pooling (output grid = input grid).
int lnamd_run(const void* const* tokens, int n_layers, int in_dtype, int batch, int tokens_per_image, int c,
              int has_cls, const int* radii, int n_radii, float eps, int flags, int pool_side, float* out,
              int out_layout, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  using namespace lnamd;
  if (!tokens || !radii || !out || n_layers < 1 || batch < 1 || c < 4 || n_radii < 1) return MUSC_ERR_INVALID_ARG;
  if (has_cls != 0 && has_cls != 1) return MUSC_ERR_INVALID_ARG;
  if (in_dtype != MUSC_DTYPE_F32 && in_dtype != MUSC_DTYPE_F16) return MUSC_ERR_INVALID_ARG;
  if (out_layout != MUSC_LAYOUT_RBPLC && out_layout != MUSC_LAYOUT_RLBPC) return MUSC_ERR_INVALID_ARG;
  if ((flags & ~(MUSC_LNAMD_L2NORM | MUSC_LNAMD_STATS_READY | MUSC_LNAMD_RAW_SUMS)) != 0) return MUSC_ERR_INVALID_ARG;
  if ((flags & MUSC_LNAMD_L2NORM) && (flags & MUSC_LNAMD_RAW_SUMS)) return MUSC_ERR_INVALID_ARG;
  if (n_layers > kMaxLayers || n_radii > kMaxRadii) return MUSC_ERR_UNSUPPORTED;
  if (c % 4 != 0 || c / 4 > 1024) return MUSC_ERR_UNSUPPORTED;
  const int grid_tokens = tokens_per_image - has_cls;
  int side = 0;
  while ((long long)(side + 1) * (side + 1) <= grid_tokens) ++side;
  if (grid_tokens < 1 || (long long)side * side != grid_tokens) return MUSC_ERR_INVALID_ARG;
  if (pool_side < 0 || pool_side > side) return MUSC_ERR_INVALID_ARG;
  const bool pooled = pool_side > 0 && pool_side < side;
  if (pooled && (flags & MUSC_LNAMD_L2NORM)) return MUSC_ERR_UNSUPPORTED;
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
  // sort radii ascending for the nested vertical sums; slot[k] is the output index
  Radii slot{};
  slot.n = n_radii;
  for (int k = 0; k < n_radii; ++k) slot.r[k] = k;
  for (int i = 1; i < n_radii; ++i)
    for (int j = i; j > 0 && rr.r[j - 1] > rr.r[j]; --j) {
      int tr = rr.r[j - 1]; rr.r[j - 1] = rr.r[j]; rr.r[j] = tr;
      int ts = slot.r[j - 1]; slot.r[j - 1] = slot.r[j]; slot.r[j] = ts;
    }
  TokenPtrs tp{};
  const size_t align = in_dtype == MUSC_DTYPE_F32 ? 16 : 8;
  for (int l = 0; l < n_layers; ++l) {
    if (!tokens[l] || (reinterpret_cast<uintptr_t>(tokens[l]) % align) != 0) return MUSC_ERR_INVALID_ARG;
    tp.p[l] = tokens[l];
  }
  if ((reinterpret_cast<uintptr_t>(out) & 15) != 0) return MUSC_ERR_INVALID_ARG;
  if (!workspace || workspace_bytes < lnamd::workspace_bytes(batch, n_layers)) return MUSC_ERR_WORKSPACE;

  // every grid below (units x chunks, units x slices <= units x 1024) stays in int
  if ((long long)batch * n_layers * 1024 > 0x7fffffffLL) return MUSC_ERR_UNSUPPORTED;
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
  int rc;
  if (flags & MUSC_LNAMD_L2NORM) {
    // fused L2 normalisation: one workgroup owns all channels of an output row
    if (c / 4 > 1024) return MUSC_ERR_UNSUPPORTED;
    const long long work = (long long)units * side;
    const long long grid = (work + kXcds - 1) / kXcds * kXcds;
    const int threads = ((c / 4 + kWave - 1) / kWave) * kWave;
    if (in_dtype == MUSC_DTYPE_F32)
      rc = dispatch_halo<MUSC_DTYPE_F32>(halo, n_radii, dim3((unsigned)grid), dim3(threads), stream, tp, n_layers,
                                         batch, tokens_per_image, c, has_cls, side, rr, slot, 1, out_layout, stats,
                                         out, work);
    else
      rc = dispatch_halo<MUSC_DTYPE_F16>(halo, n_radii, dim3((unsigned)grid), dim3(threads), stream, tp, n_layers,
                                         batch, tokens_per_image, c, has_cls, side, rr, slot, 1, out_layout, stats,
                                         out, work);
  } else {
    // streaming kernel: cg channel groups per workgroup, side*cg <= 1024 threads
    const int groups = c / 4;
    // LDS: double-buffered vertical sums, plus (pooled) one row of window sums
    const size_t bufs = pooled ? 3 : 2;
    int cg = 1;
    while (cg * 2 <= 16 && cg * 2 <= groups && side * cg * 2 <= 1024 &&
           bufs * n_radii * side * cg * 2 * sizeof(float4) <= 64 * 1024)
      cg *= 2;
    const size_t smem = bufs * n_radii * side * cg * sizeof(float4);
    if (side * cg > 1024 || smem > 64 * 1024) return MUSC_ERR_UNSUPPORTED;
    const int slices = (groups + cg - 1) / cg;
    const int threads = side * cg;
    const int raw = (flags & MUSC_LNAMD_RAW_SUMS) ? 1 : 0;
    const dim3 grid((unsigned)((units * slices + kXcds - 1) / kXcds * kXcds));
    const int pool = pooled ? pool_side : side;
    if (in_dtype == MUSC_DTYPE_F32)
      rc = pooled ? dispatch_stream<MUSC_DTYPE_F32, true>(halo, n_radii, grid, dim3(threads), smem, stream, tp,
                                                         n_layers, batch, tokens_per_image, c, has_cls, side, cg,
                                                         slices, rr, slot, raw, out_layout, pool, stats, out)
                  : dispatch_stream<MUSC_DTYPE_F32, false>(halo, n_radii, grid, dim3(threads), smem, stream, tp,
                                                          n_layers, batch, tokens_per_image, c, has_cls, side, cg,
                                                          slices, rr, slot, raw, out_layout, pool, stats, out);
    else
      rc = pooled ? dispatch_stream<MUSC_DTYPE_F16, true>(halo, n_radii, grid, dim3(threads), smem, stream, tp,
                                                         n_layers, batch, tokens_per_image, c, has_cls, side, cg,
                                                         slices, rr, slot, raw, out_layout, pool, stats, out)
                  : dispatch_stream<MUSC_DTYPE_F16, false>(halo, n_radii, grid, dim3(threads), smem, stream, tp,
                                                          n_layers, batch, tokens_per_image, c, has_cls, side, cg,
                                                          slices, rr, slot, raw, out_layout, pool, stats, out);
  }
  if (rc) return rc;
  return check_launch();
}

}  // namespace

extern "C" int musc_lnamd_f32(const void* const* tokens, int n_layers, int in_dtype, int batch,
                              int tokens_per_image, int c, int has_cls, const int* radii, int n_radii, float eps,
                              int flags, float* out, int out_layout, void* workspace, size_t workspace_bytes,
                              hipStream_t stream) {
  return lnamd_run(tokens, n_layers, in_dtype, batch, tokens_per_image, c, has_cls, radii, n_radii, eps, flags, 0,
                   out, out_layout, workspace, workspace_bytes, stream);
}

extern "C" int musc_lnamd_pooled_f32(const void* const* tokens, int n_layers, int in_dtype, int batch,
                                     int tokens_per_image, int c, int has_cls, const int* radii, int n_radii,
                                     float eps, int flags, int pool_side, float* out, int out_layout,
                                     void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (pool_side < 1) return MUSC_ERR_INVALID_ARG;
  return lnamd_run(tokens, n_layers, in_dtype, batch, tokens_per_image, c, has_cls, radii, n_radii, eps, flags,
                   pool_side, out, out_layout, workspace, workspace_bytes, stream);
}

extern "C" int musc_adaptive_pool_f32(const float* in, int batch, int side_in, int ch, int side_out, float* out,
                                      hipStream_t stream) {
  if (!in || !out || batch < 1 || side_in < 1 || side_out < 1 || ch < 4) return MUSC_ERR_INVALID_ARG;
  if (ch % 4 != 0) return MUSC_ERR_UNSUPPORTED;
  if (((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15) != 0) return MUSC_ERR_INVALID_ARG;
  const long long total = (long long)batch * side_out * side_out * (ch / 4);
  if (total == 0) return MUSC_OK;
  if ((total + 255) / 256 > 0x7fffffffLL) return MUSC_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(lnamd::adaptive_pool_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, in,
                     batch, side_in, ch / 4, side_out, out);
  return check_launch();
}
