// RsCIN image-score refinement for gfx950.
//
// Reference (models/modules/_RsCIN.py:5-32): scores are min-max normalised, the
// class-token similarity W = X X^T is formed, and for every k in k_list each row
// keeps only its k largest similarities (torch.topk zeroes the N-k smallest,
// :8-11); the refined score of image i is sum_j W_ij s_j / sum_j W_ij over the
// kept entries (the row-normalised D^-1 W times s, :12-18), averaged over k_list
// (:20).  One workgroup per image i: similarities of row i into LDS, each kept
// set found by rank counting (ties broken by column index), sums in fp64.  The
// similarities are accumulated in fp64, so the kept set is the one exact arithmetic
// selects: where two similarities lie closer together than fp32 rounding can
// resolve, the reference's own fp32 product keeps one or the other depending on its
// summation order, and no fp32 ordering could reproduce that choice in general.  The
// min-max normalisation propagates NaN like numpy's min/max (:27): one NaN raw
// score makes every refined score NaN, as in the reference.
#include "common.hpp"

namespace musc {
namespace rscin {

constexpr int kThreads = 256;
constexpr int kMaxN = 4096;
constexpr int kMaxK = 16;

__device__ inline double nmin(double a, double b) { return __builtin_elementwise_minimum(a, b); }
__device__ inline double nmax(double a, double b) { return __builtin_elementwise_maximum(a, b); }

struct KList {
  int k[kMaxK];
  int n;
};

__global__ __launch_bounds__(kThreads) void rscin_kernel(const float* __restrict__ x, const double* __restrict__ raw,
                                                         int n, int d, KList ks, float* __restrict__ out) {
  extern __shared__ double w[];  // n similarities of row i
  __shared__ double red[2][kThreads / kWave];
  __shared__ double s_min, s_max;
  const int i = blockIdx.x, tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid % kWave;
  // min / max of the raw scores
  double mn = INFINITY, mx = -INFINITY;
  for (int j = tid; j < n; j += kThreads) {
    mn = nmin(mn, raw[j]);
    mx = nmax(mx, raw[j]);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    mn = nmin(mn, __shfl_xor(mn, off, kWave));
    mx = nmax(mx, __shfl_xor(mx, off, kWave));
  }
  if (lane == 0) {
    red[0][wave] = mn;
    red[1][wave] = mx;
  }
  __syncthreads();
  if (tid == 0) {
    double a = red[0][0], b = red[1][0];
    for (int q = 1; q < kThreads / kWave; ++q) {
      a = nmin(a, red[0][q]);
      b = nmax(b, red[1][q]);
    }
    s_min = a;
    s_max = b;
  }
  // similarities W[i][j] = x_i . x_j (fp64 accumulation of the fp32 tokens)
  const float* xi = x + (long long)i * d;
  for (int j = wave; j < n; j += kThreads / kWave) {
    const float* xj = x + (long long)j * d;
    double acc = 0.0;
    for (int c = lane; c < d; c += kWave) acc = fma((double)xi[c], (double)xj[c], acc);
    acc = wave_sum(acc);
    if (lane == 0) w[j] = acc;
  }
  __syncthreads();
  const double lo = s_min, span = s_max - s_min;
  double total = 0.0;
  for (int q = 0; q < ks.n; ++q) {
    const int k = ks.k[q];
    double num = 0.0, den = 0.0;
    for (int j = tid; j < n; j += kThreads) {
      const double v = w[j];
      int rank = 0;  // entries strictly before j in descending order
      for (int m = 0; m < n; ++m) {
        const double u = w[m];
        rank += (u > v) || (u == v && m < j);
      }
      if (rank < k) {
        const float s01 = (float)((raw[j] - lo) / span);
        num += v * (double)s01;
        den += v;
      }
    }
    num = wave_sum(num);
    den = wave_sum(den);
    __syncthreads();
    if (lane == 0) {
      red[0][wave] = num;
      red[1][wave] = den;
    }
    __syncthreads();
    if (tid == 0) {
      double a = 0.0, b = 0.0;
      for (int r = 0; r < kThreads / kWave; ++r) {
        a += red[0][r];
        b += red[1][r];
      }
      total += a / b;
    }
  }
  if (tid == 0) out[i] = (float)(total / ks.n);
}

}  // namespace rscin
}  // namespace musc

using namespace musc;

extern "C" int musc_rscin_f32(const float* cls_tokens, const double* image_scores, int n, int d, const int* k_list,
                              int n_k, float* out, hipStream_t stream) {
  if (!cls_tokens || !image_scores || !out || !k_list || n < 1 || d < 1 || n_k < 1) return MUSC_ERR_INVALID_ARG;
  if (n > rscin::kMaxN || n_k > rscin::kMaxK) return MUSC_ERR_UNSUPPORTED;
  rscin::KList ks{};
  ks.n = n_k;
  for (int q = 0; q < n_k; ++q) {
    if (k_list[q] < 1 || k_list[q] > n) return MUSC_ERR_INVALID_ARG;
    ks.k[q] = k_list[q];
  }
  hipLaunchKernelGGL(rscin::rscin_kernel, dim3(n), dim3(rscin::kThreads), (size_t)n * sizeof(double), stream,
                     cls_tokens, image_scores, n, d, ks, out);
  return check_launch();
}
