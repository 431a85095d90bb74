// Score-map epilogue for gfx950: layer/radius means, bilinear upsampling with
// align_corners=True, and the per-image maximum.
//
// Reference (models/musc.py:259-288): mean over the layers' (N, P) float64 maps,
// mean over radii, view (N, 1, side, side), F.interpolate(size=S, bilinear,
// align_corners=True), image score = max of each S x S map.
//
// One workgroup per (image, band of output rows: kRows when upsampling, fewer when a
// strong downsampling would make kRows rows span more than kMaxGridRows grid rows,
// down to one).  A band touches at most a few grid rows, so the workgroup averages
// only those rows of the n_radii * n_layers score maps into LDS, then writes its
// band of S-pixel rows (coalesced
// float64 rows) and merges its band maximum into image_scores with a 64-bit
// atomicMax on the bit pattern (all scores are non-negative distances, whose
// IEEE bits order like the values).  The maximum propagates NaN, as numpy's max
// at models/musc.py:288 does: NaN bit patterns (either sign) compare above every
// non-negative number as unsigned integers, so the atomic keeps them too.
#include "common.hpp"

namespace musc {
namespace epi {

constexpr int kRows = 8;           // output rows per band at most
constexpr int kThreads = 256;
constexpr int kMaxSide = 128;
constexpr int kMaxGridRows = 16;  // grid rows one band may touch

__device__ inline double nmax(double a, double b) { return __builtin_elementwise_maximum(a, b); }

__global__ __launch_bounds__(kThreads) void maps_kernel(const double* __restrict__ scores, int n_radii, int n_layers,
                                                        int n, int side, int out_size, int rows,
                                                        double* __restrict__ maps,
                                                        unsigned long long* __restrict__ image_bits) {
  const int bands = (out_size + rows - 1) / rows;
  const int img = blockIdx.x / bands, band = blockIdx.x % bands;
  const int y0 = band * rows;
  const int y1 = min(out_size, y0 + rows);
  const int P = side * side;
  const double scale = out_size > 1 ? (double)(side - 1) / (double)(out_size - 1) : 0.0;
  // grid rows touched by output rows y0..y1-1
  const int g0 = (int)(scale * y0);
  int g1 = (int)(scale * (y1 - 1));
  g1 = min(g1 + 1, side - 1);
  const int ng = g1 - g0 + 1;

  __shared__ double avg[kMaxGridRows][kMaxSide];
  for (int t = threadIdx.x; t < ng * side; t += blockDim.x) {
    const int gr = g0 + t / side, gc = t % side;
    const long long pix = (long long)gr * side + gc;
    double rsum = 0.0;
    for (int r = 0; r < n_radii; ++r) {
      double lsum = 0.0;
      for (int l = 0; l < n_layers; ++l) lsum += scores[(((long long)r * n_layers + l) * n + img) * P + pix];
      rsum += lsum / (double)n_layers;
    }
    avg[t / side][gc] = rsum / (double)n_radii;
  }
  __syncthreads();

  double vmax = 0.0;
  const int pixels = (y1 - y0) * out_size;
  for (int t = threadIdx.x; t < pixels; t += blockDim.x) {
    const int y = y0 + t / out_size, x = t % out_size;
    const double sy = scale * y, sx = scale * x;
    const int h0 = (int)sy, w0 = (int)sx;
    const int h1 = h0 < side - 1 ? h0 + 1 : h0;
    const int w1 = w0 < side - 1 ? w0 + 1 : w0;
    const double lh1 = sy - h0, lh0 = 1.0 - lh1;
    const double lw1 = sx - w0, lw0 = 1.0 - lw1;
    const double* r0 = avg[h0 - g0];
    const double* r1 = avg[h1 - g0];
    const double v = lh0 * (lw0 * r0[w0] + lw1 * r0[w1]) + lh1 * (lw0 * r1[w0] + lw1 * r1[w1]);
    if (maps) maps[((long long)img * out_size + y) * out_size + x] = v;
    vmax = nmax(vmax, v);
  }
  if (image_bits) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) vmax = nmax(vmax, __shfl_xor(vmax, off, kWave));
    __shared__ double wmax[kThreads / kWave];
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (lane == 0) wmax[wave] = vmax;
    __syncthreads();
    if (threadIdx.x == 0) {
      double m = wmax[0];
      for (int w = 1; w < (int)(blockDim.x / kWave); ++w) m = nmax(m, wmax[w]);
      atomicMax(image_bits + img, (unsigned long long)__double_as_longlong(m));
    }
  }
}

}  // namespace epi
}  // namespace musc

using namespace musc;

extern "C" int musc_maps_f64(const double* scores, int n_radii, int n_layers, int n, int side, int out_size,
                             double* maps, double* image_scores, hipStream_t stream) {
  if (!scores || n_radii < 1 || n_layers < 1 || n < 1 || side < 1 || out_size < 1) return MUSC_ERR_INVALID_ARG;
  if (!maps && !image_scores) return MUSC_ERR_INVALID_ARG;
  if (side > epi::kMaxSide) return MUSC_ERR_UNSUPPORTED;
  // a band of R output rows starting at y0 touches grid rows floor(scale y0) ..
  // floor(scale (y0 + R - 1)) + 1, at most floor(scale (R - 1)) + 3 of them: take the
  // largest R <= kRows within kMaxGridRows (R = 1 always is: 3 rows)
  const double scale = out_size > 1 ? (double)(side - 1) / (double)(out_size - 1) : 0.0;
  int rows = epi::kRows;
  while (rows > 1 && (int)(scale * (rows - 1)) + 3 > epi::kMaxGridRows) --rows;
  const int bands = (out_size + rows - 1) / rows;
  if ((long long)n * bands > 0x7fffffffLL) return MUSC_ERR_UNSUPPORTED;
  unsigned long long* bits = reinterpret_cast<unsigned long long*>(image_scores);
  if (bits) launch_fill_u32(reinterpret_cast<uint32_t*>(bits), (size_t)n * 2, 0u, stream);
  hipLaunchKernelGGL(epi::maps_kernel, dim3((unsigned)(n * bands)), dim3(epi::kThreads), 0, stream, scores, n_radii,
                     n_layers, n, side, out_size, rows, maps, bits);
  return check_launch();
}
