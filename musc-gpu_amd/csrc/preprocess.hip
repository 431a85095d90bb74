// Image preprocessing of the data path on gfx950: decoded uint8 RGB images ->
// the encoder's normalised float32 planes, bit-identical to the reference's
// evaluation transform (models/backbone/open_clip/transform.py:118-133: Resize((S,
// S), BICUBIC) on a PIL image, CenterCrop, ToTensor, Normalize), which torchvision
// runs per image on the CPU inside the dataset item (datasets/mvtec.py:101-103).
//
// The resize is Pillow's 8-bit resampling (Pillow pinned at 11.1.0 by the
// reference, requirements.txt:13): per axis a table of 22-bit fixed-point bicubic
// coefficients (a = -0.5, support 2 stretched by max(in/out, 1)), then a horizontal
// pass over the source rows the vertical pass reads, rounding to uint8, then a
// vertical pass rounding to uint8 again; an axis that keeps its size is not
// resampled.  The coefficient tables are computed on the device with the same IEEE
// double operations in the same order as Pillow's C code (FP contraction off, so no
// fused multiply-add changes a rounding), which makes the fixed-point tables, and
// hence the integer passes, identical.  ToTensor (u8 / 255) and Normalize ((x -
// mean) / std) are fused into the vertical pass as correctly rounded float32
// division and subtraction, the operations torch performs on the CPU.
#include "common.hpp"

namespace musc {
namespace prep {

constexpr int kPrecisionBits = 22;
constexpr int kMaxTaps = 64;     // taps = 2*ceil(2*max(in/out, 1)) + 1, so in/out <= 15.5
constexpr int kThreads = 256;

struct Norm {
  float mean[3];
  float stdv[3];
};

// FP contraction is off in the coefficient code: a fused multiply-add would round
// differently from Pillow's separate multiply and add.
__host__ __device__ inline double bicubic(double x) {
#pragma clang fp contract(off)
  const double a = -0.5;
  if (x < 0.0) x = -x;
  if (x < 1.0) return ((a + 2.0) * x - (a + 3.0)) * x * x + 1;
  if (x < 2.0) return (((x - 5) * x + 8) * x - 4) * a;
  return 0.0;
}

struct AxisGeom {
  double scale, support, ss;
  int taps;
};

__host__ __device__ inline AxisGeom axis_geom(int in_size, int out_size) {
#pragma clang fp contract(off)
  AxisGeom g;
  g.scale = (double)in_size / out_size;
  const double filterscale = g.scale < 1.0 ? 1.0 : g.scale;
  g.support = 2.0 * filterscale;
  g.ss = 1.0 / filterscale;
  g.taps = (int)ceil(g.support) * 2 + 1;
  return g;
}

// Source window [xmin, xmin + count) of output index xx and its center.
__host__ __device__ inline int2 window(const AxisGeom& g, int in_size, int xx, double* center_out) {
#pragma clang fp contract(off)
  const double center = 0.0 + (xx + 0.5) * g.scale;
  int xmin = (int)(center - g.support + 0.5);
  if (xmin < 0) xmin = 0;
  int xmax = (int)(center + g.support + 0.5);
  if (xmax > in_size) xmax = in_size;
  if (center_out) *center_out = center;
  return make_int2(xmin, xmax - xmin);
}

// One thread per output index: bounds (xmin - shift, count) and `taps` fixed-point
// coefficients.  identity: the axis keeps its size and is not resampled (window
// {xx, 1}, coefficient 1.0, which reproduces the byte exactly).
__global__ __launch_bounds__(kThreads) void coeff_kernel(int in_size, int out_size, int taps, int shift,
                                                         int identity, int2* __restrict__ bounds,
                                                         int* __restrict__ kk) {
#pragma clang fp contract(off)
  const int xx = blockIdx.x * blockDim.x + threadIdx.x;
  if (xx >= out_size) return;
  int* k = kk + (long long)xx * taps;
  if (identity) {
    bounds[xx] = make_int2(xx - shift, 1);
    k[0] = 1 << kPrecisionBits;
    for (int x = 1; x < taps; ++x) k[x] = 0;
    return;
  }
  const AxisGeom g = axis_geom(in_size, out_size);
  double center;
  const int2 w = window(g, in_size, xx, &center);
  double ww = 0.0;
  for (int x = 0; x < w.y; ++x) ww += bicubic((x + w.x - center + 0.5) * g.ss);
  for (int x = 0; x < taps; ++x) {
    int q = 0;
    if (x < w.y) {
      double v = bicubic((x + w.x - center + 0.5) * g.ss);
      if (ww != 0.0) v /= ww;
      q = v < 0 ? (int)(-0.5 + v * (1 << kPrecisionBits)) : (int)(0.5 + v * (1 << kPrecisionBits));
    }
    k[x] = q;
  }
  bounds[xx] = make_int2(w.x - shift, w.y);
}

__device__ inline int clip8(int acc) {
  if (acc >= (1 << kPrecisionBits << 8)) return 255;
  if (acc <= 0) return 0;
  return acc >> kPrecisionBits;
}

// Horizontal pass: tmp (batch, rows, out_w, 3) uint8 from source rows row0 .. row0+rows-1.
__global__ __launch_bounds__(kThreads) void hpass_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ tmp,
                                                         int in_h, int in_w, int row0, int rows, int out_w, int taps,
                                                         const int2* __restrict__ bounds, const int* __restrict__ kk) {
  const int xx = blockIdx.x * kThreads + threadIdx.x;
  if (xx >= out_w) return;
  const int r = blockIdx.y, b = blockIdx.z;
  const uint8_t* row = src + (((long long)b * in_h + row0 + r) * in_w) * 3;
  const int2 bd = bounds[xx];
  const int* k = kk + (long long)xx * taps;
  int s0 = 1 << (kPrecisionBits - 1), s1 = s0, s2 = s0;
  for (int x = 0; x < bd.y; ++x) {
    const uint8_t* p = row + (bd.x + x) * 3;
    const int c = k[x];
    s0 += (int)p[0] * c;
    s1 += (int)p[1] * c;
    s2 += (int)p[2] * c;
  }
  uint8_t* o = tmp + (((long long)b * rows + r) * out_w + xx) * 3;
  o[0] = (uint8_t)clip8(s0);
  o[1] = (uint8_t)clip8(s1);
  o[2] = (uint8_t)clip8(s2);
}

// Vertical pass + ToTensor + Normalize: out (batch, 3, out_h, w) float32 from an
// interleaved uint8 (batch, rows, w, 3) image (the horizontal pass's output, or the
// source when the width is kept).
__global__ __launch_bounds__(kThreads) void vpass_kernel(const uint8_t* __restrict__ img, int rows, int w, int out_h,
                                                         int taps, const int2* __restrict__ bounds,
                                                         const int* __restrict__ kk, Norm nrm,
                                                         float* __restrict__ out) {
  const int xx = blockIdx.x * kThreads + threadIdx.x;
  if (xx >= w) return;
  const int yy = blockIdx.y, b = blockIdx.z;
  const int2 bd = bounds[yy];
  const int* k = kk + (long long)yy * taps;
  const uint8_t* col = img + ((long long)b * rows * w + xx) * 3;
  int s0 = 1 << (kPrecisionBits - 1), s1 = s0, s2 = s0;
  for (int y = 0; y < bd.y; ++y) {
    const uint8_t* p = col + (long long)(bd.x + y) * w * 3;
    const int c = k[y];
    s0 += (int)p[0] * c;
    s1 += (int)p[1] * c;
    s2 += (int)p[2] * c;
  }
  const long long plane = (long long)out_h * w;
  float* o = out + (long long)b * 3 * plane + (long long)yy * w + xx;
  const int u[3] = {clip8(s0), clip8(s1), clip8(s2)};
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const float t = (float)u[c] / 255.0f;
    o[c * plane] = (t - nrm.mean[c]) / nrm.stdv[c];
  }
}

// Workspace: h-axis bounds + coefficients | v-axis bounds + coefficients | uint8 intermediate.
struct Plan {
  AxisGeom gh, gv;
  bool need_h, need_v;
  int row0, rows;            // source rows the vertical pass reads (horizontal pass extent)
  size_t off_bh, off_kh, off_bv, off_kv, off_tmp, total;
};

inline Plan plan(int batch, int in_h, int in_w, int out_h, int out_w) {
  Plan p;
  p.gh = axis_geom(in_w, out_w);
  p.gv = axis_geom(in_h, out_h);
  p.need_h = out_w != in_w;
  p.need_v = out_h != in_h;
  if (!p.need_h) p.gh.taps = 1;
  if (!p.need_v) p.gv.taps = 1;
  if (p.need_h && p.need_v) {
    const int2 first = window(p.gv, in_h, 0, nullptr);
    const int2 last = window(p.gv, in_h, out_h - 1, nullptr);
    p.row0 = first.x;
    p.rows = last.x + last.y - first.x;
  } else {
    p.row0 = 0;
    p.rows = in_h;
  }
  size_t off = 0;
  p.off_bh = off;
  off = align_up(off + (size_t)out_w * sizeof(int2), 256);
  p.off_kh = off;
  off = align_up(off + (size_t)out_w * p.gh.taps * sizeof(int), 256);
  p.off_bv = off;
  off = align_up(off + (size_t)out_h * sizeof(int2), 256);
  p.off_kv = off;
  off = align_up(off + (size_t)out_h * p.gv.taps * sizeof(int), 256);
  p.off_tmp = off;
  if (p.need_h) off = align_up(off + (size_t)batch * p.rows * out_w * 3, 256);
  p.total = off;
  return p;
}

inline int validate(int batch, int in_h, int in_w, int out_h, int out_w) {
  if (batch < 1 || in_h < 1 || in_w < 1 || out_h < 1 || out_w < 1) return MUSC_ERR_INVALID_ARG;
  if (batch > 65535 || out_h > 65535 || in_h > 65535) return MUSC_ERR_UNSUPPORTED;  // grid y / z limits
  if ((long long)in_h * in_w * 3 > (1LL << 31)) return MUSC_ERR_UNSUPPORTED;
  const AxisGeom gh = axis_geom(in_w, out_w), gv = axis_geom(in_h, out_h);
  if (gh.taps > kMaxTaps || gv.taps > kMaxTaps) return MUSC_ERR_UNSUPPORTED;
  return MUSC_OK;
}

}  // namespace prep
}  // namespace musc

using namespace musc;

extern "C" int musc_preprocess_workspace_bytes(int batch, int in_h, int in_w, int out_h, int out_w, size_t* out) {
  if (!out) return MUSC_ERR_INVALID_ARG;
  const int rc = prep::validate(batch, in_h, in_w, out_h, out_w);
  if (rc) return rc;
  *out = prep::plan(batch, in_h, in_w, out_h, out_w).total;
  return MUSC_OK;
}

extern "C" int musc_preprocess_u8(const uint8_t* images, int batch, int in_h, int in_w, int out_h, int out_w,
                                  const float* mean3, const float* std3, float* out, void* workspace,
                                  size_t workspace_bytes, hipStream_t stream) {
  if (!images || !mean3 || !std3 || !out) return MUSC_ERR_INVALID_ARG;
  int rc = prep::validate(batch, in_h, in_w, out_h, out_w);
  if (rc) return rc;
  const prep::Plan p = prep::plan(batch, in_h, in_w, out_h, out_w);
  if (!workspace || workspace_bytes < p.total) return MUSC_ERR_WORKSPACE;
  prep::Norm nrm;
  for (int c = 0; c < 3; ++c) {
    if (!(std3[c] != 0.0f)) return MUSC_ERR_INVALID_ARG;
    nrm.mean[c] = mean3[c];
    nrm.stdv[c] = std3[c];
  }
  char* ws = static_cast<char*>(workspace);
  auto* bh = reinterpret_cast<int2*>(ws + p.off_bh);
  auto* kh = reinterpret_cast<int*>(ws + p.off_kh);
  auto* bv = reinterpret_cast<int2*>(ws + p.off_bv);
  auto* kv = reinterpret_cast<int*>(ws + p.off_kv);
  auto* tmp = reinterpret_cast<uint8_t*>(ws + p.off_tmp);
  const int T = prep::kThreads;
  hipLaunchKernelGGL(prep::coeff_kernel, dim3((out_w + T - 1) / T), dim3(T), 0, stream, in_w, out_w, p.gh.taps, 0,
                     p.need_h ? 0 : 1, bh, kh);
  hipLaunchKernelGGL(prep::coeff_kernel, dim3((out_h + T - 1) / T), dim3(T), 0, stream, in_h, out_h, p.gv.taps,
                     p.need_h ? p.row0 : 0, p.need_v ? 0 : 1, bv, kv);
  if (p.need_h) {
    hipLaunchKernelGGL(prep::hpass_kernel, dim3((out_w + T - 1) / T, p.rows, batch), dim3(T), 0, stream, images, tmp,
                       in_h, in_w, p.row0, p.rows, out_w, p.gh.taps, bh, kh);
    hipLaunchKernelGGL(prep::vpass_kernel, dim3((out_w + T - 1) / T, out_h, batch), dim3(T), 0, stream, tmp, p.rows,
                       out_w, out_h, p.gv.taps, bv, kv, nrm, out);
  } else {
    hipLaunchKernelGGL(prep::vpass_kernel, dim3((out_w + T - 1) / T, out_h, batch), dim3(T), 0, stream, images, in_h,
                       in_w, out_h, p.gv.taps, bv, kv, nrm, out);
  }
  return check_launch();
}
