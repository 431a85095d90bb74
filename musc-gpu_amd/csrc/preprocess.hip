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

// One thread per output index: bounds (xmin - shift, count) and a row of `width`
// fixed-point coefficients (zero past the window).  identity: the axis keeps its size and is not resampled (window
// {xx, 1}, coefficient 1.0, which reproduces the byte exactly).
__global__ __launch_bounds__(kThreads) void coeff_kernel(int in_size, int out_size, int width, int shift,
                                                         int identity, int2* __restrict__ bounds,
                                                         int* __restrict__ kk) {
#pragma clang fp contract(off)
  const int xx = blockIdx.x * blockDim.x + threadIdx.x;
  if (xx >= out_size) return;
  int* k = kk + (long long)xx * width;
  if (identity) {
    bounds[xx] = make_int2(xx - shift, 1);
    k[0] = 1 << kPrecisionBits;
    for (int x = 1; x < width; ++x) k[x] = 0;
    return;
  }
  const AxisGeom g = axis_geom(in_size, out_size);
  double center;
  const int2 w = window(g, in_size, xx, &center);
  double ww = 0.0;
  for (int x = 0; x < w.y; ++x) ww += bicubic((x + w.x - center + 0.5) * g.ss);
  for (int x = 0; x < width; ++x) {
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

// Coefficient rows are kW ints wide (kW a multiple of 4, zero past the window), so
// a thread fetches its whole row with kW/4 independent 16-byte loads and the tap
// loops have a compile-time trip count: every load of a pixel is in flight at once.
// Taps past the window carry weight 0; their source index is clamped into the image.
template <int kW>
__device__ inline void load_coeffs(const int* __restrict__ k, int (&c)[kW]) {
  const int4* k4 = reinterpret_cast<const int4*>(k);
#pragma unroll
  for (int i = 0; i < kW / 4; ++i) {
    const int4 v = k4[i];
    c[4 * i + 0] = v.x;
    c[4 * i + 1] = v.y;
    c[4 * i + 2] = v.z;
    c[4 * i + 3] = v.w;
  }
}

// 22-bit fixed-point sums of kW taps of interleaved RGB bytes: tap x reads
// base + min(first + x, last) * stride.
template <int kW>
__device__ inline int3 tap_sums(const uint8_t* __restrict__ base, int first, int last, long long stride,
                                const int (&c)[kW]) {
  int s0 = 1 << (kPrecisionBits - 1), s1 = s0, s2 = s0;
#pragma unroll
  for (int x = 0; x < kW; ++x) {
    const int i = first + x < last ? first + x : last;
    const uint8_t* q = base + i * stride;
    s0 += (int)q[0] * c[x];
    s1 += (int)q[1] * c[x];
    s2 += (int)q[2] * c[x];
  }
  return make_int3(s0, s1, s2);
}

__device__ inline void store_normalised(float* __restrict__ o, long long plane, int3 s, const Norm& nrm) {
  const int u[3] = {clip8(s.x), clip8(s.y), clip8(s.z)};
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const float t = (float)u[c] / 255.0f;
    o[c * plane] = (t - nrm.mean[c]) / nrm.stdv[c];
  }
}

// Horizontal pass: tmp (batch, rows, out_w, 3) uint8 from source rows row0 .. row0+rows-1.
template <int kW>
__global__ __launch_bounds__(kThreads) void hpass_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ tmp,
                                                         int in_h, int in_w, int row0, int rows, int out_w,
                                                         const int2* __restrict__ bounds, const int* __restrict__ kk) {
  const int xx = blockIdx.x * kThreads + threadIdx.x;
  if (xx >= out_w) return;
  const int r = blockIdx.y, b = blockIdx.z;
  const uint8_t* row = src + (((long long)b * in_h + row0 + r) * in_w) * 3;
  const int2 bd = bounds[xx];
  int c[kW];
  load_coeffs<kW>(kk + (long long)xx * kW, c);
  const int3 s = tap_sums<kW>(row, bd.x, in_w - 1, 3, c);
  uint8_t* o = tmp + (((long long)b * rows + r) * out_w + xx) * 3;
  o[0] = (uint8_t)clip8(s.x);
  o[1] = (uint8_t)clip8(s.y);
  o[2] = (uint8_t)clip8(s.z);
}

// Vertical pass + ToTensor + Normalize: out (batch, 3, out_h, w) float32 from an
// interleaved uint8 (batch, rows, w, 3) image (the horizontal pass's output, or the
// source when the width is kept).
template <int kW>
__global__ __launch_bounds__(kThreads) void vpass_kernel(const uint8_t* __restrict__ img, int rows, int w, int out_h,
                                                         const int2* __restrict__ bounds, const int* __restrict__ kk,
                                                         Norm nrm, float* __restrict__ out) {
  const int xx = blockIdx.x * kThreads + threadIdx.x;
  if (xx >= w) return;
  const int yy = blockIdx.y, b = blockIdx.z;
  const int2 bd = bounds[yy];
  int c[kW];
  load_coeffs<kW>(kk + (long long)yy * kW, c);
  const int3 s = tap_sums<kW>(img + ((long long)b * rows * w + xx) * 3, bd.x, rows - 1, (long long)w * 3, c);
  const long long plane = (long long)out_h * w;
  store_normalised(out + (long long)b * 3 * plane + (long long)yy * w + xx, plane, s, nrm);
}

// Fused resize: one workgroup per (image, band of `band` output rows).  The source
// rows the band's vertical windows cover stream through a double-buffered LDS row
// (coalesced 4-byte loads, one row ahead in registers, one barrier per row), each is
// resampled horizontally into an LDS block of uint8 rows, and the vertical pass +
// ToTensor + Normalize then reads that block and writes the float32 planes.  The
// uint8 intermediate never reaches HBM.  A thread owns output columns tid + 256 j
// (j < kCols) in every row, so its horizontal coefficients are loaded into registers
// once; the band's vertical coefficient rows sit in LDS.  kT is the larger of the
// two axes' tap counts (odd, <= 15), kW its coefficient row width.  Needs
// in_w % 4 == 0 (4-byte aligned rows) and out_w <= 256 * kCols; the host sizes
// `band` and the dynamic LDS (fused_plan).
constexpr int kRowRegs = 16;     // 4-byte words per thread per staged row (in_w * 3 <= 16 KB)
constexpr int kCols = 3;         // output columns per thread (out_w <= 768)
constexpr int kFusedMaxTaps = 15;

struct FusedLayout {
  int rowpad;        // bytes per staged source row (x2 buffers), with slack for the widest window read
  int bstride;       // bytes per row of the uint8 block (out_w * 3 + 12 rounded up to 16)
  int blk;           // bytes of the uint8 block (nrows x bstride)
  size_t total;      // dynamic LDS bytes
};

__host__ __device__ inline FusedLayout fused_layout(int in_w, int out_w, int nrows, int band, int width) {
  FusedLayout f;
  f.rowpad = (in_w * 3 + 3 * width + 8 + 15) & ~15;
  f.bstride = (out_w * 3 + 12 + 15) & ~15;      // the last 4-column group's 12 bytes stay in the row
  f.blk = nrows * f.bstride;
  f.total = 2 * (size_t)f.rowpad + f.blk + (size_t)band * width * 4 + (size_t)band * 8;
  return f;
}

// Horizontal tap sums of one output pixel from an LDS row: the window's 3*kT bytes
// (kT = the axis' tap count, <= kW) start at byte a; they are read as aligned 4-byte
// words, realigned by a % 4 with v_alignbyte, and each byte is then at a
// compile-time position.
template <int kW, int kT>
__device__ inline int3 hsum_words(const uint8_t* __restrict__ row, int a, const int (&c)[kW]) {
  constexpr int kE = (3 * kT + 3) / 4;           // realigned words holding the 3*kT window bytes
  constexpr int kD = kE + 1;                      // words read: the window at any offset a % 4
  const uint32_t* w = reinterpret_cast<const uint32_t*>(row + (a & ~3));
  uint32_t d[kD];
#pragma unroll
  for (int i = 0; i < kD; ++i) d[i] = w[i];
  const uint32_t sh = (uint32_t)(a & 3);
  uint32_t e[kE];
#pragma unroll
  for (int i = 0; i < kE; ++i) e[i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], sh);
  int s0 = 1 << (kPrecisionBits - 1), s1 = s0, s2 = s0;
#pragma unroll
  for (int x = 0; x < kT; ++x) {
    const int j = 3 * x;
    s0 += (int)((e[j >> 2] >> (8 * (j & 3))) & 0xffu) * c[x];
    s1 += (int)((e[(j + 1) >> 2] >> (8 * ((j + 1) & 3))) & 0xffu) * c[x];
    s2 += (int)((e[(j + 2) >> 2] >> (8 * ((j + 2) & 3))) & 0xffu) * c[x];
  }
  return make_int3(s0, s1, s2);
}

template <int kW, int kT>
__global__ __launch_bounds__(kThreads) void fused_kernel(const uint8_t* __restrict__ src, int in_h, int in_w,
                                                         int out_h, int out_w, int band, int max_rows,
                                                         const int2* __restrict__ bh, const int* __restrict__ kh,
                                                         const int2* __restrict__ bv, const int* __restrict__ kv,
                                                         Norm nrm, float* __restrict__ out) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int b = blockIdx.y, tid = threadIdx.x;
  const int y0 = blockIdx.x * band;
  const int y1 = min(y0 + band, out_h);
  const int r0 = bv[y0].x;
  const int nrows = bv[y1 - 1].x + bv[y1 - 1].y - r0;
  // the host sized the LDS for max_rows source rows with the same window arithmetic
  if (nrows > max_rows) return;
  const FusedLayout f = fused_layout(in_w, out_w, max_rows, band, kW);
  const int words = in_w * 3 / 4;                 // 4-byte words per source row
  uint8_t* rowbuf = smem;                         // [2][rowpad]
  uint8_t* blk = smem + 2 * f.rowpad;             // [nrows][out_w][3]
  int* vk = reinterpret_cast<int*>(blk + f.blk);  // [band][kW] vertical coefficients of this band
  int2* vb = reinterpret_cast<int2*>(vk + band * kW);
  for (int i = tid; i < (y1 - y0) * kW; i += kThreads) vk[i] = kv[(long long)y0 * kW + i];
  for (int i = tid; i < y1 - y0; i += kThreads) vb[i] = bv[y0 + i];

  int2 hb[kCols];
  int hc[kCols][kW];
#pragma unroll
  for (int j = 0; j < kCols; ++j) {
    const int xx = tid + j * kThreads;
    hb[j] = make_int2(0, 0);
    if (xx < out_w) {
      hb[j] = bh[xx];
      load_coeffs<kW>(kh + (long long)xx * kW, hc[j]);
    } else {
#pragma unroll
      for (int x = 0; x < kW; ++x) hc[j][x] = 0;
    }
  }

  const uint32_t* img = reinterpret_cast<const uint32_t*>(src + (long long)b * in_h * in_w * 3);
  uint32_t stage[kRowRegs];
  auto load_row = [&](int r) {
    const uint32_t* g = img + (long long)(r0 + r) * words;
#pragma unroll
    for (int i = 0; i < kRowRegs; ++i) {
      const int w = tid + i * kThreads;
      if (w < words) stage[i] = g[w];
    }
  };
  load_row(0);
  for (int r = 0; r < nrows; ++r) {
    uint32_t* buf = reinterpret_cast<uint32_t*>(rowbuf + (r & 1) * f.rowpad);
#pragma unroll
    for (int i = 0; i < kRowRegs; ++i) {
      const int w = tid + i * kThreads;
      if (w < words) buf[w] = stage[i];
    }
    if (r + 1 < nrows) load_row(r + 1);
    __syncthreads();
    const uint8_t* row = rowbuf + (r & 1) * f.rowpad;
    uint8_t* dst = blk + r * f.bstride;
#pragma unroll
    for (int j = 0; j < kCols; ++j) {
      const int xx = tid + j * kThreads;
      if (xx < out_w) {
        // taps past the window carry weight 0; they read the row's slack bytes
        const int3 s = hsum_words<kW, kT>(row, hb[j].x * 3, hc[j]);
        dst[xx * 3 + 0] = (uint8_t)clip8(s.x);
        dst[xx * 3 + 1] = (uint8_t)clip8(s.y);
        dst[xx * 3 + 2] = (uint8_t)clip8(s.z);
      }
    }
  }
  __syncthreads();
  // vertical pass: a thread takes 4 adjacent output columns (12 bytes = 3 aligned words
  // of a block row per tap; the padded row stride keeps them aligned)
  const long long plane = (long long)out_h * out_w;
  float* o = out + (long long)b * 3 * plane;
  const int groups = (out_w + 3) / 4;
  const int n = (y1 - y0) * groups;
  for (int idx = tid; idx < n; idx += kThreads) {
    const int yl = idx / groups, x0 = 4 * (idx % groups);
    const int2 bd = vb[yl];
    int c[kW];
#pragma unroll
    for (int x = 0; x < kW; ++x) c[x] = vk[yl * kW + x];
    int acc[12];
#pragma unroll
    for (int q = 0; q < 12; ++q) acc[q] = 1 << (kPrecisionBits - 1);
#pragma unroll
    for (int y = 0; y < kT; ++y) {
      const int rr = min(bd.x - r0 + y, nrows - 1);     // weight 0 past the window
      const uint32_t* w = reinterpret_cast<const uint32_t*>(blk + rr * f.bstride + x0 * 3);
      const uint32_t d[3] = {w[0], w[1], w[2]};
#pragma unroll
      for (int q = 0; q < 12; ++q) acc[q] += (int)((d[q >> 2] >> (8 * (q & 3))) & 0xffu) * c[y];
    }
    float* orow = o + (long long)(y0 + yl) * out_w + x0;
#pragma unroll
    for (int px = 0; px < 4; ++px) {
      if (x0 + px < out_w)
        store_normalised(orow + px, plane, make_int3(acc[3 * px], acc[3 * px + 1], acc[3 * px + 2]), nrm);
    }
  }
}

// Band (output rows per workgroup) and LDS of the fused kernel, or band 0 when it does
// not apply: the largest band (<= 32 rows) whose block fits 64 KB.  Larger bands
// recompute fewer halo rows, smaller blocks let more workgroups share a CU; measured at
// 1024 -> 518 the 64 KB choice (band 8, three workgroups per CU) beat both a 40 KB one
// (band 4) and a 78 KB one (band 16, two per CU; 14 % slower).
constexpr size_t kFusedLdsBudget = 64 * 1024;

struct FusedPlan {
  int band, max_rows;
  size_t lds;
};

inline FusedPlan fused_plan(int in_h, int in_w, int out_h, int out_w, const AxisGeom& gv, int taps, int width) {
  FusedPlan best{0, 0, 0};
  if (in_w % 4 != 0 || in_w * 3 > kRowRegs * kThreads * 4 || out_w > kCols * kThreads || taps > kFusedMaxTaps)
    return best;
  for (int band = 32; band >= 1; band /= 2) {
    int worst = 0;
    for (int y0 = 0; y0 < out_h; y0 += band) {
      const int y1 = y0 + band < out_h ? y0 + band : out_h;
      const int2 a = window(gv, in_h, y0, nullptr), z = window(gv, in_h, y1 - 1, nullptr);
      worst = worst > z.x + z.y - a.x ? worst : z.x + z.y - a.x;
    }
    const FusedLayout f = fused_layout(in_w, out_w, worst, band, width);
    if (f.total <= kFusedLdsBudget) return FusedPlan{band, worst, f.total};
  }
  return best;
}

// Coefficient row widths the kernels are instantiated for.
inline int table_width(int taps) {
  const int widths[] = {4, 8, 12, 16, 24, 32, 48, 64};
  for (int w : widths)
    if (taps <= w) return w;
  return 0;
}

// Workspace: h-axis bounds + coefficients | v-axis bounds + coefficients | uint8 intermediate.
struct Plan {
  AxisGeom gh, gv;
  bool need_h, need_v;
  int band;                  // > 0: the fused kernel runs with this many output rows per workgroup
  int max_rows;              // fused kernel: most source rows a band reads
  size_t lds;                // fused kernel: dynamic LDS bytes
  int width;                 // coefficient row width (both axes): a bucket >= the taps of either axis
  int taps;                  // the larger of the two axes' tap counts
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
  p.taps = p.gh.taps > p.gv.taps ? p.gh.taps : p.gv.taps;
  p.width = table_width(p.taps);
  const FusedPlan fp = (p.need_h && p.need_v) ? fused_plan(in_h, in_w, out_h, out_w, p.gv, p.taps, p.width)
                                              : FusedPlan{0, 0, 0};
  p.band = fp.band;
  p.max_rows = fp.max_rows;
  p.lds = fp.lds;
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
  off = align_up(off + (size_t)out_w * p.width * sizeof(int), 256);
  p.off_bv = off;
  off = align_up(off + (size_t)out_h * sizeof(int2), 256);
  p.off_kv = off;
  off = align_up(off + (size_t)out_h * p.width * sizeof(int), 256);
  p.off_tmp = off;
  if (p.need_h && p.band == 0) off = align_up(off + (size_t)batch * p.rows * out_w * 3, 256);
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
  if (p.band > 0 && (reinterpret_cast<uintptr_t>(images) & 3) != 0) return MUSC_ERR_INVALID_ARG;
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
  // the two-pass path reads the horizontal pass's rows from 0; the fused kernel reads source rows
  const int vshift = (p.need_h && p.band == 0) ? p.row0 : 0;
  hipLaunchKernelGGL(prep::coeff_kernel, dim3((out_w + T - 1) / T), dim3(T), 0, stream, in_w, out_w, p.width, 0,
                     p.need_h ? 0 : 1, bh, kh);
  hipLaunchKernelGGL(prep::coeff_kernel, dim3((out_h + T - 1) / T), dim3(T), 0, stream, in_h, out_h, p.width,
                     vshift, p.need_v ? 0 : 1, bv, kv);
  if (p.band > 0) {
#define MUSC_PREP_FUSED(W, TAPS)                                                                                   \
  hipLaunchKernelGGL((prep::fused_kernel<W, TAPS>), dim3((out_h + p.band - 1) / p.band, batch), dim3(T), p.lds,    \
                     stream, images, in_h, in_w, out_h, out_w, p.band, p.max_rows, bh, kh, bv, kv, nrm, out)
    switch (p.taps) {
      case 1: case 3: case 5: MUSC_PREP_FUSED(8, 5); break;   // taps are odd; short windows use 5 (zero weights)
      case 7: MUSC_PREP_FUSED(8, 7); break;
      case 9: MUSC_PREP_FUSED(12, 9); break;
      case 11: MUSC_PREP_FUSED(12, 11); break;
      case 13: MUSC_PREP_FUSED(16, 13); break;
      case 15: MUSC_PREP_FUSED(16, 15); break;
      default: return MUSC_ERR_UNSUPPORTED;
    }
#undef MUSC_PREP_FUSED
    return check_launch();
  }
#define MUSC_PREP_LAUNCH(W)                                                                                        \
  if (p.need_h) {                                                                                                  \
    hipLaunchKernelGGL(prep::hpass_kernel<W>, dim3((out_w + T - 1) / T, p.rows, batch), dim3(T), 0, stream,       \
                       images, tmp, in_h, in_w, p.row0, p.rows, out_w, bh, kh);                                     \
    hipLaunchKernelGGL(prep::vpass_kernel<W>, dim3((out_w + T - 1) / T, out_h, batch), dim3(T), 0, stream, tmp,   \
                       p.rows, out_w, out_h, bv, kv, nrm, out);                                                    \
  } else {                                                                                                         \
    hipLaunchKernelGGL(prep::vpass_kernel<W>, dim3((out_w + T - 1) / T, out_h, batch), dim3(T), 0, stream, images,\
                       in_h, in_w, out_h, bv, kv, nrm, out);                                                       \
  }
  switch (p.width) {
    case 4: MUSC_PREP_LAUNCH(4); break;
    case 8: MUSC_PREP_LAUNCH(8); break;
    case 12: MUSC_PREP_LAUNCH(12); break;
    case 16: MUSC_PREP_LAUNCH(16); break;
    case 24: MUSC_PREP_LAUNCH(24); break;
    case 32: MUSC_PREP_LAUNCH(32); break;
    case 48: MUSC_PREP_LAUNCH(48); break;
    case 64: MUSC_PREP_LAUNCH(64); break;
    default: return MUSC_ERR_UNSUPPORTED;
  }
#undef MUSC_PREP_LAUNCH
  return check_launch();
}
