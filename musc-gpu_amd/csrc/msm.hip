// Mutual scoring module (MSM) for gfx950.
//
// Reference semantics (models/modules/_MSM.py:10-30,53-59): for every patch q of
// image i, d(q, j) = min_r ||z[i,q] - z[j,r]||_2 for every other image j, then the
// score is the mean of ascending ranks [a, b) of {d(q, j)}_{j != i}.
//
// MI355X design
//   1. msm_norms_kernel      ||z_row||^2 for all n*p rows (one wave per row).
//   2. fill                  per-(row, image) minima buffer := +inf bits.
//   3. msm_pair_min_kernel   (msm_pair.hip) the whole pool is one (n*p) x (n*p) Gram
//                            matrix; the upper triangle of 128x128 tiles on fp32
//                            MFMA, each tile reduced along rows and columns into
//                            the per-(patch, image) minima keys.
//   4. msm_refine_kernel     exact minima where ||a||^2 + ||b||^2 - 2 a.b cancels.
//   5. msm_rank_*_kernel     ranks each patch's n-1 minima (NaN last) and averages
//                            the square roots of ranks [a, b): sorted register
//                            lists of the b smallest (b <= 32; two lanes per patch,
//                            merged by a bitonic network), or the a-th and b-th
//                            smallest by a binary search over the key bits (one
//                            lane per patch for n <= 192, one wave per patch beyond).
#include <mutex>

#include "msm_common.hpp"

namespace musc {
namespace msm {

// ---------------------------------------------------------------------------
// Row norms.
// ---------------------------------------------------------------------------
// norms[row] = ||z_row||^2 and inv[row] = 1.  With `normalize`, the row is
// treated as z / ||z|| (the L2 normalisation of models/musc.py:238 applied on the
// fly): inv[row] = 1 / ||z_row|| and norms[row] = ||z_row||^2 * inv^2.  scale[row]
// (the refinement's row scale) = inv[row].
__global__ __launch_bounds__(256) void msm_norms_kernel(const float* __restrict__ z, int rows, int c,
                                                        int normalize, float* __restrict__ norms,
                                                        float* __restrict__ inv, float* __restrict__ scale) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const long long row = (long long)blockIdx.x * (blockDim.x / kWave) + wave;
  if (row >= rows) return;
  const double acc = row_sumsq(z + row * (long long)c, c, lane);
  if (lane == 0) {
    float nrm, s;
    if (normalize) {
      const double r = 1.0 / sqrt(acc);
      s = (float)r;
      nrm = (float)(acc * r * r);
    } else {
      s = 1.f;
      nrm = (float)acc;
    }
    inv[row] = s;
    scale[row] = s;
    norms[row] = nrm;
  }
}

// ---------------------------------------------------------------------------
// Trimmed rank means.  A row's minima keys (own image excluded) are ranked in
// ascending order, NaN last (torch.topk(largest=False) of models/modules/_MSM.py:27
// ranks NaN after every number).  The score is (S(b) - S(a)) / (b - a), S(k) being
// the sum of the square roots of the k smallest minima (fp64), rounded to fp32 like
// the reference's fp32 mean and widened (:30, :57).  With t the k-th smallest key,
//   S(k) = sum_{key < t} sqrt(key) + (k - #{key < t}) * sqrt(t),
// which holds for any ties; a NaN among the k smallest makes t = 0xffffffff (the NaN
// key) and S(k) NaN, as the reference's mean over a window holding a NaN.
// ---------------------------------------------------------------------------
constexpr uint32_t kNoKey = 0xffffffffu;  // NaN minimum, own image, or padding

// One thread per row, its n keys in registers (n <= kKeys).  t is found by a binary
// search over the key bits: the largest t with #{key < t} < k, built from the most
// significant bit down (32 steps of one compare and one add per key).  A workgroup is
// one wave of 64 consecutive rows; their keys pass through LDS in chunks of 32 images
// (coalesced loads of 32 consecutive words per row, a pitch of 33 words so that each
// lane reading its own row hits a distinct bank), which keeps the LDS per wave at 8 KB.
constexpr int kRankRows = 64;
constexpr int kRankChunk = 32;

template <int kKeys>
__global__ __launch_bounds__(kRankRows) void msm_rank_select_kernel(const uint32_t* __restrict__ minbits, int rows,
                                                                    int n, int p, int a, int b,
                                                                    double* __restrict__ scores) {
  __shared__ uint32_t s_chunk[kRankRows * (kRankChunk + 1)];
  const int t = threadIdx.x;
  const long long row0 = (long long)blockIdx.x * kRankRows;
  const int nrows = (int)min((long long)kRankRows, rows - row0);
  const long long row = row0 + t;
  const int self = t < nrows ? (int)(row / p) : -1;
  uint32_t key[kKeys];
#pragma unroll
  for (int c0 = 0; c0 < kKeys; c0 += kRankChunk) {
    // 64 rows x 32 images: lanes 32h .. 32h+31 of step i read row 2i + h
#pragma unroll 8
    for (int i = 0; i < kRankRows / 2; ++i) {
      const int r = 2 * i + (t >> 5), k = t & 31;
      uint32_t v = kNoKey;
      if (r < nrows && c0 + k < n) v = minbits[(row0 + r) * n + c0 + k];
      s_chunk[r * (kRankChunk + 1) + k] = v;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kRankChunk; ++k) {
      const int j = c0 + k;
      if (j < kKeys) {
        const uint32_t v = s_chunk[t * (kRankChunk + 1) + k];
        key[j] = (j < n && j != self) ? key_bits(v) : kNoKey;
      }
    }
    __syncthreads();
  }
  if (t >= nrows) return;
  uint32_t ta = 0, tb = 0;  // a-th and b-th smallest keys (ta stays 0 for a = 0)
  if (a == 0) {
#pragma unroll 1
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t cb = tb | (1u << bit);
      int nb = 0;
#pragma unroll
      for (int q = 0; q < kKeys; ++q) nb += key[q] < cb;
      tb = nb < b ? cb : tb;
    }
  } else {
#pragma unroll 1
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t ca = ta | (1u << bit), cb = tb | (1u << bit);
      int na = 0, nb = 0;
#pragma unroll
      for (int q = 0; q < kKeys; ++q) {
        na += key[q] < ca;
        nb += key[q] < cb;
      }
      ta = na < a ? ca : ta;
      tb = nb < b ? cb : tb;
    }
  }
  double sa = 0.0, sb = 0.0;
  int la = 0, lb = 0;
#pragma unroll
  for (int q = 0; q < kKeys; ++q) {
    const double r = (double)sqrtf(__uint_as_float(key[q]));
    if (key[q] < tb) {
      sb += r;
      ++lb;
    }
    if (key[q] < ta) {
      sa += r;
      ++la;
    }
  }
  sb += (double)(b - lb) * (double)sqrtf(__uint_as_float(tb));
  if (a > 0) sa += (double)(a - la) * (double)sqrtf(__uint_as_float(ta));
  // S(a) is infinite only when the a-th smallest key is +inf: every key of the window
  // is then +inf or NaN, and the window's mean is S(b) itself (+inf, or NaN when a NaN
  // falls inside), where S(b) - S(a) would give inf - inf = NaN
  const double win = isinf(sa) ? sb : sb - sa;
  scores[row] = (double)(float)(win / (double)(b - a));
}

// Short windows (b <= 32, every BASELINE configuration): ascending register lists of
// the kList smallest keys, each key inserted by a min/max pass down the list (2 kList
// instructions per key, against 64 per register slot for the bit search).  Two lanes
// per row: lane lr of each wave half takes row lr of the workgroup's 32 and half of
// its keys (lower half the first (n+1)/2 images, upper half the rest) into its own
// list.  The lower lane then takes its partner's list through v_permlane32_swap, forms
// C[i] = min(A[i], B[N2-1-i]) over both lists padded to N2 = a power of two >= kList
// (the N2 smallest of the union, a bitonic sequence: A ascending against B descending),
// sorts it with a bitonic merge (log2 N2 stages of min/max pairs) and sums ranks [a, b)
// in ascending order: the same keys in the same order as one list over all n keys.
// Rows start every n words in LDS; for even n a lane starts at key lr of its half so
// that the 32 lanes of a half read 32 distinct banks (for odd n they already do).
constexpr int kRank2Rows = 32;

template <int kList>
__global__ __launch_bounds__(kWave) void msm_rank_insert2_kernel(const uint32_t* __restrict__ minbits, int rows,
                                                                 int n, int p, int a, int b,
                                                                 double* __restrict__ scores) {
  constexpr int N2 = kList <= 8 ? 8 : (kList <= 16 ? 16 : 32);
  extern __shared__ __attribute__((aligned(16))) uint32_t s_rowkeys[];  // kRank2Rows * n
  const int t = threadIdx.x;
  const int lr = t & 31, lh = t >> 5;
  const long long row0 = (long long)blockIdx.x * kRank2Rows;
  const int nrows = (int)min((long long)kRank2Rows, rows - row0);
  const int count = nrows * n;
  const uint32_t* src = minbits + row0 * n;
  // row0 * n * 4 bytes is a multiple of 128: 16-byte loads are aligned
  const int n4 = count / 4;
  for (int i = t; i < n4; i += kWave) reinterpret_cast<uint4*>(s_rowkeys)[i] = reinterpret_cast<const uint4*>(src)[i];
  for (int i = 4 * n4 + t; i < count; i += kWave) s_rowkeys[i] = src[i];
  __syncthreads();
  // every lane runs the exchange below; lanes past the last row work on row 0's keys
  const bool active = lr < nrows;
  const int rr = active ? lr : 0;
  const long long row = row0 + rr;
  const int self = (int)(row / p);
  const uint32_t* mine = s_rowkeys + rr * n;
  const int h = (n + 1) / 2;
  const int first = lh ? h : 0, cnt = lh ? n - h : h;  // cnt >= 1 for n >= 2
  uint32_t list[kList];
#pragma unroll
  for (int i = 0; i < kList; ++i) list[i] = kNoKey;
  int j = first + ((n & 1) ? 0 : rr % cnt);  // distinct banks across the half's lanes
#pragma unroll 2
  for (int q = 0; q < cnt; ++q) {
    const uint32_t v = mine[j];
    uint32_t x = j != self ? key_bits(v) : kNoKey;
#pragma unroll
    for (int i = 0; i < kList; ++i) {
      const uint32_t lo = min(list[i], x);
      x = max(list[i], x);
      list[i] = lo;
    }
    j = j + 1 == first + cnt ? first : j + 1;
  }
  // lower lanes: partner's list (the upper lanes' registers reach them through the swap)
  uint32_t other[kList];
#pragma unroll
  for (int i = 0; i < kList; ++i) other[i] = __builtin_amdgcn_permlane32_swap(list[i], list[i], false, false)[1];
  uint32_t cc[N2];
#pragma unroll
  for (int i = 0; i < N2; ++i) {
    const uint32_t ai = i < kList ? list[i] : kNoKey;
    const uint32_t bi = N2 - 1 - i < kList ? other[N2 - 1 - i] : kNoKey;
    cc[i] = min(ai, bi);
  }
#pragma unroll
  for (int s = N2 / 2; s >= 1; s >>= 1)
#pragma unroll
    for (int i = 0; i < N2; ++i)
      if ((i & s) == 0) {
        const uint32_t x = cc[i], y = cc[i + s];
        cc[i] = min(x, y);
        cc[i + s] = max(x, y);
      }
  if (lh || !active) return;
  double sum = 0.0;
#pragma unroll
  for (int i = 0; i < kList; ++i)
    if (i >= a && i < b) sum += (double)sqrtf(__uint_as_float(cc[i]));
  scores[row] = (double)(float)(sum / (double)(b - a));
}

// Rows of more than 192 images: one wave per row.  Slot i of lane l holds key 64 i + l of
// the row (the own image and the slots past n hold kNoKey, which no threshold counts),
// and the a-th and b-th smallest keys are found by the same 32-step search over the key
// bits as msm_rank_select_kernel.  Each count #{key < t} is the sum over slots of the
// popcount of a ballot (one compare per slot, the sum wave-uniform in scalar registers,
// no cross-lane reduction), so a row costs 64 ceil(n / 64) compares where counting every
// key's rank cost n^2 / 64 per lane (16 ms against 4 ms per call at N = 400, P = 1369).
constexpr int kRankWaves = 4;
constexpr int kMaxSelectKeys = 192;

template <int kSlots>
__global__ __launch_bounds__(kRankWaves * kWave) void msm_rank_wave_kernel(
    const uint32_t* __restrict__ minbits, int rows, int n, int p, int a, int b, double* __restrict__ scores) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const long long row = (long long)blockIdx.x * kRankWaves + wave;
  if (row >= rows) return;
  const int self = (int)(row / p);
  const uint32_t* src = minbits + row * n;
  uint32_t key[kSlots];
#pragma unroll
  for (int i = 0; i < kSlots; ++i) {
    const int j = i * kWave + lane;
    key[i] = (j < n && j != self) ? key_bits(src[j]) : kNoKey;
  }
  auto below = [&](uint32_t t) {  // #{key < t} over the row, the same in every lane
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < kSlots; ++i) cnt += __popcll(__ballot(key[i] < t));
    return cnt;
  };
  uint32_t ta = 0, tb = 0;  // a-th and b-th smallest keys (ta stays 0 for a = 0)
#pragma unroll 1
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cb = tb | (1u << bit);
    if (below(cb) < b) tb = cb;
    if (a > 0) {
      const uint32_t ca = ta | (1u << bit);
      if (below(ca) < a) ta = ca;
    }
  }
  double sa = 0.0, sb = 0.0;
#pragma unroll
  for (int i = 0; i < kSlots; ++i) {
    const double r = (double)sqrtf(__uint_as_float(key[i]));
    if (key[i] < tb) sb += r;
    if (key[i] < ta) sa += r;
  }
  sb = wave_sum(sb);
  sa = wave_sum(sa);
  sb += (double)(b - below(tb)) * (double)sqrtf(__uint_as_float(tb));
  if (a > 0) sa += (double)(a - below(ta)) * (double)sqrtf(__uint_as_float(ta));
  // as in msm_rank_select_kernel: an infinite S(a) means a window of +inf (or NaN) keys
  const double win = isinf(sa) ? sb : sb - sa;
  if (lane == 0) scores[row] = (double)(float)(win / (double)(b - a));
}

__global__ __launch_bounds__(256) void msm_nearest_kernel(const uint32_t* __restrict__ minbits,
                                                          size_t count, int n, int p,
                                                          float* __restrict__ nearest) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
    const size_t row = i / n;
    const int j = (int)(i % n);
    nearest[i] = (j == (int)(row / p)) ? __int_as_float(kInfBits) : sqrtf(__uint_as_float(key_bits(minbits[i])));
  }
}

// ---------------------------------------------------------------------------
// Cancellation refinement.  The pair kernels form ||a||^2 + ||b||^2 - 2 a.b, whose
// rounding error is of the order of eps (||a||^2 + ||b||^2) whatever the distance, so
// a minimum near 0 (a duplicated image, near-duplicate patches) keeps only the square
// root of that error: a few 1e-4 in d for unit rows.  The reference's accelerated MSM
// recomputes every pair with d^2 <= 32 eps C (||q||^2 + ||r||^2) by explicit
// differences (models/modules/_MSM_gpu.py:219-228).  Here one pass over the minima
// keys flags each (row, image) minimum at or below max(32 C, 4096) eps (norms[row] +
// the largest norm of the image) -- the reference's bound with the image's largest
// norm, so every pair the reference recomputes lies in a flagged (row, image) or
// cannot be its minimum, and never below 4096 eps: the roundings of the two norms and
// of the final sum leave ~3 eps (||q||^2 + ||r||^2) in d^2 whatever C is, which 32 eps C
// does not cover for small C (at C = 3, minima just above it came out 2.2e-5 from the
// exact value); above 4096 eps (||q||^2 + ||r||^2) they move d by at most ~1e-5 at C = 3
// -- and the wave recomputes that minimum over all P patches of the image as
// sum_c (s_a a_c - s_b b_c)^2 in fp32 (s the row scales: 1 / ||z|| with row
// normalisation, else 1), accurate to a few ulps of d^2 itself; identical rows give
// exactly 0.  For C >= 128 the bound is the reference's.  A flagged minimum is replaced
// (stored), not merged: the exact value may lie above the expanded one.  NaN minima
// (key 0), the own image and +inf (key kMinFill) are left alone.  With nothing
// flagged the pass reads the keys once (37.7 MB at N = 83, P = 1369).
// ---------------------------------------------------------------------------
constexpr int kRefineRows = 16;                 // rows per wave
constexpr float kRefineEps = 1.192092896e-7f;   // the fp32 machine epsilon of the reference's bound
constexpr float kRefineFloor = 4096.f;          // smallest multiplier of eps (norm[q] + max norm[r])

// Minimum over rows q in [q0, q1) of sum_c (s_row z_row,c - s_q z_q,c)^2, in every lane.
// The products are rounded before the difference (no contraction), as the
// reference's normalised features are rounded before cdist, so identical rows give 0.
__device__ inline float exact_min_sq(const float* __restrict__ z, const float* __restrict__ scale, long long row,
                                     long long q0, long long q1, int c, int lane) {
#pragma clang fp contract(off)
  const float sa = scale[row];
  const float* a = z + row * (long long)c;
  float best = __int_as_float(kInfBits);
  for (long long q = q0; q < q1; q += 4) {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    float sb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) sb[j] = q + j < q1 ? scale[q + j] : 0.f;
    if ((c & 3) == 0) {
      for (int k = 4 * lane; k < c; k += 4 * kWave) {
        const float4 av = *reinterpret_cast<const float4*>(a + k);
        const float ax = av.x * sa, ay = av.y * sa, az = av.z * sa, aw = av.w * sa;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (q + j < q1) {
            const float4 bv = *reinterpret_cast<const float4*>(z + (q + j) * (long long)c + k);
            const float dx = ax - bv.x * sb[j], dy = ay - bv.y * sb[j];
            const float dz = az - bv.z * sb[j], dw = aw - bv.w * sb[j];
            acc[j] = fmaf(dx, dx, acc[j]);
            acc[j] = fmaf(dy, dy, acc[j]);
            acc[j] = fmaf(dz, dz, acc[j]);
            acc[j] = fmaf(dw, dw, acc[j]);
          }
        }
      }
    } else {
      for (int k = lane; k < c; k += kWave) {
        const float ax = a[k] * sa;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (q + j < q1) {
            const float d = ax - z[(q + j) * (long long)c + k] * sb[j];
            acc[j] = fmaf(d, d, acc[j]);
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float d2 = wave_sum(acc[j]);
      if (q + j < q1) best = nmin(best, d2);
    }
  }
  return best;
}

// One wave per kRefineRows consecutive rows: their keys are read with consecutive
// lanes on consecutive keys; a ballot collects the flagged ones, which the whole wave
// then recomputes one at a time.
__global__ __launch_bounds__(256) void msm_refine_kernel(const float* __restrict__ z, int rows, int n, int p, int c,
                                                         const float* __restrict__ norms,
                                                         const float* __restrict__ scale,
                                                         const uint32_t* __restrict__ imgmax,
                                                         uint32_t* __restrict__ minbits, float thr) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const long long row0 = ((long long)blockIdx.x * (blockDim.x / kWave) + wave) * kRefineRows;
  if (row0 >= rows) return;
  const int nk = (int)min((long long)kRefineRows, rows - row0) * n;  // <= 16 * 4096
  uint32_t* keys = minbits + row0 * n;
  for (int base = 0; base < nk; base += kWave) {
    const int i = base + lane;
    bool flag = false;
    if (i < nk) {
      const uint32_t key = keys[i];
      if (key != 0u && key < kMinFill) {
        const float d2 = __uint_as_float(key - 1u);
        flag = d2 <= thr * (norms[row0 + i / n] + __uint_as_float(imgmax[i % n]));
      }
    }
    unsigned long long mask = __ballot(flag);
    while (mask) {
      const int l = __ffsll((unsigned long long)mask) - 1;
      mask &= mask - 1;
      const int ii = base + l;
      const long long row = row0 + ii / n;
      const int img = ii % n;
      const long long q0 = (long long)img * p, q1 = min(q0 + p, (long long)rows);
      const float d2 = exact_min_sq(z, scale, row, q0, q1, c, lane);
      if (lane == 0) keys[ii] = min_key(d2);
    }
  }
}

// The workspace holds arrays read with 16-byte loads and merged with 4-byte atomics,
// each at a 256-byte-aligned offset from its start: the start must be 256-byte aligned.
inline bool ws_aligned(const void* ws) { return (reinterpret_cast<uintptr_t>(ws) & 255) == 0; }

inline int validate(const float* z, int n, int p, int c, void* ws, size_t ws_bytes) {
  if (!z || n < 2 || p < 1 || c < 1) return MUSC_ERR_INVALID_ARG;
  const long long rows = (long long)n * p;
  if (rows > (1LL << 30)) return MUSC_ERR_UNSUPPORTED;
  if (n > 4096) return MUSC_ERR_UNSUPPORTED;  // rank kernels hold a row's n keys in at most 64 slots per lane
  if (!ws || ws_bytes < workspace_bytes(n, p)) return MUSC_ERR_WORKSPACE;
  if (!ws_aligned(ws)) return MUSC_ERR_INVALID_ARG;
  if ((c & 3) == 0 && (reinterpret_cast<uintptr_t>(z) & 15) != 0) return MUSC_ERR_INVALID_ARG;
  return MUSC_OK;
}

// Stage 1: row norms and the +inf fill of the minima buffer.
inline void run_prepare(const float* z, int n, int p, int c, int normalize, const Workspace& w, hipStream_t s) {
  const long long rows = (long long)n * p;
  hipLaunchKernelGGL(msm_norms_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, z, (int)rows, c,
                     normalize, w.norms, w.inv, w.scale);
  launch_image_max(w.norms, n, p, w.imgmax, s);
  launch_fill_u32(w.minbits, (size_t)rows * n, kMinFill, s);
}

// Stage 3: exact minima where the expanded form cancels (either engine's keys).
int run_refine(const float* z, int n, int p, int c, const Workspace& w, hipStream_t s) {
  const long long rows = (long long)n * p;
  const long long blocks = ((rows + kRefineRows - 1) / kRefineRows + 3) / 4;
  hipLaunchKernelGGL(msm_refine_kernel, dim3((unsigned)blocks), dim3(256), 0, s, z, (int)rows, n, p, c, w.norms,
                     w.scale, w.imgmax, w.minbits, fmaxf(32.f * (float)c, kRefineFloor) * kRefineEps);
  return check_launch();
}

// Stage 4: trimmed rank means.
int run_rank(int n, int p, int a, int b, double* scores, const Workspace& w, hipStream_t s) {
  const long long rows = (long long)n * p;
  if (n <= kMaxSelectKeys && b <= 32) {
    const dim3 grid((unsigned)((rows + kRank2Rows - 1) / kRank2Rows)), block(kWave);
    const size_t smem = (size_t)kRank2Rows * n * sizeof(uint32_t);  // <= 24 KB
#define MUSC_RANK_INSERT(K) \
  hipLaunchKernelGGL(msm_rank_insert2_kernel<K>, grid, block, smem, s, w.minbits, (int)rows, n, p, a, b, scores)
    if (b <= 8) MUSC_RANK_INSERT(8);
    else if (b <= 16) MUSC_RANK_INSERT(16);
    else if (b <= 24) MUSC_RANK_INSERT(24);
    else MUSC_RANK_INSERT(32);
#undef MUSC_RANK_INSERT
    return check_launch();
  }
  if (n <= kMaxSelectKeys) {
    const dim3 grid((unsigned)((rows + kRankRows - 1) / kRankRows)), block(kRankRows);
    const size_t smem = 0;  // the chunk buffer is static
#define MUSC_RANK_LAUNCH(K) \
  hipLaunchKernelGGL(msm_rank_select_kernel<K>, grid, block, smem, s, w.minbits, (int)rows, n, p, a, b, scores)
    if (n <= 32) MUSC_RANK_LAUNCH(32);
    else if (n <= 64) MUSC_RANK_LAUNCH(64);
    else if (n <= 96) MUSC_RANK_LAUNCH(96);
    else if (n <= 128) MUSC_RANK_LAUNCH(128);
    else if (n <= 160) MUSC_RANK_LAUNCH(160);
    else MUSC_RANK_LAUNCH(192);
#undef MUSC_RANK_LAUNCH
    return check_launch();
  }
  const dim3 grid((unsigned)((rows + kRankWaves - 1) / kRankWaves)), block(kRankWaves * kWave);
#define MUSC_RANK_WAVE(K) \
  hipLaunchKernelGGL(msm_rank_wave_kernel<K>, grid, block, 0, s, w.minbits, (int)rows, n, p, a, b, scores)
  if (n <= 256) MUSC_RANK_WAVE(4);
  else if (n <= 512) MUSC_RANK_WAVE(8);
  else if (n <= 1024) MUSC_RANK_WAVE(16);
  else if (n <= 2048) MUSC_RANK_WAVE(32);
  else MUSC_RANK_WAVE(64);  // n <= 4096 (validate)
#undef MUSC_RANK_WAVE
  return check_launch();
}

}  // namespace msm
}  // namespace musc

using namespace musc;

extern "C" int musc_msm_workspace_bytes(int n, int p, int c, size_t* out) {
  if (!out || n < 2 || p < 1 || c < 1) return MUSC_ERR_INVALID_ARG;
  *out = msm::workspace_bytes(n, p);
  return MUSC_OK;
}

extern "C" int musc_msm_prepare_f32(const float* z, int n, int p, int c, int flags, void* workspace,
                                    size_t workspace_bytes, hipStream_t stream) {
  int rc = msm::validate(z, n, p, c, workspace, workspace_bytes);
  if (rc) return rc;
  if (flags & ~MUSC_MSM_NORMALIZE_ROWS) return MUSC_ERR_INVALID_ARG;
  msm::run_prepare(z, n, p, c, (flags & MUSC_MSM_NORMALIZE_ROWS) ? 1 : 0, msm::carve(workspace, n, p), stream);
  return check_launch();
}

extern "C" int musc_msm_pair_minima_f32(const float* z, int n, int p, int c, void* workspace,
                                        size_t workspace_bytes, hipStream_t stream) {
  int rc = msm::validate(z, n, p, c, workspace, workspace_bytes);
  if (rc) return rc;
  return msm::run_pairs(z, n, p, c, msm::carve(workspace, n, p), stream);
}

extern "C" int musc_msm_refine_f32(const float* z, int n, int p, int c, void* workspace, size_t workspace_bytes,
                                   hipStream_t stream) {
  int rc = msm::validate(z, n, p, c, workspace, workspace_bytes);
  if (rc) return rc;
  return msm::run_refine(z, n, p, c, msm::carve(workspace, n, p), stream);
}

extern "C" int musc_msm_rank_f32(int n, int p, int rank_lo, int rank_hi, double* scores, void* workspace,
                                 size_t workspace_bytes, hipStream_t stream) {
  if (!scores || n < 2 || p < 1 || rank_lo < 0 || rank_lo >= rank_hi || rank_hi > n - 1) return MUSC_ERR_INVALID_ARG;
  if (n > 4096 || (long long)n * p > (1LL << 30)) return MUSC_ERR_UNSUPPORTED;
  if (!workspace || workspace_bytes < msm::workspace_bytes(n, p)) return MUSC_ERR_WORKSPACE;
  if (!msm::ws_aligned(workspace)) return MUSC_ERR_INVALID_ARG;
  return msm::run_rank(n, p, rank_lo, rank_hi, scores, msm::carve(workspace, n, p), stream);
}

extern "C" int musc_msm_scores_f32(const float* z, int n, int p, int c, int rank_lo, int rank_hi,
                                   double* scores, void* workspace, size_t workspace_bytes,
                                   hipStream_t stream) {
  int rc = msm::validate(z, n, p, c, workspace, workspace_bytes);
  if (rc) return rc;
  if (!scores || rank_lo < 0 || rank_lo >= rank_hi || rank_hi > n - 1) return MUSC_ERR_INVALID_ARG;
  const msm::Workspace w = msm::carve(workspace, n, p);
  msm::run_prepare(z, n, p, c, 0, w, stream);
  rc = msm::run_pairs(z, n, p, c, w, stream);
  if (rc) return rc;
  rc = msm::run_refine(z, n, p, c, w, stream);
  if (rc) return rc;
  return msm::run_rank(n, p, rank_lo, rank_hi, scores, w, stream);
}

// ---------------------------------------------------------------------------
// Scores without allocation: the workspace of musc_msm_scores_f32 lives in a
// file-scope device array (one per GPU, for the life of the process), for callers
// that cannot allocate.  Host code never passes the array's name to a kernel: its
// device address comes from hipGetSymbolAddress, once per device.
// ---------------------------------------------------------------------------
namespace {

constexpr size_t kScratchBytes = size_t(256) << 20;  // MUSC_NOALLOC_SCRATCH_BYTES
static_assert(kScratchBytes == MUSC_NOALLOC_SCRATCH_BYTES, "header and library disagree on the scratch size");
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices];  // device address of `scratch` per device, set on first use

// Device address of the current device's scratch array.
int current_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxScratchDevices) return MUSC_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return static_cast<int>(e);
    if (!ptr) return MUSC_ERR_UNSUPPORTED;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MUSC_OK;
}

}  // namespace

extern "C" int musc_msm_scores_f32_noalloc(const float* z, int n, int p, int c, int rank_lo, int rank_hi,
                                           double* scores, hipStream_t stream) {
  if (!z || n < 2 || p < 1 || c < 1) return MUSC_ERR_INVALID_ARG;
  if ((long long)n * p > (1LL << 30) || n > 4096) return MUSC_ERR_UNSUPPORTED;
  if (msm::workspace_bytes(n, p) > kScratchBytes) return MUSC_ERR_SCRATCH_LIMIT;
  void* ws = nullptr;
  const int rc = current_scratch(&ws);
  if (rc) return rc;
  // every array of the workspace is rewritten by every call (prepare); nothing carries over
  return musc_msm_scores_f32(z, n, p, c, rank_lo, rank_hi, scores, ws, kScratchBytes, stream);
}

extern "C" int musc_msm_nearest_f32(const float* z, int n, int p, int c, float* nearest, void* workspace,
                                    size_t workspace_bytes, hipStream_t stream) {
  int rc = msm::validate(z, n, p, c, workspace, workspace_bytes);
  if (rc) return rc;
  if (!nearest) return MUSC_ERR_INVALID_ARG;
  const msm::Workspace w = msm::carve(workspace, n, p);
  msm::run_prepare(z, n, p, c, 0, w, stream);
  rc = msm::run_pairs(z, n, p, c, w, stream);
  if (rc) return rc;
  rc = msm::run_refine(z, n, p, c, w, stream);
  if (rc) return rc;
  const size_t count = (size_t)n * p * n;
  const size_t blocks = (count + 255) / 256 < 65536 ? (count + 255) / 256 : 65536;  // grid-stride beyond
  hipLaunchKernelGGL(msm::msm_nearest_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, w.minbits, count, n, p,
                     nearest);
  return check_launch();
}
