// MSM pair minima with fp32-accurate dot products formed on the fp16 matrix cores.
//
// Same contract as msm_pair_min_kernel (msm.hip), i.e. models/modules/_MSM.py:10-30:
// per (patch, other image) the minimum squared distance ||a||^2 + ||b||^2 - 2 a.b,
// clamped at 0, NaN-propagating, merged with atomicMin on min_key (msm_common.hpp);
// the trimmed rank means are shared with the fp32 engine.  Only the dot products are
// formed differently.  One difference at the edge: a row holding +-inf (possible only
// without row normalisation; models/musc.py:238 turns such a row into NaN) has NaN
// distances to every row here, where the expanded form of the fp32 engine and of
// torch.cdist gives +inf for the pairs in which the infinite term adds to +inf.
//
// Split (Ootomo & Yokota, "Recovering single precision accuracy from Tensor Cores
// while surpassing the FP32 theoretical peak performance", IJHPCA 2022, restated for
// fp16 MFMA): every row is L2-normalised and scaled by 2^kScaleShift (so its entries
// lie in fp16's normal range), then split as v = hi + lo with hi = fp16(v) and
// lo = fp16(v - hi).  a.b is accumulated in fp32 as hi_a.hi_b + hi_a.lo_b + lo_a.hi_b;
// the dropped lo_a.lo_b term and the rounding of lo are below 2^-22 |a||b|, the
// order of fp32's own accumulation error, and a per-row scale restores the units.
// v_mfma_f32_32x32x16_f16 runs 16x the fp32 MFMA rate, so the three products cost
// 3/16 of one fp32 product.
//
// MI355X layout
//   split array   per row, per 16-channel block: hi[16] | lo[16] fp16 (64 bytes, one
//                 row's share of a pipeline stage); channels padded to a multiple of
//                 16 with zeros.
//   pair kernel   256 x 256 tiles of the upper triangle (symmetric reuse, bands of
//                 8 tile rows, XCD-grouped); a workgroup takes one 128-row half, two
//                 workgroups share a CU, 4 waves each own 64 x 128.  Stages of 16
//                 channels go straight from global memory into LDS
//                 (buffer_load_dwordx4 ... lds: lane l of a load lands at base + 16 l,
//                 so one load fills 16 rows of 64 bytes) through a 3-deep ring, loads
//                 2 stages ahead of the MFMAs, one barrier per stage, no staging
//                 registers.  The 16-byte segment s of staged row r sits at position
//                 s ^ ((r >> 2) & 3), which keeps the MFMA operand reads free of bank
//                 conflicts.
//                 Register epilogues as in the fp32 kernel (one image segment per
//                 dimension, or two when the tile straddles an image boundary:
//                 p >= 256 is required).
#include <hip/hip_fp16.h>

#include "msm_common.hpp"

namespace musc {
namespace msm {
namespace split {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));

constexpr int TM = 256;                      // triangle tile: rows = columns
constexpr int TR = 128;                      // tile rows per workgroup (half a triangle tile)
constexpr int TC = 256;                      // tile columns per workgroup
constexpr int KB = 16;                       // channels per stage (each of hi and lo)
constexpr int ROWB = 4 * KB;                 // bytes per row and stage: hi[16] lo[16] fp16
constexpr int NSTAGE = 3;                    // LDS ring depth: loads run NSTAGE - 1 stages ahead
constexpr int THREADS = 256;                 // 4 waves: 2 (rows) x 2 (columns) of 64 x 128
constexpr int kStageRows = TR + TC;          // A rows then B rows
constexpr int kStageBytes = kStageRows * ROWB;  // 24 KB
constexpr int kScaleShift = 10;              // normalised rows are scaled by 2^10
constexpr int kBandSplit = BAND;             // tile rows per band of the triangle enumeration
constexpr int kRowsPerLoad = kWave * 16 / ROWB;                          // 16 staged rows per direct load
constexpr int kLoads = kStageRows / kRowsPerLoad / (THREADS / kWave);    // direct loads per wave per stage

static_assert(kLoads == 6, "stage loads: 384 rows, 16 per load, over 4 waves (the vmcnt(6) of the main loop)");
static_assert(NSTAGE == 3, "the vmcnt waits of the main loop are written for a 3-deep ring");
static_assert(THREADS == TC && TR <= THREADS, "the prologue and the final merge map thread t to column t");

typedef __attribute__((address_space(3))) void lds_void;
typedef int int4v __attribute__((ext_vector_type(4)));
constexpr int kBufferFlags = 0x00020000;     // buffer resource word 3 for raw byte-addressed loads

// ---------------------------------------------------------------------------
// Prepare: one wave per row.  norms[], scale[] and the image maxima exactly as
// msm_norms_kernel; inv[] holds the epilogue's per-row scale of the split dot product.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void split_prepare_kernel(const float* __restrict__ z, int rows, int c, int nkb,
                                                            int normalize, float* __restrict__ norms,
                                                            float* __restrict__ inv, float* __restrict__ scale,
                                                            _Float16* __restrict__ hl) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const long long row = (long long)blockIdx.x * (blockDim.x / kWave) + wave;
  if (row >= rows) return;
  const float* src = z + row * (long long)c;
  const double acc = row_sumsq(src, c, lane);
  const double unit = ldexp(1.0, -kScaleShift);
  if (lane == 0) {
    float nrm;
    if (normalize) {
      const double r = 1.0 / sqrt(acc);
      nrm = (float)(acc * r * r);
      inv[row] = (float)unit;
      scale[row] = (float)r;
    } else {
      nrm = (float)acc;
      inv[row] = (float)(sqrt(acc) * unit);
      scale[row] = 1.f;
    }
    norms[row] = nrm;
  }
  const double sc = acc > 0.0 ? ldexp(1.0 / sqrt(acc), kScaleShift) : 0.0;
  _Float16* dst = hl + row * (long long)nkb * (2 * KB);
  const int cp = nkb * KB;
  auto split1 = [&](float x, _Float16& hi, _Float16& lo) {
    const double v = (double)x * sc;
    hi = (_Float16)(float)v;
    lo = (_Float16)(float)(v - (double)(float)hi);
  };
  if ((c & 7) == 0) {
    // eight channels per lane: one 16-byte store of hi and one of lo (half a
    // 16-channel block each); c % 8 == 0 keeps every group inside one block
    for (int k0 = 8 * lane; k0 < cp; k0 += 8 * kWave) {
      half8 hi, lo;
      if (k0 < c) {
        const float4 x0 = *reinterpret_cast<const float4*>(src + k0);
        const float4 x1 = *reinterpret_cast<const float4*>(src + k0 + 4);
        const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          _Float16 h, l;
          split1(xs[j], h, l);
          hi[j] = h;
          lo[j] = l;
        }
      } else {
        hi = half8{};
        lo = half8{};
      }
      _Float16* blk = dst + (k0 / KB) * (2 * KB) + (k0 % KB);
      *reinterpret_cast<half8*>(blk) = hi;
      *reinterpret_cast<half8*>(blk + KB) = lo;
    }
  } else {
    for (int k = lane; k < cp; k += kWave) {
      _Float16 hi = (_Float16)0.f, lo = (_Float16)0.f;
      if (k < c) split1(src[k], hi, lo);
      dst[(k / KB) * (2 * KB) + (k % KB)] = hi;
      dst[(k / KB) * (2 * KB) + KB + (k % KB)] = lo;
    }
  }
}

// ---------------------------------------------------------------------------
// Pair minima.  Workgroup w takes half (w & 1) -- 128 rows x all 256 columns -- of
// triangle tile (w >> 1); two workgroups share a CU, so one's barrier and LDS-read
// bubbles are covered by the other's MFMAs.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(THREADS, 2) void split_pair_kernel(const _Float16* __restrict__ hl,
                                                               const float* __restrict__ norms,
                                                               const float* __restrict__ inv,
                                                               uint32_t* __restrict__ minbits, int rows, int n, int p,
                                                               int nkb, int T, long long ntiles) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[NSTAGE * kStageBytes];
  __shared__ __attribute__((aligned(16))) float s_rnorm[TR];
  __shared__ __attribute__((aligned(16))) float s_rinv[TR];
  __shared__ __attribute__((aligned(16))) int s_rimg[TR];
  __shared__ float s_cnorm[TC];
  __shared__ float s_cinv[TC];
  __shared__ int s_cimg[TC];

  const long long w = xcd_logical_id(blockIdx.x, gridDim.x);
  if (w >= 2 * ntiles) return;
  const int2 tile = decode_tile<kBandSplit>(w >> 1, T);
  const int row0 = tile.x * TM + (int)(w & 1) * TR, col0 = tile.y * TM;
  if (row0 >= rows) return;  // lower half of a last tile row that lies in padding
  const int rlast = min(row0 + TR, rows) - 1, clast = min(col0 + TC, rows) - 1;
  const int rimg0 = row0 / p, cimg0 = col0 / p;
  const bool simple = (row0 + TR <= rows) && (col0 + TC <= rows) && (rlast / p == rimg0) && (clast / p == cimg0);
  if (simple && rimg0 == cimg0) return;

  const int t = threadIdx.x;  // THREADS == TC: thread t stages column t and, for t < TR, row t
  {
    const int cc = col0 + t;
    s_cnorm[t] = cc < rows ? norms[cc] : 0.f;
    s_cinv[t] = cc < rows ? inv[cc] : 0.f;
    s_cimg[t] = cc < rows ? cc / p : n;  // n marks "no image" (padding)
    if (t < TR) {
      const int r = row0 + t;
      s_rnorm[t] = r < rows ? norms[r] : 0.f;
      s_rinv[t] = r < rows ? -2.f * inv[r] : 0.f;  // -2 x row scale (exact)
      s_rimg[t] = r < rows ? r / p : n;
    }
  }

  const int wave = t / kWave, lane = t % kWave;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lh = lane >> 5;

  floatx16 acc[2][4];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.f;

  // Loads go straight from global memory into LDS (buffer_load_dwordx4 ... lds: lane
  // l of a load lands at M0 + 16 l, so one load fills 16 staged rows of 64 bytes).
  // Wave wv fills staged rows wv*96 .. wv*96 + 95; staged rows 0..127 are tile rows
  // (A), 128..383 tile columns (B).  Lane l of a load carries row R = R0 + l/4 into
  // LDS position l % 4, i.e. segment (l % 4) ^ ((R >> 2) & 3).  Padded rows re-read
  // the last row (masked in the epilogue).
  // Addressing: two buffer resources, one based at the first row of the A panel and
  // one at the first row of the B panel (64-bit bases, so the split array may have any
  // size; each extent ends with its panel's last row), one 32-bit byte offset per load
  // within its panel (row + segment, loop-invariant) and the stage offset as the scalar
  // offset.  A load's 16 staged rows lie all in A or all in B (128 = 8 loads of 16
  // rows), so each load names one resource.  The loads are issued from inline
  // assembly so that the compiler, which cannot tell the ring buffers apart, does
  // not wait for them before reading another buffer; the loop waits for them
  // explicitly.
  const int lrow = lane >> 2;
  auto panel_rsrc = [&](int first, int last) {
    const unsigned long long addr =
        reinterpret_cast<unsigned long long>(hl) + (unsigned long long)first * (unsigned long long)(nkb * ROWB);
    int4v r;
    r.x = (int)(uint32_t)(addr & 0xffffffffull);
    r.y = (int)(uint32_t)(addr >> 32);  // base high bits; stride 0
    r.z = (int)((uint32_t)(last - first + 1) * (uint32_t)(nkb * ROWB));
    r.w = kBufferFlags;
    return r;
  };
  const int4v rsrcA = panel_rsrc(row0, rlast), rsrcB = panel_rsrc(col0, clast);
  constexpr int kWaveRows = kStageRows / (THREADS / kWave);
  static_assert(TR % kRowsPerLoad == 0, "a load's staged rows lie in one panel");
  uint32_t voff[kLoads];
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const int R = wave * kWaveRows + i * kRowsPerLoad + lrow;
    const int prow = R < TR ? min(R, rlast - row0) : min(R - TR, clast - col0);
    const int lseg = (lane & 3) ^ ((R >> 2) & 3);
    voff[i] = (uint32_t)prow * (uint32_t)(nkb * ROWB) + (uint32_t)(lseg * 16);
  }
  const uint32_t lds0 = (uint32_t)(size_t)(lds_void*)smem;
  auto issue = [&](int kb, int buf) {
    const uint32_t soff = (uint32_t)(kb * ROWB);
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      // wave-uniform LDS base of this load (M0 is a scalar register)
      const uint32_t m0 = __builtin_amdgcn_readfirstlane(
          lds0 + (uint32_t)(buf * kStageBytes + (wave * kWaveRows + i * kRowsPerLoad) * ROWB));
      // s_nop: one wait state between the scalar write of M0 and the load that reads it
      const bool inA = __builtin_amdgcn_readfirstlane(wave * kWaveRows + i * kRowsPerLoad) < TR;  // wave-uniform
      asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                   :
                   : "s"(m0), "v"(voff[i]), "s"(inA ? rsrcA : rsrcB), "s"(soff)
                   : "memory", "m0");
    }
  };
  // Segments of a staged row: 0, 1 = hi channels 0-7, 8-15; 2, 3 = lo.  Segment s of
  // staged row r sits at position s ^ ((r >> 2) & 3); the operand rows here are
  // (multiple of 32) + lr, so the swizzle is (lr >> 2) & 3.  Over any 16 consecutive
  // rows (the lanes an LDS read serves together) the pairs (r & 3, (r >> 2) & 3) take
  // 16 distinct 16-byte slots of a 256-byte bank window: conflict-free reads.
  const int sw = (lr >> 2) & 3;
  const int phi = (lh ^ sw) * 16, plo = ((2 + lh) ^ sw) * 16;
  auto compute = [&](int buf) {
    const unsigned char* As = smem + buf * kStageBytes + (wm * 64 + lr) * ROWB;
    const unsigned char* Bs = smem + buf * kStageBytes + (TR + wn * 128 + lr) * ROWB;
    half8 ahi[2], alo[2], bhi[4], blo[4];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      ahi[mb] = *reinterpret_cast<const half8*>(As + mb * 32 * ROWB + phi);
      alo[mb] = *reinterpret_cast<const half8*>(As + mb * 32 * ROWB + plo);
    }
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      bhi[nb] = *reinterpret_cast<const half8*>(Bs + nb * 32 * ROWB + phi);
      blo[nb] = *reinterpret_cast<const half8*>(Bs + nb * 32 * ROWB + plo);
    }
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ahi[mb], bhi[nb], acc[mb][nb], 0, 0, 0);
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ahi[mb], blo[nb], acc[mb][nb], 0, 0, 0);
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(alo[mb], bhi[nb], acc[mb][nb], 0, 0, 0);
  };

  // Stage kc lives in LDS buffer kc % NSTAGE and its loads go out NSTAGE - 1 stages
  // ahead.  Iteration kc waits until this thread's loads of stage kc have landed
  // (loads complete in order, so only the next stage's kLoads may still be in
  // flight); the barrier then makes every wave's loads visible and guarantees that
  // buffer (kc - 1) % NSTAGE is no longer read (compute(kc - 1) is done everywhere),
  // so the loads of stage kc + NSTAGE - 1 can refill it.
  for (int st = 0; st < NSTAGE - 1 && st < nkb; ++st) issue(st, st);
  for (int kc = 0; kc < nkb; ++kc) {
    if (kc + 1 < nkb)
      asm volatile("s_waitcnt vmcnt(6)" ::: "memory");  // the next stage's kLoads may be in flight
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (kc + NSTAGE - 1 < nkb) issue(kc + NSTAGE - 1, (kc + NSTAGE - 1) % NSTAGE);
    compute(kc % NSTAGE);
  }

  // Epilogue.  Lane (lr, lh) of wave (wm, wn) holds, for mb < 2, nb < 4, v < 16, the
  // dot of tile row wm*64 + mb*32 + (v/4)*8 + lh*4 + v%4 with tile column
  // wn*128 + nb*32 + lr.
  const float inf = __int_as_float(kInfBits);
  const int rA = rimg0, cA = cimg0;
  float d2[2][4][16];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int i0 = wm * 64 + mb * 32 + g * 8 + lh * 4;
      const float4 rn = *reinterpret_cast<const float4*>(&s_rnorm[i0]);
      const float4 ri = *reinterpret_cast<const float4*>(&s_rinv[i0]);
      const float rv[4] = {rn.x, rn.y, rn.z, rn.w};
      const float rs[4] = {ri.x, ri.y, ri.z, ri.w};
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const int j = wn * 128 + nb * 32 + lr;
        const float cn = s_cnorm[j];
        const float ci = s_cinv[j];
#pragma unroll
        for (int e = 0; e < 4; ++e)  // clamped at 0 by min_key, after the minima
          d2[mb][nb][g * 4 + e] = fmaf(rs[e] * ci, acc[mb][nb][g * 4 + e], rv[e] + cn);
      }
    }

  if (simple) {
    // column minima over this wave's 64 rows; the two lane halves then split the
    // column blocks: half lh keeps blocks 2q + lh (q = 0, 1)
    float cmin[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      float m = d2[0][nb][0];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int v = 0; v < 16; ++v) m = nmin(m, d2[mb][nb][v]);
      cmin[nb] = m;
    }
    float cm[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) cm[q] = halves_min2(cmin[2 * q], cmin[2 * q + 1]);
    // row minima over this wave's 128 columns: in-lane over nb, then the transposing
    // butterfly over the 32 lanes of each half
    float rv[32];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        rv[mb * 16 + v] = nmin(nmin(d2[mb][0][v], d2[mb][1][v]), nmin(d2[mb][2][v], d2[mb][3][v]));
    transpose_min32(rv, lr);
    __syncthreads();  // operand buffers are no longer read
    float* s_cmin = reinterpret_cast<float*>(smem);  // [2 (wm)][TC]
    float* s_rmin = s_cmin + 2 * TC;                  // [2 (wn)][TR]
#pragma unroll
    for (int q = 0; q < 2; ++q) s_cmin[wm * TC + wn * 128 + (2 * q + lh) * 32 + lr] = cm[q];
    s_rmin[wn * TR + wm * 64 + transposed_row(lr, lh)] = rv[0];
    __syncthreads();
    atomicMin(minbits + (long long)(col0 + t) * n + rA, min_key(nmin(s_cmin[t], s_cmin[TC + t])));
    if (t < TR)
      atomicMin(minbits + (long long)(row0 + t) * n + cA, min_key(nmin(s_rmin[t], s_rmin[TR + t])));
    return;
  }

  // Two image segments per dimension (P >= 256: one boundary at most per tile
  // dimension).  Tile rows [0, rsplit) are image rA, the rest image rA + 1 or padding;
  // columns likewise with csplit and cA.  Whether a pair is masked (same image, or
  // padding) depends only on the two segments, so minima are taken per segment over
  // the raw distances and a masked segment pair becomes +inf afterwards; a wave whose
  // rows (or columns) lie in one segment reduces them without per-distance selects.
  const int rsplit = min(TR, min((rA + 1) * p, rows) - row0);
  const int csplit = min(TC, min((cA + 1) * p, rows) - col0);
  const int rBimg = row0 + rsplit < rows ? rA + 1 : n;  // used only when segment B is not empty
  const int cBimg = col0 + csplit < rows ? cA + 1 : n;
  const bool mAA = rA == cA, mAB = cBimg == n || rA == cBimg;
  const bool mBA = rBimg == n || rBimg == cA, mBB = rBimg == n || cBimg == n || rBimg == cBimg;
  const int wr0 = wm * 64, wc0 = wn * 128;
  float cminA[4], cminB[4];
  if (rsplit >= wr0 + 64 || rsplit <= wr0) {
    const bool inA = rsplit > wr0;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      float m = d2[0][nb][0];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int v = 0; v < 16; ++v) m = nmin(m, d2[mb][nb][v]);
      cminA[nb] = inA ? m : inf;
      cminB[nb] = inA ? inf : m;
    }
  } else {
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      float a = inf, b = inf;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const bool inB = wr0 + mb * 32 + (v >> 2) * 8 + lh * 4 + (v & 3) >= rsplit;
          a = nmin(a, inB ? inf : d2[mb][nb][v]);
          b = nmin(b, inB ? d2[mb][nb][v] : inf);
        }
      cminA[nb] = a;
      cminB[nb] = b;
    }
  }
  float cmA[2], cmB[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    cmA[q] = halves_min2(cminA[2 * q], cminA[2 * q + 1]);  // column wc0 + (2q + lh) * 32 + lr
    cmB[q] = halves_min2(cminB[2 * q], cminB[2 * q + 1]);
    const bool colInB = wc0 + (2 * q + lh) * 32 + lr >= csplit;
    if (colInB ? mAB : mAA) cmA[q] = inf;
    if (colInB ? mBB : mBA) cmB[q] = inf;
  }
  float rowminA, rowminB;
  if (csplit >= wc0 + 128 || csplit <= wc0) {
    float rv[32];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        rv[mb * 16 + v] = nmin(nmin(d2[mb][0][v], d2[mb][1][v]), nmin(d2[mb][2][v], d2[mb][3][v]));
    const float m = transpose_min32(rv, lr);
    const bool inA = csplit > wc0;
    rowminA = inA ? m : inf;
    rowminB = inA ? inf : m;
  } else {
    bool colB[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) colB[nb] = wc0 + nb * 32 + lr >= csplit;
    {
      float rv[32];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          float m = inf;
#pragma unroll
          for (int nb = 0; nb < 4; ++nb) m = nmin(m, colB[nb] ? inf : d2[mb][nb][v]);
          rv[mb * 16 + v] = m;
        }
      rowminA = transpose_min32(rv, lr);
    }
    {
      float rv[32];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          float m = inf;
#pragma unroll
          for (int nb = 0; nb < 4; ++nb) m = nmin(m, colB[nb] ? d2[mb][nb][v] : inf);
          rv[mb * 16 + v] = m;
        }
      rowminB = transpose_min32(rv, lr);
    }
  }
  const int rk = wm * 64 + transposed_row(lr, lh);
  {
    const bool rowInB = rk >= rsplit;
    if (rowInB ? mBA : mAA) rowminA = inf;
    if (rowInB ? mBB : mAB) rowminB = inf;
  }
  __syncthreads();  // operand buffers are no longer read
  float* s_cminA = reinterpret_cast<float*>(smem);  // [2 (wm)][TC]
  float* s_cminB = s_cminA + 2 * TC;
  float* s_rminA = s_cminB + 2 * TC;                 // [2 (wn)][TR]
  float* s_rminB = s_rminA + 2 * TR;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    s_cminA[wm * TC + wn * 128 + (2 * q + lh) * 32 + lr] = cmA[q];
    s_cminB[wm * TC + wn * 128 + (2 * q + lh) * 32 + lr] = cmB[q];
  }
  s_rminA[wn * TR + rk] = rowminA;
  s_rminB[wn * TR + rk] = rowminB;
  __syncthreads();
  {
    const int cc = col0 + t;
    if (cc < rows) {
      // a segment with no pair of different images is exactly +inf (masked): skip it,
      // also because segment B may be the padding image n
      const float a = nmin(s_cminA[t], s_cminA[TC + t]);
      const float b = nmin(s_cminB[t], s_cminB[TC + t]);
      if (a != inf) atomicMin(minbits + (long long)cc * n + rA, min_key(a));
      if (b != inf) atomicMin(minbits + (long long)cc * n + rA + 1, min_key(b));
    }
  }
  if (t < TR) {
    const int r = row0 + t;
    if (r < rows) {
      const float a = nmin(s_rminA[t], s_rminA[TR + t]);
      const float b = nmin(s_rminB[t], s_rminB[TR + t]);
      if (a != inf) atomicMin(minbits + (long long)r * n + cA, min_key(a));
      if (b != inf) atomicMin(minbits + (long long)r * n + cA + 1, min_key(b));
    }
  }
}

inline int nkb_of(int c) { return (c + KB - 1) / KB; }

inline size_t split_array_bytes(long long rows, int c) { return align_up((size_t)rows * nkb_of(c) * ROWB, 256); }

inline size_t workspace_bytes(long long n, long long p, int c) {
  return msm::workspace_bytes(n, p) + split_array_bytes(n * p, c);
}

inline _Float16* split_array(void* ws, long long n, long long p) {
  return reinterpret_cast<_Float16*>(static_cast<char*>(ws) + msm::workspace_bytes(n, p));
}

inline int validate(int n, int p, int c, void* ws, size_t ws_bytes) {
  if (n < 2 || p < 1 || c < 1) return MUSC_ERR_INVALID_ARG;
  const long long rows = (long long)n * p;
  if (rows > (1LL << 30) || n > 4096) return MUSC_ERR_UNSUPPORTED;
  // 32-bit offsets within a 256-row panel (the buffer resources are based at each tile's panels)
  if ((long long)TC * nkb_of(c) * ROWB > 0x7fffffffLL) return MUSC_ERR_UNSUPPORTED;
  if (!ws || ws_bytes < workspace_bytes(n, p, c)) return MUSC_ERR_WORKSPACE;
  if ((reinterpret_cast<uintptr_t>(ws) & 255) != 0) return MUSC_ERR_INVALID_ARG;
  return MUSC_OK;
}

inline void run_prepare(const float* z, int n, int p, int c, int normalize, void* ws, hipStream_t s) {
  const long long rows = (long long)n * p;
  const Workspace w = carve(ws, n, p);
  hipLaunchKernelGGL(split_prepare_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, z, (int)rows, c,
                     nkb_of(c), normalize, w.norms, w.inv, w.scale, split_array(ws, n, p));
  launch_image_max(w.norms, n, p, w.imgmax, s);
  launch_fill_u32(w.minbits, (size_t)rows * n, kMinFill, s);
}

inline int run_pairs(int n, int p, int c, void* ws, hipStream_t s) {
  if (p < TM) return MUSC_ERR_UNSUPPORTED;  // the two-segment epilogue needs p >= 256
  const long long rows = (long long)n * p;
  const long long T = (rows + TM - 1) / TM;
  const long long ntiles = total_tiles(T);
  const long long grid = (2 * ntiles + kXcds - 1) / kXcds * kXcds;  // two half-tile workgroups per tile
  if (grid > 0x7fffffffLL) return MUSC_ERR_UNSUPPORTED;
  const Workspace w = carve(ws, n, p);
  hipLaunchKernelGGL(split_pair_kernel, dim3((unsigned)grid), dim3(THREADS), 0, s, split_array(ws, n, p), w.norms,
                     w.inv, w.minbits, (int)rows, n, p, nkb_of(c), (int)T, ntiles);
  return check_launch();
}

}  // namespace split
}  // namespace msm
}  // namespace musc

using namespace musc;

extern "C" int musc_msm_split_workspace_bytes(int n, int p, int c, size_t* out) {
  if (!out || n < 2 || p < 1 || c < 1) return MUSC_ERR_INVALID_ARG;
  *out = msm::split::workspace_bytes(n, p, c);
  return MUSC_OK;
}

extern "C" int musc_msm_split_prepare_f32(const float* z, int n, int p, int c, int flags, void* workspace,
                                          size_t workspace_bytes, hipStream_t stream) {
  int rc = msm::split::validate(n, p, c, workspace, workspace_bytes);
  if (rc) return rc;
  if (!z || (flags & ~MUSC_MSM_NORMALIZE_ROWS)) return MUSC_ERR_INVALID_ARG;
  if ((c & 3) == 0 && (reinterpret_cast<uintptr_t>(z) & 15) != 0) return MUSC_ERR_INVALID_ARG;
  msm::split::run_prepare(z, n, p, c, (flags & MUSC_MSM_NORMALIZE_ROWS) ? 1 : 0, workspace, stream);
  return check_launch();
}

extern "C" int musc_msm_split_pair_minima(int n, int p, int c, void* workspace, size_t workspace_bytes,
                                          hipStream_t stream) {
  int rc = msm::split::validate(n, p, c, workspace, workspace_bytes);
  if (rc) return rc;
  return msm::split::run_pairs(n, p, c, workspace, stream);
}

extern "C" int musc_msm_split_scores_f32(const float* z, int n, int p, int c, int rank_lo, int rank_hi, int flags,
                                         double* scores, void* workspace, size_t workspace_bytes,
                                         hipStream_t stream) {
  int rc = msm::split::validate(n, p, c, workspace, workspace_bytes);
  if (rc) return rc;
  if (!z || !scores || rank_lo < 0 || rank_lo >= rank_hi || rank_hi > n - 1) return MUSC_ERR_INVALID_ARG;
  if (flags & ~MUSC_MSM_NORMALIZE_ROWS) return MUSC_ERR_INVALID_ARG;
  if ((c & 3) == 0 && (reinterpret_cast<uintptr_t>(z) & 15) != 0) return MUSC_ERR_INVALID_ARG;
  if (p < msm::split::TM) return MUSC_ERR_UNSUPPORTED;
  msm::split::run_prepare(z, n, p, c, (flags & MUSC_MSM_NORMALIZE_ROWS) ? 1 : 0, workspace, stream);
  rc = msm::split::run_pairs(n, p, c, workspace, stream);
  if (rc) return rc;
  const msm::Workspace w = msm::carve(workspace, n, p);
  rc = msm::run_refine(z, n, p, c, w, stream);
  if (rc) return rc;
  return msm::run_rank(n, p, rank_lo, rank_hi, scores, w, stream);
}
