// Mutual scoring module (MSM) for gfx950.
//
// Reference semantics (models/modules/_MSM.py:10-30,53-59): for every patch q of
// image i, d(q, j) = min_r ||z[i,q] - z[j,r]||_2 for every other image j, then the
// score is the mean of ascending ranks [a, b) of {d(q, j)}_{j != i}.
//
// MI355X design
//   1. msm_norms_kernel      ||z_row||^2 for all n*p rows (one wave per row).
//   2. fill                  per-(row, image) minima buffer := +inf bits.
//   3. msm_pair_min_kernel   the whole pool is one (n*p) x (n*p) Gram matrix.  Only
//                            the upper triangle of 128x128 tiles is computed, on
//                            fp32 MFMA (v_mfma_f32_32x32x2f32), so each unordered
//                            patch pair's dot product is formed once.  The epilogue
//                            turns dots into squared distances
//                            ||a||^2 + ||b||^2 - 2 a.b (clamped at 0, as
//                            torch.cdist's matmul path does), masks same-image
//                            pairs, and reduces the tile along BOTH rows and
//                            columns, segmented by image, with NaN-propagating
//                            minima (as torch.min), merging the partial minima
//                            with unsigned atomicMin on an order-preserving key
//                            in which NaN wins (min_key, msm_common.hpp).
//                            The distance matrix never reaches HBM.
//   4. msm_rank_*_kernel     ranks each patch's n-1 minima (NaN last) and averages
//                            the square roots of ranks [a, b): sorted register
//                            lists of the b smallest (b <= 32; two lanes per patch,
//                            merged by a bitonic network), or the a-th and b-th
//                            smallest by a binary search over the key bits (one
//                            lane per patch).
#include <mutex>

#include "msm_common.hpp"

namespace musc {
namespace msm {

constexpr int BM = 128;          // tile rows (query patches)
constexpr int BN = 128;          // tile columns (reference patches)
constexpr int BK = 16;           // K chunk (channels) per pipeline stage: the double-buffered
                                 // stage is 40 KB of LDS, so three workgroups share a CU
                                 // (three waves per SIMD cover each other's epilogues and barriers)
constexpr int PITCH = BK + 4;    // LDS row pitch in floats for staged operands
constexpr int EPITCH = BN + 1;   // LDS row pitch of the epilogue distance tile
constexpr int THREADS = 256;     // 4 waves, each owns a 64x64 sub-tile
constexpr int kRowsPerPass = THREADS / (BK / 4);  // rows one 16-byte load per thread covers
constexpr int kPasses = BM / kRowsPerPass;         // such loads per thread per staged operand

constexpr int kStageFloats = 2 * (BM + BN) * PITCH;       // double-buffered A and B
constexpr int kEpiFloats = BM * EPITCH;
constexpr int kSmemFloats = kStageFloats > kEpiFloats ? kStageFloats : kEpiFloats;
constexpr int kBufferFlags = 0x00020000;  // buffer resource word 3 for raw byte-addressed loads

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
// Pairwise minima on fp32 MFMA.
// ---------------------------------------------------------------------------
// Staged operand registers are a native vector type: HIP's float4 is a struct, and
// assigning one loaded from global memory into an array element is an aggregate copy
// that the compiler left in scratch memory for the whole-chunk path.
typedef float stage4 __attribute__((ext_vector_type(4)));

// Channel-masked operand loads: kLoad 1 = 16-byte loads (c % 4 == 0), 0 = scalar loads.
// (kLoad 2, whole chunks through a buffer resource, is in the kernel.)
template <int kLoad>
__device__ inline void load_chunk(const float* __restrict__ z, int rows, int c, int row0, int k0,
                                  stage4 (&reg)[kPasses]) {
  static_assert(kLoad == 0 || kLoad == 1, "whole-chunk loads are issued by the kernel");
  const int t = threadIdx.x;
  const int lrow = t / (BK / 4);
  const int lk = (t % (BK / 4)) * 4;
#pragma unroll
  for (int i = 0; i < kPasses; ++i) {
    const int r = row0 + lrow + kRowsPerPass * i;
    const int k = k0 + lk;
    stage4 v = {0.f, 0.f, 0.f, 0.f};
    if (r < rows) {
      const float* src = z + (long long)r * c + k;
      if constexpr (kLoad == 1) {
        if (k < c) v = *reinterpret_cast<const stage4*>(src);
      } else {
        if (k + 0 < c) v.x = src[0];
        if (k + 1 < c) v.y = src[1];
        if (k + 2 < c) v.z = src[2];
        if (k + 3 < c) v.w = src[3];
      }
    }
    reg[i] = v;
  }
}

__device__ inline void store_chunk(float* __restrict__ dst, const stage4 (&reg)[kPasses]) {
  const int t = threadIdx.x;
  const int lrow = t / (BK / 4);
  const int lk = (t % (BK / 4)) * 4;
#pragma unroll
  for (int i = 0; i < kPasses; ++i)
    *reinterpret_cast<stage4*>(dst + (lrow + kRowsPerPass * i) * PITCH + lk) = reg[i];
}

// kSplit (p >= BM): a 128-row or 128-column range holds at most one image boundary,
// so tiles straddling a boundary reduce in registers too, with two image segments
// per dimension; otherwise (small p) they go through the LDS epilogue.
template <int kLoad, bool kSplit>
__global__ __launch_bounds__(THREADS, kSplit ? 3 : 2) void msm_pair_min_kernel(
    const float* __restrict__ z, const float* __restrict__ norms, const float* __restrict__ inv,
    uint32_t* __restrict__ minbits, int rows, int n, int p, int c, int T, long long ntiles) {
  __shared__ __attribute__((aligned(16))) float smem[kSplit ? kStageFloats : kSmemFloats];
  __shared__ __attribute__((aligned(16))) float s_rnorm[BM];
  __shared__ __attribute__((aligned(16))) float s_cnorm[BN];
  __shared__ __attribute__((aligned(16))) float s_rinv[BM];   // -2 x row scale (the scale is 1 unless normalising)
  __shared__ __attribute__((aligned(16))) float s_cinv[BN];
  __shared__ int s_rimg[BM], s_cimg[BN];

  const long long w = xcd_logical_id(blockIdx.x, gridDim.x);
  if (w >= ntiles) return;
  const int2 tile = decode_tile(w, T);
  const int row0 = tile.x * BM, col0 = tile.y * BN;
  // A tile is "simple" when its rows lie in one image and its columns in one image
  // (all valid): the epilogue then reduces in registers.  A simple tile whose row
  // and column image coincide holds only same-image pairs and is skipped.
  const int rlast = min(row0 + BM, rows) - 1, clast = min(col0 + BN, rows) - 1;
  const int rimg0 = row0 / p, cimg0 = col0 / p;
  const bool simple = (row0 + BM <= rows) && (col0 + BN <= rows) && (rlast / p == rimg0) && (clast / p == cimg0);
  if (simple && rimg0 == cimg0) return;

  const int t = threadIdx.x;
  if (t < BM) {
    const int r = row0 + t;
    s_rnorm[t] = r < rows ? norms[r] : 0.f;
    s_rinv[t] = r < rows ? -2.f * inv[r] : 0.f;  // exact: a power-of-two factor
    s_rimg[t] = r < rows ? r / p : n;  // n marks "no image" (padding)
  } else {
    const int cc = col0 + (t - BM);
    s_cnorm[t - BM] = cc < rows ? norms[cc] : 0.f;
    s_cinv[t - BM] = cc < rows ? inv[cc] : 0.f;
    s_cimg[t - BM] = cc < rows ? cc / p : n;
  }

  const int wave = t / kWave, lane = t % kWave;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lh = lane >> 5;

  floatx16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.f;

  // Stage buffer `b` holds A rows at smem + b*(BM+BN)*PITCH, then B rows.
  constexpr int kStage = (BM + BN) * PITCH;

  stage4 ra0[kPasses], rb0[kPasses], ra1[kPasses], rb1[kPasses];
  // Whole-chunk loads (kLoad 2) go through two buffer resources, one based at the first
  // row of the tile's A panel and one at the first row of its B panel (64-bit bases, so
  // the pool may have any size; 32-bit offsets within a 128-row panel): the byte offset
  // of each staged row is computed once per tile and the chunk offset is the scalar
  // offset, so the K loop does no address arithmetic.  Padded rows re-read the panel's
  // last row (masked in the epilogue); the extents end with the panels' last rows.
  const __amdgpu_buffer_rsrc_t zrA = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(z + (long long)row0 * c), (short)0,
      (int)((uint32_t)(rlast - row0 + 1) * (uint32_t)c * 4u), kBufferFlags);
  const __amdgpu_buffer_rsrc_t zrB = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(z + (long long)col0 * c), (short)0,
      (int)((uint32_t)(clast - col0 + 1) * (uint32_t)c * 4u), kBufferFlags);
  uint32_t voffA[kPasses], voffB[kPasses];
  if constexpr (kLoad == 2) {
    const int lrow = t / (BK / 4), lk = (t % (BK / 4)) * 4;
#pragma unroll
    for (int i = 0; i < kPasses; ++i) {
      voffA[i] = ((uint32_t)min(lrow + kRowsPerPass * i, rlast - row0) * (uint32_t)c + (uint32_t)lk) * 4u;
      voffB[i] = ((uint32_t)min(lrow + kRowsPerPass * i, clast - col0) * (uint32_t)c + (uint32_t)lk) * 4u;
    }
  }
  auto load = [&](bool rowsA, int k0, stage4 (&reg)[kPasses]) {
    if constexpr (kLoad == 2) {
#pragma unroll
      for (int i = 0; i < kPasses; ++i)
        reg[i] = __builtin_bit_cast(stage4, __builtin_amdgcn_raw_buffer_load_b128(rowsA ? zrA : zrB,
                                                                                  (int)(rowsA ? voffA[i] : voffB[i]),
                                                                                  k0 * 4, 0));
    } else {
      load_chunk<kLoad>(z, rows, c, rowsA ? row0 : col0, k0, reg);
    }
  };
  // An even number of chunks, so the K loop below leaves only at its end: an exit
  // between its two halves makes the compiler carry the accumulators in two register
  // sets and copy all 64 of them every iteration.  A chunk past the channel count
  // loads zeros and adds nothing (kLoad 2 requires c to be a multiple of two chunks).
  // Prefetches and stores are unconditional, the prefetched chunk index clamped to
  // the last chunk, so the loop body is straight-line code: the count of loads in
  // flight is the same at every wait and the wait before each LDS store leaves the
  // newer set in flight.
  const int nk = ((c + BK - 1) / BK + 1) & ~1;
  load(true, 0, ra0);
  load(false, 0, rb0);
  load(true, BK, ra1);
  load(false, BK, rb1);
  store_chunk(smem, ra0);
  store_chunk(smem + BM * PITCH, rb0);
  load(true, min(2, nk - 1) * BK, ra0);
  load(false, min(2, nk - 1) * BK, rb0);
  __syncthreads();

  auto compute = [&](int buf) {
    const float* A = smem + buf * kStage + (wm * 64 + lr) * PITCH + 4 * lh;
    const float* B = smem + buf * kStage + BM * PITCH + (wn * 64 + lr) * PITCH + 4 * lh;
#pragma unroll
    for (int s = 0; s < BK / 8; ++s) {
      const float4 a0 = *reinterpret_cast<const float4*>(A + 8 * s);
      const float4 a1 = *reinterpret_cast<const float4*>(A + 32 * PITCH + 8 * s);
      const float4 b0 = *reinterpret_cast<const float4*>(B + 8 * s);
      const float4 b1 = *reinterpret_cast<const float4*>(B + 32 * PITCH + 8 * s);
      const float av[2][4] = {{a0.x, a0.y, a0.z, a0.w}, {a1.x, a1.y, a1.z, a1.w}};
      const float bv[2][4] = {{b0.x, b0.y, b0.z, b0.w}, {b1.x, b1.y, b1.z, b1.w}};
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int nb = 0; nb < 2; ++nb)
            acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[mb][e], bv[nb][e], acc[mb][nb], 0, 0, 0);
    }
  };
  // chunk j lives in register set j % 2 from its load until its LDS store one
  // iteration before it is consumed; loads run two compute phases ahead.
  for (int kc = 0; kc < nk; kc += 2) {
    compute(0);
    store_chunk(smem + kStage, ra1);
    store_chunk(smem + kStage + BM * PITCH, rb1);
    load(true, min(kc + 3, nk - 1) * BK, ra1);
    load(false, min(kc + 3, nk - 1) * BK, rb1);
    __syncthreads();
    compute(1);
    // after the last compute this stores a clamped prefetch into buffer 0, which
    // nothing reads any more (the epilogue reuses the buffers after two barriers)
    store_chunk(smem, ra0);
    store_chunk(smem + BM * PITCH, rb0);
    load(true, min(kc + 4, nk - 1) * BK, ra0);
    load(false, min(kc + 4, nk - 1) * BK, rb0);
    __syncthreads();
  }

  if (simple) {
    // Register epilogue.  Lane (lr, lh) of wave (wm, wn) holds, for mb, nb in {0,1} and
    // v in 0..15, the dot of tile row wm*64 + mb*32 + (v/4)*8 + lh*4 + v%4 with tile
    // column wn*64 + nb*32 + lr.
    float d2[2][2][16];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 rn = *reinterpret_cast<const float4*>(&s_rnorm[wm * 64 + mb * 32 + g * 8 + lh * 4]);
        const float4 ri = *reinterpret_cast<const float4*>(&s_rinv[wm * 64 + mb * 32 + g * 8 + lh * 4]);
        const float rv[4] = {rn.x, rn.y, rn.z, rn.w};
        const float rs[4] = {ri.x, ri.y, ri.z, ri.w};
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          const float cn = s_cnorm[wn * 64 + nb * 32 + lr];
          const float ci = s_cinv[wn * 64 + nb * 32 + lr];
#pragma unroll
          for (int e = 0; e < 4; ++e)  // clamped at 0 after the minima: max(., 0) commutes with min
            d2[mb][nb][g * 4 + e] = fmaf(rs[e] * ci, acc[mb][nb][g * 4 + e], rv[e] + cn);
        }
      }
    // column minima over this wave's 64 rows: in-lane, then across the two lane halves
    float cmin[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      float m = d2[0][nb][0];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int v = 0; v < 16; ++v) m = nmin(m, d2[mb][nb][v]);
      cmin[nb] = m;
    }
    // half lh keeps column block nb = lh, with the other half's minimum for it
    cmin[0] = halves_min2(cmin[0], cmin[1]);
    // row minima over this wave's 64 columns: min over nb in-lane, then a transposing
    // butterfly over the 32 lanes of each half (31 exchanges); lane lr ends with the
    // minimum of value index k = lr, i.e. row (lr/16)*32 + ((lr%16)/4)*8 + lh*4 + lr%4.
    float rv[32];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int v = 0; v < 16; ++v) rv[mb * 16 + v] = nmin(d2[mb][0][v], d2[mb][1][v]);
    transpose_min32(rv, lr);
    __syncthreads();  // operand buffers are no longer read
    float* s_cmin = smem;             // [2 (wm)][BN]
    float* s_rmin = smem + 2 * BN;    // [2 (wn)][BM]
    s_cmin[wm * BN + wn * 64 + lh * 32 + lr] = cmin[0];
    s_rmin[wn * BM + wm * 64 + (lr >> 4) * 32 + ((lr & 15) >> 2) * 8 + lh * 4 + (lr & 3)] = rv[0];
    __syncthreads();
    if (t < BM) {
      atomicMin(minbits + (long long)(row0 + t) * n + cimg0, min_key(nmin(s_rmin[t], s_rmin[BM + t])));
    } else {
      const int j = t - BM;
      atomicMin(minbits + (long long)(col0 + j) * n + rimg0, min_key(nmin(s_cmin[j], s_cmin[BN + j])));
    }
    return;
  }

  if constexpr (kSplit) {
    // Two-segment register epilogue (P >= 128, so a 128-row or 128-column range holds
    // at most one image boundary).  Tile rows [0, rsplit) belong to image rA, rows
    // [rsplit, BM) to image rA + 1 or to the padding (image n); columns likewise with
    // csplit and cA.  Whether a pair is masked (same image, or padding) depends only
    // on the segments of its row and column, so minima are taken per segment over the
    // raw distances and a masked segment pair is replaced by +inf afterwards, the same
    // as masking every distance first (min over +inf only).  A wave whose 64 rows (or
    // columns) lie in one segment reduces them without per-distance selects.
    const float inf = __int_as_float(kInfBits);
    const int rA = rimg0, cA = cimg0;
    const int rsplit = min(BM, min((rA + 1) * p, rows) - row0);
    const int csplit = min(BN, min((cA + 1) * p, rows) - col0);
    const int rBimg = row0 + rsplit < rows ? rA + 1 : n;  // used only when segment B is not empty
    const int cBimg = col0 + csplit < rows ? cA + 1 : n;
    const bool mAA = rA == cA, mAB = cBimg == n || rA == cBimg;
    const bool mBA = rBimg == n || rBimg == cA, mBB = rBimg == n || cBimg == n || rBimg == cBimg;
    float d2[2][2][16];
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
        for (int nb = 0; nb < 2; ++nb) {
          const float cn = s_cnorm[wn * 64 + nb * 32 + lr];
          const float ci = s_cinv[wn * 64 + nb * 32 + lr];
#pragma unroll
          for (int e = 0; e < 4; ++e)  // clamped at 0 after the minima
            d2[mb][nb][g * 4 + e] = fmaf(rs[e] * ci, acc[mb][nb][g * 4 + e], rv[e] + cn);
        }
      }
    // column minima over this wave's 64 rows, per row segment, then across lane halves
    const int wr0 = wm * 64, wc0 = wn * 64;
    float cminA[2], cminB[2];
    if (rsplit >= wr0 + 64 || rsplit <= wr0) {
      float m[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        float x = d2[0][nb][0];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int v = 0; v < 16; ++v) x = nmin(x, d2[mb][nb][v]);
        m[nb] = x;
      }
      const bool inA = rsplit > wr0;
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        cminA[nb] = inA ? m[nb] : inf;
        cminB[nb] = inA ? inf : m[nb];
      }
    } else {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
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
    float colA = halves_min2(cminA[0], cminA[1]);  // column wc0 + lh * 32 + lr
    float colB = halves_min2(cminB[0], cminB[1]);
    {
      const bool colInB = wc0 + lh * 32 + lr >= csplit;
      if (colInB ? mAB : mAA) colA = inf;
      if (colInB ? mBB : mBA) colB = inf;
    }
    // row minima over this wave's 64 columns, per column segment: transposing
    // butterflies as in the single-segment path, two when the boundary falls inside
    float rowminA, rowminB;
    if (csplit >= wc0 + 64 || csplit <= wc0) {
      float rv[32];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int v = 0; v < 16; ++v) rv[mb * 16 + v] = nmin(d2[mb][0][v], d2[mb][1][v]);
      const float m = transpose_min32(rv, lr);
      const bool inA = csplit > wc0;
      rowminA = inA ? m : inf;
      rowminB = inA ? inf : m;
    } else {
      const bool colB0 = wc0 + lr >= csplit, colB1 = wc0 + 32 + lr >= csplit;
      {
        float rv[32];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            rv[mb * 16 + v] = nmin(colB0 ? inf : d2[mb][0][v], colB1 ? inf : d2[mb][1][v]);
        rowminA = transpose_min32(rv, lr);
      }
      {
        float rv[32];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            rv[mb * 16 + v] = nmin(colB0 ? d2[mb][0][v] : inf, colB1 ? d2[mb][1][v] : inf);
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
    float* s_cminA = smem;            // [2 (wm)][BN]
    float* s_cminB = smem + 2 * BN;
    float* s_rminA = smem + 4 * BN;   // [2 (wn)][BM]
    float* s_rminB = smem + 4 * BN + 2 * BM;
    s_cminA[wm * BN + wn * 64 + lh * 32 + lr] = colA;
    s_cminB[wm * BN + wn * 64 + lh * 32 + lr] = colB;
    s_rminA[wn * BM + rk] = rowminA;
    s_rminB[wn * BM + rk] = rowminB;
    __syncthreads();
    if (t < BM) {
      const int r = row0 + t;
      if (r < rows) {
        // a segment pair with no pair of different images is exactly +inf (masked):
        // skip it, also because segment B may be the padding image n
        const float a = nmin(s_rminA[t], s_rminA[BM + t]);
        const float b = nmin(s_rminB[t], s_rminB[BM + t]);
        if (a != inf) atomicMin(minbits + (long long)r * n + cA, min_key(a));
        if (b != inf) atomicMin(minbits + (long long)r * n + cA + 1, min_key(b));
      }
    } else {
      const int j = t - BM;
      const int cc = col0 + j;
      if (cc < rows) {
        const float a = nmin(s_cminA[j], s_cminA[BN + j]);
        const float b = nmin(s_cminB[j], s_cminB[BN + j]);
        if (a != inf) atomicMin(minbits + (long long)cc * n + rA, min_key(a));
        if (b != inf) atomicMin(minbits + (long long)cc * n + rA + 1, min_key(b));
      }
    }
    return;
  } else {
  // Epilogue: squared distances into LDS (the operand buffers are free now).
  float* E = smem;
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int j = wn * 64 + nb * 32 + lr;
      const float cn = s_cnorm[j];
      const float cs = s_cinv[j];
      const int ci = s_cimg[j];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int i = wm * 64 + mb * 32 + (v >> 2) * 8 + lh * 4 + (v & 3);
        const float d2 = fmaf(cs * s_rinv[i], acc[mb][nb][v], s_rnorm[i] + cn);  // clamped by min_key
        const int ri = s_rimg[i];
        E[i * EPITCH + j] = (ri == ci || ri == n || ci == n) ? __int_as_float(kInfBits) : d2;
      }
    }
  __syncthreads();

  if (t < BM) {
    // Row pass: minimum over this tile's columns, one segment per column image.
    const int r = row0 + t;
    if (r < rows) {
      uint32_t* dst = minbits + (long long)r * n;
      int seg = s_cimg[0];
      float cur = __int_as_float(kInfBits);
      for (int j = 0; j < BN; ++j) {
        const int ci = s_cimg[j];
        if (ci != seg) {
          if (seg < n && cur != __int_as_float(kInfBits)) atomicMin(dst + seg, min_key(cur));
          seg = ci;
          cur = __int_as_float(kInfBits);
        }
        cur = nmin(cur, E[t * EPITCH + j]);
      }
      if (seg < n && cur != __int_as_float(kInfBits)) atomicMin(dst + seg, min_key(cur));
    }
  } else {
    // Column pass: the same tile seen from the reference side (symmetric reuse).
    const int j = t - BM;
    const int cc = col0 + j;
    if (cc < rows) {
      uint32_t* dst = minbits + (long long)cc * n;
      int seg = s_rimg[0];
      float cur = __int_as_float(kInfBits);
      for (int i = 0; i < BM; ++i) {
        const int ri = s_rimg[i];
        if (ri != seg) {
          if (seg < n && cur != __int_as_float(kInfBits)) atomicMin(dst + seg, min_key(cur));
          seg = ri;
          cur = __int_as_float(kInfBits);
        }
        cur = nmin(cur, E[i * EPITCH + j]);
      }
      if (seg < n && cur != __int_as_float(kInfBits)) atomicMin(dst + seg, min_key(cur));
    }
  }
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
// keys flags each (row, image) minimum at or below 32 eps C (norms[row] + the largest
// norm of the image) -- the same bound with the image's largest norm, so every pair
// the reference recomputes lies in a flagged (row, image) or cannot be its minimum --
// and the wave recomputes that minimum over all P patches of the image as
// sum_c (s_a a_c - s_b b_c)^2 in fp32 (s the row scales: 1 / ||z|| with row
// normalisation, else 1), accurate to a few ulps of d^2 itself; identical rows give
// exactly 0.  Above the bound the expanded form's error in d is at most about
// eps ||.||^2 / (2 d), far below the 2e-5 gate.  A flagged minimum is replaced
// (stored), not merged: the exact value may lie above the expanded one.  NaN minima
// (key 0), the own image and +inf (key kMinFill) are left alone.  With nothing
// flagged the pass reads the keys once (37.7 MB at N = 83, P = 1369).
// ---------------------------------------------------------------------------
constexpr int kRefineRows = 16;                 // rows per wave
constexpr float kRefineEps = 1.192092896e-7f;   // the fp32 machine epsilon of the reference's bound

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

// Stage 2: the fp32 MFMA pairwise-minima kernel (leaves squared minima bits).
inline int run_pairs(const float* z, int n, int p, int c, const Workspace& w, hipStream_t s) {
  const long long rows = (long long)n * p;
  const long long T = (rows + BM - 1) / BM;
  const long long ntiles = total_tiles(T);
  const long long grid = (ntiles + kXcds - 1) / kXcds * kXcds;
  if (grid > 0x7fffffffLL) return MUSC_ERR_UNSUPPORTED;
#define MUSC_PAIR_LAUNCH(V4, SPLIT)                                                                              \
  hipLaunchKernelGGL((msm_pair_min_kernel<V4, SPLIT>), dim3((unsigned)grid), dim3(THREADS), 0, s, z, w.norms, w.inv, \
                     w.minbits, (int)rows, n, p, c, (int)T, ntiles)
  const bool split = p >= BM;
  // whole-chunk loads: c a multiple of two chunks, and a 128-row panel addressable with
  // 32-bit offsets (any pool size: the buffer resources are based at each tile's panels)
  if (c % (2 * BK) == 0 && (unsigned long long)BM * (unsigned long long)c * 4ull < (1ull << 31)) {
    if (split) MUSC_PAIR_LAUNCH(2, true); else MUSC_PAIR_LAUNCH(2, false);
  } else if ((c & 3) == 0) {
    if (split) MUSC_PAIR_LAUNCH(1, true); else MUSC_PAIR_LAUNCH(1, false);
  } else {
    if (split) MUSC_PAIR_LAUNCH(0, true); else MUSC_PAIR_LAUNCH(0, false);
  }
#undef MUSC_PAIR_LAUNCH
  return check_launch();
}

// Stage 3: exact minima where the expanded form cancels (either engine's keys).
int run_refine(const float* z, int n, int p, int c, const Workspace& w, hipStream_t s) {
  const long long rows = (long long)n * p;
  const long long blocks = ((rows + kRefineRows - 1) / kRefineRows + 3) / 4;
  hipLaunchKernelGGL(msm_refine_kernel, dim3((unsigned)blocks), dim3(256), 0, s, z, (int)rows, n, p, c, w.norms,
                     w.scale, w.imgmax, w.minbits, 32.f * kRefineEps * (float)c);
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
