// fp32 MFMA pairwise minima of the mutual scoring module (MSM) for gfx950.
//
// msm_pair_min_kernel: the whole pool is one (n*p) x (n*p) Gram matrix.  Only the
// upper triangle of 128x128 tiles is computed, on fp32 MFMA (v_mfma_f32_32x32x2f32),
// so each unordered patch pair's dot product is formed once.  The epilogue turns dots
// into squared distances ||a||^2 + ||b||^2 - 2 a.b (clamped at 0, as torch.cdist's
// matmul path does; models/modules/_MSM.py:16-17), masks same-image pairs, and
// reduces the tile along BOTH rows and columns, segmented by image, with
// NaN-propagating minima (as torch.min), merging the partial minima with unsigned
// atomicMin on an order-preserving key in which NaN wins (min_key, msm_common.hpp).
// The distance matrix never reaches HBM.  The stages around it (norms, refinement,
// ranks) and the C-ABI are in msm.hip; this file holds only what the kernel is
// compiled from, so that measurements of it can name their sources.
#include "msm_common.hpp"

namespace musc {
namespace msm {

constexpr int BM = 128;          // tile rows (query patches)
constexpr int BN = 128;          // tile columns (reference patches)
constexpr int BK = 16;           // K chunk (channels) per pipeline stage: the double-buffered
                                 // stage is 40 KB of LDS, so three workgroups share a CU
                                 // (three waves per SIMD cover each other's epilogues and barriers)
constexpr int PITCH = BK;        // LDS row pitch in floats for staged operands (64 bytes)
constexpr int EPITCH = BN + 1;   // LDS row pitch of the epilogue distance tile
constexpr int THREADS = 256;     // 4 waves, each owns a 64x64 sub-tile
constexpr int kRowsPerPass = THREADS / (BK / 4);  // rows one 16-byte load per thread covers
constexpr int kPasses = BM / kRowsPerPass;         // such loads per thread per staged operand

static_assert(BK == 16 && kRowsPerPass % 16 == 0, "the segment swizzle assumes 4 segments per row");
constexpr int kStageFloats = 2 * (BM + BN) * PITCH;       // double-buffered A and B
constexpr int kEpiFloats = BM * EPITCH;
constexpr int kSmemFloats = kStageFloats > kEpiFloats ? kStageFloats : kEpiFloats;
constexpr int kBufferFlags = 0x00020000;  // buffer resource word 3 for raw byte-addressed loads

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

// A staged row is four 16-byte segments; segment s of row r sits at s ^ seg_swizzle(r).
// The LDS serves 16 lanes of a 16-byte access per 256-byte window: in the operand reads
// they are 16 consecutive rows at one segment, in the stores 4 rows x 4 segments, and
// with the swizzle both land on 16 distinct bank groups (without it, rows r and r + 4
// of a 64-byte pitch, or r and r + 3 of an 80-byte one, share banks).
__device__ inline int seg_swizzle(int row) { return (row >> 2) & 3; }

__device__ inline void store_chunk(float* __restrict__ dst, const stage4 (&reg)[kPasses]) {
  const int t = threadIdx.x;
  const int lrow = t / (BK / 4);
  // kRowsPerPass is a multiple of 16, so every pass of this thread has the same swizzle
  const int lk = ((t % (BK / 4)) ^ seg_swizzle(lrow)) * 4;
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

  // lane (lr, lh) reads segments lh and lh + 2 of rows wm*64 + lr (+ 32) and wn*64 + lr
  // (+ 32): the row offsets are multiples of 16, so the swizzle is that of lr
  const int seg_off[2] = {4 * (lh ^ seg_swizzle(lr)), 4 * ((lh + 2) ^ seg_swizzle(lr))};
  auto compute = [&](int buf) {
    const float* A = smem + buf * kStage + (wm * 64 + lr) * PITCH;
    const float* B = smem + buf * kStage + BM * PITCH + (wn * 64 + lr) * PITCH;
#pragma unroll
    for (int s = 0; s < BK / 8; ++s) {
      const float4 a0 = *reinterpret_cast<const float4*>(A + seg_off[s]);
      const float4 a1 = *reinterpret_cast<const float4*>(A + 32 * PITCH + seg_off[s]);
      const float4 b0 = *reinterpret_cast<const float4*>(B + seg_off[s]);
      const float4 b1 = *reinterpret_cast<const float4*>(B + 32 * PITCH + seg_off[s]);
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

// Stage 2: the fp32 MFMA pairwise-minima kernel (leaves squared minima bits).
int run_pairs(const float* z, int n, int p, int c, const Workspace& w, hipStream_t s) {
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

}  // namespace msm
}  // namespace musc
