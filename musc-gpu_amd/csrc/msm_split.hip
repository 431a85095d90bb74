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
//                 row's share of a pipeline stage); channels padded with zeros to a
//                 whole number of 32-channel pairs of blocks.
//   pair kernel   256 x 256 tiles of the upper triangle (symmetric reuse, bands of
//                 8 tile rows, XCD-grouped), one workgroup per tile and CU, 4 waves
//                 each own 128 x 128 (accumulators in AGPRs).  Stages of 16 channels
//                 (32 KB: 256 A rows + 256 B rows) go straight from global memory into
//                 LDS (buffer_load_dwordx4 ... lds: lane l of a load lands at base +
//                 16 l, so one load fills 16 rows of 64 bytes) through a 4-deep ring,
//                 loads 4 stages ahead, one barrier per stage, no staging registers;
//                 the next stage's operands are read into a second register set, and
//                 the loads and reads are interleaved with the 48 MFMAs of a stage, so
//                 that the one wave per SIMD keeps the matrix pipe fed.  The 16-byte
//                 segment s of staged row r sits at position s ^ ((r >> 2) & 3), which
//                 keeps the MFMA operand reads free of bank conflicts.
//                 Register epilogues: tiles of one image pair fold each distance into
//                 the row and column minima at once; tiles that straddle an image
//                 boundary (p >= 256: one at most per dimension) keep the minima per
//                 image segment, 64 rows at a time.
#include <hip/hip_fp16.h>

#include "msm_common.hpp"

namespace musc {
namespace msm {
namespace split {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));

constexpr int TM = 256;                      // triangle tile: rows = columns, one workgroup per tile
constexpr int KB = 16;                       // channels per stage (each of hi and lo)
constexpr int ROWB = 4 * KB;                 // bytes per row and stage: hi[16] lo[16] fp16
constexpr int NSTAGE = 4;                    // LDS ring depth: loads run NSTAGE stages ahead of the MFMAs
constexpr int THREADS = 256;                 // 4 waves: 2 (rows) x 2 (columns) of 128 x 128
constexpr int kWaveTile = 128;               // rows (and columns) per wave
constexpr int kBlocks = kWaveTile / 32;      // 32 x 32 MFMA blocks per wave dimension
constexpr int kStageRows = 2 * TM;           // A rows (tile rows) then B rows (tile columns)
constexpr int kStageBytes = kStageRows * ROWB;  // 32 KB
constexpr int kScaleShift = 10;              // normalised rows are scaled by 2^10
constexpr int kBandSplit = BAND;             // tile rows per band of the triangle enumeration
constexpr int kRowsPerLoad = kWave * 16 / ROWB;              // 16 staged rows per direct load
constexpr int kWaveRows = kStageRows / (THREADS / kWave);    // 128 staged rows per wave and stage
constexpr int kLoads = kWaveRows / kRowsPerLoad;             // direct loads per wave per stage

static_assert(kLoads == 8, "the vmcnt waits of the main loop count 8 loads per wave and stage");
static_assert(NSTAGE == 4, "the vmcnt waits of the main loop are written for a 4-deep ring");
static_assert(THREADS == TM, "the prologue and the final merge map thread t to tile row t and column t");
static_assert(TM % kWaveRows == 0, "a wave's staged rows lie in one panel");

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
  // A row of whole 32-channel pairs of blocks, up to 1024 channels (the pools' C), stays in
  // registers between its norm and its split (at most 4 float4 per lane, taken by the same
  // lanes in the same order as row_sumsq, so the same sum); otherwise the split reads the
  // row again.
  const bool in_regs = (c & 31) == 0 && c <= 16 * kWave;
  float4 xv[4];
  double acc = 0.0;
  if (in_regs) {
    const float4* s4 = reinterpret_cast<const float4*>(src);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = lane + j * kWave;
      if (k < c / 4) {
        const float4 v = s4[k];
        xv[j] = v;
        acc += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
      }
    }
    acc = wave_sum(acc);
  } else {
    acc = row_sumsq(src, c, lane);
  }
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
  // hi = fp16(fp32(v)), lo = fp16(fp32(v - hi)) with v = x * sc rounded to fp64, each step
  // rounded to nearest even as written: the empty asm statements keep the compiler from
  // folding the two narrowing steps into one (a software f64 -> f16 rounding, which
  // differs on ties of the fp32 step) or fusing x * sc into the subtraction, which it
  // otherwise does in some paths and not in others.
  auto split1 = [&](float x, _Float16& hi, _Float16& lo) {
    double v = (double)x * sc;
    asm volatile("" : "+v"(v));
    float vf = (float)v;
    asm volatile("" : "+v"(vf));
    hi = (_Float16)vf;
    float rf = (float)(v - (double)(float)hi);
    asm volatile("" : "+v"(rf));
    lo = (_Float16)rf;
  };
  if (in_regs) {
    // channels 4k .. 4k+3 (k = lane + j*64): one 8-byte store of hi and one of lo in
    // block k / 4 (no padding channels: c is a multiple of 32)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = lane + j * kWave;
      if (k < c / 4) {
        const float xs[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
        half4 hi, lo;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          _Float16 h, l;
          split1(xs[e], h, l);
          hi[e] = h;
          lo[e] = l;
        }
        _Float16* blk = dst + (k >> 2) * (2 * KB) + (k & 3) * 4;
        *reinterpret_cast<half4*>(blk) = hi;
        *reinterpret_cast<half4*>(blk + KB) = lo;
      }
    }
  } else if ((c & 7) == 0) {
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
// Pair minima.  Workgroup w takes triangle tile w (256 x 256), one workgroup per CU;
// wave (wm, wn) owns tile rows wm*128 .. +127 x columns wn*128 .. +127, 4 x 4 blocks of
// 32 x 32 accumulated in registers (AGPRs).  The operands of stage j+1 are read from
// LDS into a second register set while the MFMAs of stage j run, so the single wave
// per SIMD keeps issuing MFMAs; the 4-deep LDS ring holds loads up to four stages
// ahead.
// ---------------------------------------------------------------------------
struct SplitOps {
  half8 ahi[kBlocks], alo[kBlocks], bhi[kBlocks], blo[kBlocks];
};

__global__ __launch_bounds__(THREADS, 1) void split_pair_kernel(const _Float16* __restrict__ hl,
                                                               const float* __restrict__ norms,
                                                               const float* __restrict__ inv,
                                                               uint32_t* __restrict__ minbits, int rows, int n, int p,
                                                               int nkb, int T, long long ntiles) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[NSTAGE * kStageBytes];
  __shared__ __attribute__((aligned(16))) float s_rnorm[TM];
  __shared__ __attribute__((aligned(16))) float s_rinv[TM];
  __shared__ float s_cnorm[TM];
  __shared__ float s_cinv[TM];

  const long long w = xcd_logical_id(blockIdx.x, gridDim.x);
  if (w >= ntiles) return;
  const int2 tile = decode_tile<kBandSplit>(w, T);
  const int row0 = tile.x * TM, col0 = tile.y * TM;
  const int rlast = min(row0 + TM, rows) - 1, clast = min(col0 + TM, rows) - 1;
  const int rimg0 = row0 / p, cimg0 = col0 / p;
  // simple: the tile's rows lie in one image and its columns in one image (no boundary,
  // no padding); a tile of one image only has no pair to score
  const bool simple = (row0 + TM <= rows) && (col0 + TM <= rows) && (rlast / p == rimg0) && (clast / p == cimg0);
  if (simple && rimg0 == cimg0) return;

  const int t = threadIdx.x;  // THREADS == TM: thread t merges tile row t and tile column t
  const int wave = t / kWave, lane = t % kWave;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lh = lane >> 5;

  floatx16 acc[kBlocks][kBlocks];
#pragma unroll
  for (int a = 0; a < kBlocks; ++a)
#pragma unroll
    for (int b = 0; b < kBlocks; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.f;

  // Loads go straight from global memory into LDS (buffer_load_dwordx4 ... lds: lane
  // l of a load lands at M0 + 16 l, so one load fills 16 staged rows of 64 bytes).
  // Wave wv fills staged rows wv*128 .. wv*128 + 127: waves 0 and 1 the tile rows (A
  // panel), waves 2 and 3 the tile columns (B panel).  Lane l of a load carries row
  // R = R0 + l/4 into LDS position l % 4, i.e. segment (l % 4) ^ ((R >> 2) & 3).
  // Padded rows re-read the last row (their pairs are masked in the epilogue).
  // Addressing: one buffer resource per wave, based at the first row of its panel
  // (64-bit base, so the split array may have any size; the extent ends with the
  // panel's last row), one 32-bit byte offset per load within the panel (row +
  // segment, loop-invariant) and the stage offset as the scalar offset.  The loads are
  // issued from inline assembly so that the compiler, which cannot tell the ring
  // buffers apart, does not wait for them before reading another buffer; the loop
  // waits for them explicitly.
  const int wv = __builtin_amdgcn_readfirstlane(wave);
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
  const bool waveA = wv * kWaveRows < TM;  // wave-uniform
  const int4v rsrc = waveA ? panel_rsrc(row0, rlast) : panel_rsrc(col0, clast);
  uint32_t voff[kLoads];
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const int R = wave * kWaveRows + i * kRowsPerLoad + lrow;
    const int prow = R < TM ? min(R, rlast - row0) : min(R - TM, clast - col0);
    const int lseg = (lane & 3) ^ ((R >> 2) & 3);
    voff[i] = (uint32_t)prow * (uint32_t)(nkb * ROWB) + (uint32_t)(lseg * 16);
  }
  // wave-uniform LDS base of this wave's staged rows in buffer 0 (M0 is a scalar register)
  const uint32_t lds_wave =
      __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(lds_void*)smem + (uint32_t)(wv * kWaveRows * ROWB));
  // load i (0 .. kLoads-1) of this wave's share of stage kb into LDS buffer buf
  auto issue_one = [&](int kb, int buf, int i) {
    const uint32_t soff = (uint32_t)(kb * ROWB);
    const uint32_t base = lds_wave + (uint32_t)(buf * kStageBytes);
    // M0 = base + this load's 16 rows; s_nop: one wait state between the scalar write
    // of M0 and the load that reads it
    asm volatile("s_add_u32 m0, %0, %4\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(base), "v"(voff[i]), "s"(rsrc), "s"(soff), "i"(i * kRowsPerLoad * ROWB)
                 : "memory", "m0", "scc");
  };
  auto issue = [&](int kb, int buf) {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) issue_one(kb, buf, i);
  };
  // Waits until this thread's loads of stage `st` have landed, given that the loads of
  // every stage up to `last_issued` have been issued (loads complete in order).
  auto wait_stage = [&](int st, int last_issued) {
    const int later = last_issued - st;
    if (later >= 3)
      asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
    else if (later == 2)
      asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    else if (later == 1)
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  };
  // Segments of a staged row: 0, 1 = hi channels 0-7, 8-15; 2, 3 = lo.  Segment s of
  // staged row r sits at position s ^ ((r >> 2) & 3); the operand rows here are
  // (multiple of 32) + lr, so the swizzle is (lr >> 2) & 3.  Over any 16 consecutive
  // rows (the lanes an LDS read serves together) the pairs (r & 3, (r >> 2) & 3) take
  // 16 distinct 16-byte slots of a 256-byte bank window: conflict-free reads.
  const int sw = (lr >> 2) & 3;
  const int phi = (lh ^ sw) * 16, plo = ((2 + lh) ^ sw) * 16;
  const int aoff = (wm * kWaveTile + lr) * ROWB, boff = (TM + wn * kWaveTile + lr) * ROWB;
  // operand vector r (0 .. 15) of stage buffer buf: block r / 4, one of A hi, A lo,
  // B hi, B lo by r % 4
  auto read_one = [&](int buf, SplitOps& o, int r) {
    const int b = r >> 2, kind = r & 3;
    const unsigned char* base = smem + buf * kStageBytes + (kind < 2 ? aoff : boff) + b * 32 * ROWB;
    const half8 x = *reinterpret_cast<const half8*>(base + ((kind & 1) ? plo : phi));
    if (kind == 0) o.ahi[b] = x;
    if (kind == 1) o.alo[b] = x;
    if (kind == 2) o.bhi[b] = x;
    if (kind == 3) o.blo[b] = x;
  };
  auto read_ops = [&](int buf, SplitOps& o) {
#pragma unroll
    for (int r = 0; r < 16; ++r) read_one(buf, o, r);
  };
  // MFMA idx (0 .. 47) of a stage: product idx / 16 (hi.hi, hi.lo, lo.hi), block
  // (mb, nb) = ((idx % 16) / 4, idx % 4); per accumulator: hi.hi, then hi.lo, then lo.hi
  auto mfma_one = [&](const SplitOps& o, int idx) {
    const int prod = idx >> 4, mb = (idx >> 2) & 3, nb = idx & 3;
    const half8 a = prod == 2 ? o.alo[mb] : o.ahi[mb];
    const half8 b = prod == 1 ? o.blo[nb] : o.bhi[nb];
    acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[mb][nb], 0, 0, 0);
  };
  using F = std::false_type;
  using Tr = std::true_type;

  // The norms and epilogue scales of the tile's rows and columns go into LDS the same way
  // (lane l of a dword load lands at M0 + 4 l; wave wv takes entries wv*64 .. +63), issued
  // before the stages' loads, so they have landed once stage 0 has (loads complete in
  // order) and no wave waits for them at the start of the tile; entries past the pool's
  // last row read 0 (the buffer extent).
  {
    auto vec_rsrc = [&](const float* base, int first) {
      const unsigned long long addr = reinterpret_cast<unsigned long long>(base + first);
      int4v r;
      r.x = (int)(uint32_t)(addr & 0xffffffffull);
      r.y = (int)(uint32_t)(addr >> 32);
      r.z = min(rows - first, TM) * 4;
      r.w = kBufferFlags;
      return r;
    };
    const uint32_t nvoff = (uint32_t)((wave * kWave + lane) * 4);
    auto load_vec = [&](const int4v& rs, float* dst) {
      const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(lds_void*)dst + (uint32_t)(wv * kWave * 4));
      asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                   :
                   : "s"(m0), "v"(nvoff), "s"(rs)
                   : "memory", "m0");
    };
    load_vec(vec_rsrc(norms, row0), s_rnorm);
    load_vec(vec_rsrc(inv, row0), s_rinv);
    load_vec(vec_rsrc(norms, col0), s_cnorm);
    load_vec(vec_rsrc(inv, col0), s_cinv);
  }
  // Stage j lives in LDS buffer j % NSTAGE.  Step j: wait for this thread's loads of
  // stage j + 1; the barrier then makes every wave's loads of stage j + 1 visible and
  // guarantees that every wave has finished reading stage j (its reads completed before
  // the barrier; its operands are in registers), so buffer j % NSTAGE takes the loads of
  // stage j + NSTAGE; then the MFMAs of stage j run from registers while the operands of
  // stage j + 1 are read into the other register set.  The last step reads a stale
  // buffer into registers it never uses.  nkb is even (the split array is padded to
  // whole pairs of stages), so the loop takes two steps per iteration with the two
  // register sets in fixed roles.
  for (int st = 0; st < NSTAGE && st < nkb; ++st) issue(st, st);
  wait_stage(0, min(NSTAGE, nkb) - 1);
  __syncthreads();
  SplitOps o0, o1;
  read_ops(0, o0);
  // Within a step the 48 MFMAs go in 8 groups of 6, each group preceded by one direct
  // load of stage j + NSTAGE (steps that have one) and two operand reads of stage j + 1,
  // with scheduling barriers between the groups: with one wave per SIMD nothing else
  // covers a load whose issue stalls or a read's latency, so they overlap the MFMAs
  // already in the matrix pipe.
  auto step = [&](int j, const SplitOps& cur, SplitOps& nxt, auto with_loads) {
    wait_stage(j + 1, min(j + NSTAGE - 1, nkb - 1));
    __syncthreads();
#pragma unroll
    for (int gi = 0; gi < kLoads; ++gi) {
      if constexpr (decltype(with_loads)::value) issue_one(j + NSTAGE, j % NSTAGE, gi);
      read_one((j + 1) % NSTAGE, nxt, 2 * gi);
      read_one((j + 1) % NSTAGE, nxt, 2 * gi + 1);
#pragma unroll
      for (int k = 0; k < 6; ++k) mfma_one(cur, gi * 6 + k);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // j even and nkb even: j + NSTAGE < nkb also gives j + 1 + NSTAGE < nkb
  int j = 0;
  for (; j + NSTAGE < nkb; j += 2) {
    step(j, o0, o1, Tr{});
    step(j + 1, o1, o0, Tr{});
  }
  for (; j < nkb; j += 2) {
    step(j, o0, o1, F{});
    step(j + 1, o1, o0, F{});
  }

  // Epilogue.  Lane (lr, lh) of wave (wm, wn) holds, for mb, nb < 4, v < 16, the dot
  // of tile row wm*128 + mb*32 + (v/4)*8 + lh*4 + v%4 with tile column
  // wn*128 + nb*32 + lr.
  // The thread's indices are derived again from an opaque copy of the thread index
  // (the wave's in scalar registers): otherwise the compiler keeps their prologue
  // values live across the main loop, where every register is taken, and spills them
  // to scratch memory, whose reloads here each wait a full memory round trip.
  int t_epi = threadIdx.x;
  asm volatile("" : "+v"(t_epi));
  {
  const int t = t_epi;
  const int wave = __builtin_amdgcn_readfirstlane(t_epi / kWave), lane = t_epi % kWave;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lh = lane >> 5;
  const int rA = rimg0, cA = cimg0;
  const int wc0 = wn * kWaveTile;
  const float inf = __int_as_float(kInfBits);
  float cn[kBlocks], ci[kBlocks];
#pragma unroll
  for (int nb = 0; nb < kBlocks; ++nb) {
    cn[nb] = s_cnorm[wc0 + nb * 32 + lr];
    ci[nb] = s_cinv[wc0 + nb * 32 + lr];
  }

  if (__builtin_expect(simple, 1)) {  // about two thirds of the tiles at P = 1369
    // Rows of image rA, columns of image cA: each squared distance is formed and folded
    // at once into the column minima (per nb, over this lane's rows) and the
    // row-minimum items (per row, over this lane's columns), one 64-row half at a time.
    const int wr0 = wm * kWaveTile;
    float cmin[kBlocks], rmin[2];
#pragma unroll
    for (int nb = 0; nb < kBlocks; ++nb) cmin[nb] = inf;
    // Unit rows: when every row and column of this wave has norm 1 and scale 2^-10 (rows
    // L2-normalised by the prepare stage), each distance is fma(-2^-19, dot, 2) -- the
    // general formula with those values, exactly -- which never increases with the dot,
    // and rounding keeps that order: the minimum distance over any set of pairs is
    // fma(-2^-19, maximum dot, 2), bit for bit (NaN and infinities included).  Then only
    // the dots are reduced (as minima of their negations, with the same butterflies) and
    // the formula is applied to the four minima of each lane.
    const float kUnit = 1.f / (float)(1 << kScaleShift);
    bool unit = true;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int rr = wr0 + k * 64 + lane, cc2 = wc0 + k * 64 + lane;
      unit = unit && s_rnorm[rr] == 1.f && s_rinv[rr] == kUnit && s_cnorm[cc2] == 1.f && s_cinv[cc2] == kUnit;
    }
    if (__all(unit)) {
      constexpr float kNegUnitScale = 2.f / (float)(1 << (2 * kScaleShift));  // -(-2 x 2^-10 x 2^-10)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float rv[32];
#pragma unroll
        for (int m2 = 0; m2 < 2; ++m2) {
          const int mb = 2 * h + m2;
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            float m = inf;
#pragma unroll
            for (int nb = 0; nb < kBlocks; ++nb) {
              const float x = -acc[mb][nb][v];
              cmin[nb] = nmin(cmin[nb], x);
              m = nmin(m, x);
            }
            rv[m2 * 16 + v] = m;
          }
        }
        rmin[h] = fmaf(kNegUnitScale, transpose_min32(rv, lr), 2.f);
      }
#pragma unroll
      for (int nb = 0; nb < kBlocks; ++nb) cmin[nb] = fmaf(kNegUnitScale, cmin[nb], 2.f);
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float rv[32];
#pragma unroll
        for (int m2 = 0; m2 < 2; ++m2) {
          const int mb = 2 * h + m2;
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int i0 = wr0 + mb * 32 + g * 8 + lh * 4;
            const float4 rn = *reinterpret_cast<const float4*>(&s_rnorm[i0]);
            const float4 ri = *reinterpret_cast<const float4*>(&s_rinv[i0]);
            const float rnv[4] = {rn.x, rn.y, rn.z, rn.w};
            const float rs[4] = {-2.f * ri.x, -2.f * ri.y, -2.f * ri.z, -2.f * ri.w};  // -2 x row scale (exact)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float m = inf;
#pragma unroll
              for (int nb = 0; nb < kBlocks; ++nb) {  // clamped at 0 by min_key, after the minima
                const float d = fmaf(rs[e] * ci[nb], acc[mb][nb][g * 4 + e], rnv[e] + cn[nb]);
                cmin[nb] = nmin(cmin[nb], d);
                m = nmin(m, d);
              }
              rv[m2 * 16 + g * 4 + e] = m;
            }
          }
        }
        // row wr0 + h*64 + transposed_row(lr, lh): minimum over the wave's 128 columns
        rmin[h] = transpose_min32(rv, lr);
      }
    }
    // column wc0 + (2q + lh)*32 + lr: minimum over the wave's 128 rows
    float cm[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) cm[q] = halves_min2(cmin[2 * q], cmin[2 * q + 1]);
    __syncthreads();  // operand buffers are no longer read
    float* s_cmin = reinterpret_cast<float*>(smem);  // [2 (wm)][TM]
    float* s_rmin = s_cmin + 2 * TM;                  // [2 (wn)][TM]
#pragma unroll
    for (int q = 0; q < 2; ++q) s_cmin[wm * TM + wc0 + (2 * q + lh) * 32 + lr] = cm[q];
#pragma unroll
    for (int h = 0; h < 2; ++h) s_rmin[wn * TM + wr0 + h * 64 + transposed_row(lr, lh)] = rmin[h];
    __syncthreads();
    atomicMin(minbits + (long long)(col0 + t) * n + rA, min_key(nmin(s_cmin[t], s_cmin[TM + t])));
    atomicMin(minbits + (long long)(row0 + t) * n + cA, min_key(nmin(s_rmin[t], s_rmin[TM + t])));
    return;
  }

  // Two image segments per dimension (P >= 256: one boundary at most per tile
  // dimension).  Tile rows [0, rsplit) are image rA, the rest image rA + 1 or padding;
  // columns likewise with csplit and cA.  Whether a pair is masked (same image, or
  // padding) depends only on the two segments, so minima are taken per segment over
  // the raw distances and a masked segment pair becomes +inf afterwards.  Each 64-row
  // half of the wave is reduced in one pass over its accumulators, as in the one-pair
  // case: with unit rows, only a half that the row boundary crosses sorts each distance
  // into the column minima of its row's segment, and only a wave that the column
  // boundary crosses sorts it into the row minima of its column's segment; with rows not
  // normalised every distance is sorted both ways (one variant: more of them left the
  // register allocator no room).  Sorting is a select per distance, so that a NaN
  // distance of a masked pair cannot reach an unmasked minimum.
  const int rsplit = min(TM, min((rA + 1) * p, rows) - row0);
  const int csplit = min(TM, min((cA + 1) * p, rows) - col0);
  const int rBimg = row0 + rsplit < rows ? rA + 1 : n;  // used only when segment B is not empty
  const int cBimg = col0 + csplit < rows ? cA + 1 : n;
  const bool mAA = rA == cA, mAB = cBimg == n || rA == cBimg;
  const bool mBA = rBimg == n || rBimg == cA, mBB = rBimg == n || cBimg == n || rBimg == cBimg;
  const bool colsplit = csplit > wc0 && csplit < wc0 + kWaveTile;  // the column boundary crosses this wave
  const bool colsA = csplit >= wc0 + kWaveTile;                    // otherwise: all its columns in segment A
  bool colB[kBlocks];
#pragma unroll
  for (int nb = 0; nb < kBlocks; ++nb) colB[nb] = wc0 + nb * 32 + lr >= csplit;
  // unit rows and columns (see the one-image-pair case): reduce the negated dots and
  // apply fma(2^-19, ., 2) to the results; a masked +inf stays +inf
  const float kUnit = 1.f / (float)(1 << kScaleShift);
  constexpr float kNegUnitScale = 2.f / (float)(1 << (2 * kScaleShift));
  bool unit = true;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int rr = wm * kWaveTile + k * 64 + lane, cc2 = wc0 + k * 64 + lane;
    unit = unit && s_rnorm[rr] == 1.f && s_rinv[rr] == kUnit && s_cnorm[cc2] == 1.f && s_cinv[cc2] == kUnit;
  }
  const bool unitw = __all(unit);
  float cminA[kBlocks], cminB[kBlocks];  // column minima per row segment, over both halves (masked below)
#pragma unroll
  for (int nb = 0; nb < kBlocks; ++nb) cminA[nb] = cminB[nb] = inf;
  float rmA[2], rmB[2];
  auto reduce_half = [&](auto h_c, auto unit_c, auto rowsplit_c, auto colsplit_c) {
    constexpr int h = decltype(h_c)::value;
    constexpr bool kUnitRows = decltype(unit_c)::value;
    constexpr bool kRowSplit = decltype(rowsplit_c)::value, kColSplit = decltype(colsplit_c)::value;
    const int wr0 = wm * kWaveTile + h * 64;  // this half's 64 rows
    float hA[kBlocks], hB[kBlocks];            // this half's column minima (per row segment when split)
#pragma unroll
    for (int nb = 0; nb < kBlocks; ++nb) hA[nb] = hB[nb] = inf;
    float rv[32], rvB[32];  // per row item: minimum over the columns (of segment A, B when split)
#pragma unroll
    for (int m2 = 0; m2 < 2; ++m2) {
      const int mb = 2 * h + m2;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float rnv[4] = {0.f, 0.f, 0.f, 0.f}, rs[4] = {0.f, 0.f, 0.f, 0.f};
        const int i0 = wr0 + m2 * 32 + g * 8 + lh * 4;
        if constexpr (!kUnitRows) {
          const float4 rn = *reinterpret_cast<const float4*>(&s_rnorm[i0]);
          const float4 ri = *reinterpret_cast<const float4*>(&s_rinv[i0]);
          rnv[0] = rn.x;
          rnv[1] = rn.y;
          rnv[2] = rn.z;
          rnv[3] = rn.w;
          rs[0] = -2.f * ri.x;  // -2 x row scale (exact)
          rs[1] = -2.f * ri.y;
          rs[2] = -2.f * ri.z;
          rs[3] = -2.f * ri.w;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool inB = i0 + e >= rsplit;
          float mA = inf, mB = inf;
#pragma unroll
          for (int nb = 0; nb < kBlocks; ++nb) {  // clamped at 0 by min_key, after the minima
            const float dot = acc[mb][nb][g * 4 + e];
            const float x = kUnitRows ? -dot : fmaf(rs[e] * ci[nb], dot, rnv[e] + cn[nb]);
            if constexpr (kRowSplit) {
              hA[nb] = nmin(hA[nb], inB ? inf : x);
              hB[nb] = nmin(hB[nb], inB ? x : inf);
            } else {
              hA[nb] = nmin(hA[nb], x);
            }
            if constexpr (kColSplit) {
              mA = nmin(mA, colB[nb] ? inf : x);
              mB = nmin(mB, colB[nb] ? x : inf);
            } else {
              mA = nmin(mA, x);
            }
          }
          rv[m2 * 16 + g * 4 + e] = mA;
          rvB[m2 * 16 + g * 4 + e] = mB;
        }
      }
    }
    // row wr0 + transposed_row(lr, lh): minima over the wave's 128 columns, per column segment
    float rowminA, rowminB;
    if constexpr (kColSplit) {
      rowminA = transpose_min32(rv, lr);
      rowminB = transpose_min32(rvB, lr);
    } else {
      const float m = transpose_min32(rv, lr);
      rowminA = colsA ? m : inf;
      rowminB = colsA ? inf : m;
    }
    // this half's column minima into the row segments' (a half the boundary does not
    // cross lies in one segment)
    const bool halfA = rsplit > wr0;
#pragma unroll
    for (int nb = 0; nb < kBlocks; ++nb) {
      if constexpr (kRowSplit) {
        cminA[nb] = nmin(cminA[nb], hA[nb]);
        cminB[nb] = nmin(cminB[nb], hB[nb]);
      } else {
        cminA[nb] = nmin(cminA[nb], halfA ? hA[nb] : inf);
        cminB[nb] = nmin(cminB[nb], halfA ? inf : hA[nb]);
      }
    }
    const bool rowInB = wr0 + transposed_row(lr, lh) >= rsplit;
    rmA[h] = (rowInB ? mBA : mAA) ? inf : rowminA;
    rmB[h] = (rowInB ? mBB : mAB) ? inf : rowminB;
    if constexpr (kUnitRows) {
      rmA[h] = fmaf(kNegUnitScale, rmA[h], 2.f);
      rmB[h] = fmaf(kNegUnitScale, rmB[h], 2.f);
    }
  };
  using F = std::false_type;
  using Tr = std::true_type;
  auto run_half = [&](auto h_c) {
    const int wr0 = wm * kWaveTile + decltype(h_c)::value * 64;
    const bool rowsplit = rsplit > wr0 && rsplit < wr0 + 64;  // the row boundary crosses this half
    if (unitw) {
      if (!rowsplit && !colsplit)
        reduce_half(h_c, Tr{}, F{}, F{});
      else if (!colsplit)
        reduce_half(h_c, Tr{}, Tr{}, F{});
      else if (!rowsplit)
        reduce_half(h_c, Tr{}, F{}, Tr{});
      else
        reduce_half(h_c, Tr{}, Tr{}, Tr{});
    } else {
      reduce_half(h_c, F{}, Tr{}, Tr{});  // rows not normalised: every distance selected
    }
  };
  run_half(std::integral_constant<int, 0>{});
  run_half(std::integral_constant<int, 1>{});
  // column wc0 + (2q + lh) * 32 + lr: minima over the wave's 128 rows, per row segment
  float cmA[2], cmB[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    cmA[q] = halves_min2(cminA[2 * q], cminA[2 * q + 1]);
    cmB[q] = halves_min2(cminB[2 * q], cminB[2 * q + 1]);
  }
  if (unitw) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      cmA[q] = fmaf(kNegUnitScale, cmA[q], 2.f);
      cmB[q] = fmaf(kNegUnitScale, cmB[q], 2.f);
    }
  }
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const bool colInB = wc0 + (2 * q + lh) * 32 + lr >= csplit;
    if (colInB ? mAB : mAA) cmA[q] = inf;
    if (colInB ? mBB : mBA) cmB[q] = inf;
  }
  __syncthreads();  // operand buffers are no longer read
  float* s_cminA = reinterpret_cast<float*>(smem);  // [2 (wm)][TM]
  float* s_cminB = s_cminA + 2 * TM;
  float* s_rminA = s_cminB + 2 * TM;                 // [2 (wn)][TM]
  float* s_rminB = s_rminA + 2 * TM;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    s_cminA[wm * TM + wc0 + (2 * q + lh) * 32 + lr] = cmA[q];
    s_cminB[wm * TM + wc0 + (2 * q + lh) * 32 + lr] = cmB[q];
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int rk = wm * kWaveTile + h * 64 + transposed_row(lr, lh);
    s_rminA[wn * TM + rk] = rmA[h];
    s_rminB[wn * TM + rk] = rmB[h];
  }
  __syncthreads();
  {
    const int cc = col0 + t;
    if (cc < rows) {
      // a segment with no pair of different images is exactly +inf (masked): skip it,
      // also because segment B may be the padding image n
      const float a = nmin(s_cminA[t], s_cminA[TM + t]);
      const float b = nmin(s_cminB[t], s_cminB[TM + t]);
      if (a != inf) atomicMin(minbits + (long long)cc * n + rA, min_key(a));
      if (b != inf) atomicMin(minbits + (long long)cc * n + rA + 1, min_key(b));
    }
  }
  {
    const int r = row0 + t;
    if (r < rows) {
      const float a = nmin(s_rminA[t], s_rminA[TM + t]);
      const float b = nmin(s_rminB[t], s_rminB[TM + t]);
      if (a != inf) atomicMin(minbits + (long long)r * n + cA, min_key(a));
      if (b != inf) atomicMin(minbits + (long long)r * n + cA + 1, min_key(b));
    }
  }
  }  // epilogue indices
}

inline int nkb_of(int c) { return (c + 2 * KB - 1) / (2 * KB) * 2; }

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
  if ((long long)TM * nkb_of(c) * ROWB > 0x7fffffffLL) return MUSC_ERR_UNSUPPORTED;
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
  const long long grid = (ntiles + kXcds - 1) / kXcds * kXcds;  // one workgroup per tile
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
