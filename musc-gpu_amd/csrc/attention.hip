// ViT block attention for gfx950: out = softmax(q k^T * scale) v, one pass with
// online softmax (the logits never reach HBM).
//
// Reference: nn.MultiheadAttention's math path inside
// models/backbone/open_clip/transformer.py:232-234 (bmm, softmax, bmm) and the
// fused row softmax of models/modules/_attention_gpu.py:41-81 (fp32 max/sum,
// fp16 storage).
//
// Layout trick: each wave computes S^T = K Q^T on fp32 MFMA
// (v_mfma_f32_32x32x2f32) so that a lane owns ONE query (lane % 32) and 16 of the
// 32 keys of a block in registers.  The row max / sum of the online softmax are
// then in-register reductions plus one cross-half exchange, the rescale of the
// running output is a per-lane scalar, and the probabilities already sit in the
// B-operand layout of the second product O^T += V^T P^T, so P never goes through
// LDS.  Blocks of 32 keys are staged in LDS and shared by the waves of a workgroup
// (fp32: 12 waves, 384 queries, one workgroup per CU; fp16: 4 waves, 128 queries).
#include <hip/hip_fp16.h>

#include <type_traits>

#include "common.hpp"

namespace musc {
namespace attn {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int D = 64;
constexpr int KB = 32;              // keys per block
constexpr int QW = 32;              // queries per wave
constexpr int WAVES = 4;
constexpr int KPITCH = D + 4;       // K block row pitch (floats)

// 2^x for the online softmax: the bare v_exp_f32 (about 1 ulp).  exp2f adds a
// rescaling path for results below 2^-126; the arguments here are <= 0 and such
// terms are far below what the fp32 sums and fp16 probabilities resolve, so that
// path (5 VALU instructions per exponential) is dropped.
__device__ inline float softmax_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
constexpr int VPITCH = KB + 4;      // V^T block row pitch (floats)
constexpr float kLazyLog2 = 8.f;    // running-maximum slack of the online softmax (exponentials <= 2^8)

// max / sum of a value and its partner 32 lanes away (the two halves of a wave hold
// the same query): v_permlane32_swap exchanges the halves in a VALU instruction, where
// a shuffle would go through LDS, and both swapped copies feed one symmetric operation.
__device__ inline float2 swap_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float halves_max(float v) {
  const float2 p = swap_halves(v);
  return fmaxf(p.x, p.y);
}
__device__ inline float halves_sum(float v) {
  const float2 p = swap_halves(v);
  return p.x + p.y;
}

// Where head bh = b * heads + h of a (batch, heads, t, 64) tensor lives: element
// (bh, row, d) is at b * sb + h * sh + row * st + d (strides in elements).  The
// contiguous (batch*heads, t, 64) layout is sb = heads*t*64, sh = t*64, st = 64; the
// packed in-projection output (t, batch, 3, heads, 64) of nn.MultiheadAttention is
// read in place with st = batch*3*heads*64, sb = 3*heads*64, sh = 64.
constexpr int kBufferFlags = 0x00020000;  // buffer resource word 3 for raw byte-addressed loads

// Forward work unit of workgroup blockIdx.x: (head, query tile), or x = -1 for the
// grid's padding.  Units are numbered head-major, so the query tiles of one head are
// consecutive logical ids, which xcd_logical_id places on one XCD: that XCD's L2 then
// serves the head's K and V blocks to all of its query tiles.
template <int kTile = QW * WAVES>  // queries per workgroup
__device__ inline int2 fwd_unit(int t, int nbh) {
  const int nqt = (t + kTile - 1) / kTile;
  const long long u = xcd_logical_id(blockIdx.x, gridDim.x);
  if (u >= (long long)nqt * nbh) return make_int2(-1, 0);
  return make_int2((int)(u / nqt), (int)(u % nqt));
}

struct HeadLayout {
  long long sb, sh, st;
  int heads;
  __device__ inline long long base(int bh) const { return (long long)(bh / heads) * sb + (long long)(bh % heads) * sh; }
};

template <int kDtype>
__device__ inline float4 ld4(const void* base, long long idx4) {
  if (kDtype == MUSC_DTYPE_F32) return reinterpret_cast<const float4*>(base)[idx4];
  const uint2 raw = reinterpret_cast<const uint2*>(base)[idx4];
  const float2 a = __half22float2(*reinterpret_cast<const __half2*>(&raw.x));
  const float2 b = __half22float2(*reinterpret_cast<const __half2*>(&raw.y));
  return make_float4(a.x, a.y, b.x, b.y);
}

template <int kDtype>
__device__ inline void st4(void* base, long long idx4, float4 v) {
  if (kDtype == MUSC_DTYPE_F32) {
    reinterpret_cast<float4*>(base)[idx4] = v;
  } else {
    __half2 lo = __floats2half2_rn(v.x, v.y), hi = __floats2half2_rn(v.z, v.w);
    uint2 raw;
    raw.x = *reinterpret_cast<uint32_t*>(&lo);
    raw.y = *reinterpret_cast<uint32_t*>(&hi);
    reinterpret_cast<uint2*>(base)[idx4] = raw;
  }
}

__device__ inline void store_kv_row(float* __restrict__ Ks, float* __restrict__ Vt, int idx, float4 kv, float4 vv) {
  const int key = idx / (D / 4), d4 = (idx % (D / 4)) * 4;
  *reinterpret_cast<float4*>(&Ks[key * KPITCH + d4]) = kv;
  Vt[(d4 + 0) * VPITCH + key] = vv.x;
  Vt[(d4 + 1) * VPITCH + key] = vv.y;
  Vt[(d4 + 2) * VPITCH + key] = vv.z;
  Vt[(d4 + 3) * VPITCH + key] = vv.w;
}

// The fp32 kernel runs one 12-wave workgroup (384 queries, 3 waves per SIMD) per CU
// rather than three 4-wave ones: the wave arbiter favours the oldest waves, so of three
// workgroups sharing a CU one finishes first and the last runs its final blocks alone,
// with too few waves to keep the MFMA pipe busy; the barrier keeps 12 waves in step.
constexpr int WAVES32 = 12;
__global__ __launch_bounds__(WAVES32 * kWave, 1) void attn_fwd_kernel(const float* __restrict__ qg,
                                                                 const float* __restrict__ kg,
                                                                 const float* __restrict__ vg,
                                                                 float* __restrict__ og, int t, float scale_log2,
                                                                 HeadLayout in, HeadLayout out, int nbh) {
  __shared__ __attribute__((aligned(16))) float Ks[2][KB * KPITCH];
  __shared__ __attribute__((aligned(16))) float Vt[2][D * VPITCH];

  const int2 unit = fwd_unit<QW * WAVES32>(t, nbh);
  if (unit.x < 0) return;
  const int bh = unit.x;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int lq = lane & 31, lh = lane >> 5;
  const int q = unit.y * (QW * WAVES32) + wave * QW + lq;
  // waves whose 32 queries all lie past t only stage and synchronise
  const bool active = unit.y * (QW * WAVES32) + wave * QW < t;
  const long long head = in.base(bh), st = in.st;

  // This lane's query row, pre-scaled by scale*log2(e): qr[s][j] = q[8s + 4h + j].
  float qr[8][4];
  {
    const bool ok = q < t;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      float4 v = ok ? *reinterpret_cast<const float4*>(qg + head + (long long)q * st + 8 * s + 4 * lh)
                    : make_float4(0.f, 0.f, 0.f, 0.f);
      qr[s][0] = v.x * scale_log2;
      qr[s][1] = v.y * scale_log2;
      qr[s][2] = v.z * scale_log2;
      qr[s][3] = v.w * scale_log2;
    }
  }

  floatx16 o0, o1;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    o0[v] = 0.f;
    o1[v] = 0.f;
  }
  float m = -INFINITY, l = 0.f;

  const int nkb = (t + KB - 1) / KB;
  // K / V^T staging: threads 0-511 each move element idx = tid of each 32-key block (key
  // idx/16, channels 4*(idx%16)) of K and of V, loaded one block ahead; the LDS
  // copy is double-buffered, so one barrier per block suffices.  The loads go through
  // a buffer resource based at the block's first key whose extent ends with the last
  // valid key, so a key past t reads zeros and each thread's byte offset within the
  // block is loop-invariant: no address arithmetic or bounds test per block.
  const bool stager = threadIdx.x < KB * D / 4;  // waves 0-7: one float4 of K and one of V each
  const int i0 = threadIdx.x & (KB * D / 4 - 1);
  const uint32_t vo0 = (uint32_t)(((long long)(i0 / (D / 4)) * st + 4 * (i0 % (D / 4))) * 4);
  auto block_rsrc = [&](const float* src, int kb) {
    const long long rem = min(t - kb * KB, KB);  // valid keys of the block, >= 1
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(src + head + (long long)kb * KB * st), (short)0,
                                             (int)(((rem - 1) * st + D) * 4), kBufferFlags);
  };
  auto ldkv = [&](__amdgpu_buffer_rsrc_t r, uint32_t vo) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)vo, 0, 0));
  };
  float4 k0 = {}, v0 = {};
  if (stager) {
    const __amdgpu_buffer_rsrc_t rk = block_rsrc(kg, 0), rv = block_rsrc(vg, 0);
    k0 = ldkv(rk, vo0);
    v0 = ldkv(rv, vo0);
  }
  for (int kb = 0; kb < nkb; ++kb) {
    const int buf = kb & 1;
    if (stager) {
      store_kv_row(Ks[buf], Vt[buf], i0, k0, v0);
      // the block after the last is loaded again as the last block (never stored)
      const int nb = min(kb + 1, nkb - 1);
      const __amdgpu_buffer_rsrc_t rk = block_rsrc(kg, nb), rv = block_rsrc(vg, nb);
      k0 = ldkv(rk, vo0);
      v0 = ldkv(rv, vo0);
    }
    __syncthreads();
    if (!active) continue;

    // S^T (keys x queries), already in log2 units
    floatx16 s;
#pragma unroll
    for (int v = 0; v < 16; ++v) s[v] = 0.f;
    const float* krow = &Ks[buf][lq * KPITCH + 4 * lh];
#pragma unroll
    for (int ss = 0; ss < 8; ++ss) {
      const float4 a = *reinterpret_cast<const float4*>(krow + 8 * ss);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, qr[ss][0], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, qr[ss][1], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, qr[ss][2], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, qr[ss][3], s, 0, 0, 0);
    }
    // register v holds key (v/4)*8 + 4h + v%4 of the block; only the last block is ragged
    if ((kb + 1) * KB > t) {
#pragma unroll
      for (int v = 0; v < 16; ++v)
        if (kb * KB + (v >> 2) * 8 + lh * 4 + (v & 3) >= t) s[v] = -INFINITY;
    }
    float bmax = s[0];
#pragma unroll
    for (int v = 1; v < 16; ++v) bmax = fmaxf(bmax, s[v]);
    bmax = halves_max(bmax);
    // lazy rescaling, as in the fp16 kernel: the running maximum moves only past kLazyLog2
    if (!__all(bmax <= m + kLazyLog2)) {
      const float mnew = fmaxf(m, bmax);
      const float alpha = softmax_exp2(m - mnew);  // 0 on the first block (m = -inf)
      l *= alpha;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        o0[v] *= alpha;
        o1[v] *= alpha;
      }
      m = mnew;
    }
    float psum = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      s[v] = softmax_exp2(s[v] - m);
      psum += s[v];
    }
    psum = halves_sum(psum);
    l += psum;
    // O^T += V^T P^T ; step e uses key 8*(e/4) + 4h + e%4 = register e of s
    const float* vrow0 = &Vt[buf][lq * VPITCH + 4 * lh];
    const float* vrow1 = &Vt[buf][(32 + lq) * VPITCH + 4 * lh];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 a0 = *reinterpret_cast<const float4*>(vrow0 + 8 * j);
      const float4 a1 = *reinterpret_cast<const float4*>(vrow1 + 8 * j);
      o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.x, s[4 * j + 0], o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.x, s[4 * j + 0], o1, 0, 0, 0);
      o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.y, s[4 * j + 1], o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.y, s[4 * j + 1], o1, 0, 0, 0);
      o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.z, s[4 * j + 2], o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.z, s[4 * j + 2], o1, 0, 0, 0);
      o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.w, s[4 * j + 3], o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.w, s[4 * j + 3], o1, 0, 0, 0);
    }
  }

  if (q < t) {
    const float inv = 1.f / l;
    // register v of tile dt holds d = 32*dt + (v/4)*8 + 4h + v%4
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 a = make_float4(o0[4 * g] * inv, o0[4 * g + 1] * inv, o0[4 * g + 2] * inv, o0[4 * g + 3] * inv);
      const float4 b = make_float4(o1[4 * g] * inv, o1[4 * g + 1] * inv, o1[4 * g + 2] * inv, o1[4 * g + 3] * inv);
      float* orow = og + out.base(bh) + (long long)q * out.st;
      *reinterpret_cast<float4*>(orow + 8 * g + 4 * lh) = a;
      *reinterpret_cast<float4*>(orow + 32 + 8 * g + 4 * lh) = b;
    }
  }
}

// fp16 storage on fp16 MFMA (v_mfma_f32_32x32x16_f16): same S^T = K Q^T layout as
// the fp32 kernel, four MFMAs per 32-key block for S (K = d = 64) and two per
// 32-wide d tile for O^T += V^T P^T, with P rounded to fp16 (the reference feeds
// fp16 probabilities to its second bmm, models/modules/_attention_gpu.py:141-146).
// The softmax statistics stay fp32.  For MFMA m, lane half h, element j the
// reduction index is k = 16m + 8h + j in S and key 16m + 8(j/4) + 4h + j%4 in
// P V, which is exactly where register 8m + j of the S^T tile holds that key.
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((ext_vector_type(4)));
constexpr int KP16 = D + 8;        // K block pitch (halves): 144 B rows
constexpr int VR16 = D + 8;        // V block pitch (halves), row-major: 144 B rows

__global__ __launch_bounds__(WAVES * kWave) void attn_fwd_f16_kernel(const _Float16* __restrict__ qg,
                                                                     const _Float16* __restrict__ kg,
                                                                     const _Float16* __restrict__ vg,
                                                                     _Float16* __restrict__ og, int t,
                                                                     float scale_log2, HeadLayout in,
                                                                     HeadLayout out, int nbh) {
  __shared__ __attribute__((aligned(16))) _Float16 Ks[2][KB * KP16];
  __shared__ __attribute__((aligned(16))) _Float16 Vs[2][KB * VR16];

  const int2 unit = fwd_unit(t, nbh);
  if (unit.x < 0) return;
  const int bh = unit.x;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int lq = lane & 31, lh = lane >> 5;
  const int q = unit.y * (QW * WAVES) + wave * QW + lq;
  const long long head = in.base(bh), st = in.st;

  half8 qf[4];
  {
    const bool ok = q < t;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      half8 v = {};
      if (ok) v = *reinterpret_cast<const half8*>(qg + head + (long long)q * st + 16 * m + 8 * lh);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = (_Float16)((float)v[j] * scale_log2);
      qf[m] = v;
    }
  }

  floatx16 o0, o1;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    o0[v] = 0.f;
    o1[v] = 0.f;
  }
  // m_run: running maximum of this lane's query (the same in both halves of the wave);
  // l_run: this half-wave's share of the probability sum (the halves' shares are added
  // once, after the key loop)
  float m_run = -INFINITY, l_run = 0.f;

  const int nkb = (t + KB - 1) / KB;
  const int tid = threadIdx.x;
  // staging: thread tid moves row tid/8, halves 8*(tid%8).. (16 B) of a K block and of a
  // V block; both are stored row-major in LDS
  const int skey = tid / 8, sd8 = (tid % 8) * 8;
  // loads through a buffer resource based at the block's first key whose extent ends
  // with the last valid key: keys past t read zeros, offsets are loop-invariant; the
  // extent of a full block (all KB keys valid) is loop-invariant too
  const uint32_t vo = (uint32_t)(((long long)skey * st + sd8) * 2);
  const int full_extent = (int)(((long long)(KB - 1) * st + D) * 2);
  auto block_rsrc = [&](const _Float16* src, int kb, auto full_c) {
    const int extent = decltype(full_c)::value ? full_extent
                                               : (int)(((long long)(min(t - kb * KB, KB) - 1) * st + D) * 2);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(src + head + (long long)kb * KB * st), (short)0,
                                             extent, kBufferFlags);
  };
  auto load_block = [&](const _Float16* src, int kb, auto full_c) -> half8 {
    return __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(block_rsrc(src, kb, full_c), (int)vo, 0, 0));
  };
  using Whole = std::integral_constant<bool, true>;
  using Part = std::integral_constant<bool, false>;
  auto store_k = [&](int buf, half8 r) { *reinterpret_cast<half8*>(&Ks[buf][skey * KP16 + sd8]) = r; };
  auto store_v = [&](int buf, half8 r) { *reinterpret_cast<half8*>(&Vs[buf][skey * VR16 + sd8]) = r; };

  // S^T of one staged key block (4 MFMAs over d = 64) plus one MFMA that adds -base to
  // every logit: the A operand's k column 0 is 1 for every key, the B operand's k row 0
  // holds -base for every query (this lane's running maximum as of the issue).  The
  // logits come out shifted, so the softmax needs no subtraction per logit; base is an
  // integer of at most 2048 in magnitude (exact in fp16) or 0.
  half8 ones_col = {};
  ones_col[0] = lh == 0 ? (_Float16)1.f : (_Float16)0.f;
  // The running maximum is kept an integer while |m_run| <= 2048 (raised to the next
  // integer, which only lowers the exponentials), so that it is exact as an fp16 base.
  constexpr float kBaseLimit = 2048.f;
  // base of the next logits and the B operand of the shift MFMA for it; both change
  // only where m_run does
  float cur_base = 0.f;
  half8 shift_row = {};
  auto set_base = [&]() {
    cur_base = fabsf(m_run) <= kBaseLimit ? m_run : 0.f;  // -inf -> 0
    shift_row[0] = lh == 0 ? (_Float16)(-cur_base) : (_Float16)0.f;
  };
  auto read_k = [&](int buf, half8 (&kf)[4]) {
#pragma unroll
    for (int m = 0; m < 4; ++m) kf[m] = *reinterpret_cast<const half8*>(&Ks[buf][lq * KP16 + 16 * m + 8 * lh]);
  };
  auto logits = [&](const half8 (&kf)[4]) -> floatx16 {
    floatx16 r;
#pragma unroll
    for (int v = 0; v < 16; ++v) r[v] = 0.f;
    r = __builtin_amdgcn_mfma_f32_32x32x16_f16(ones_col, shift_row, r, 0, 0, 0);
#pragma unroll
    for (int m = 0; m < 4; ++m) r = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[m], qf[m], r, 0, 0, 0);
    return r;
  };
  // V^T fragments of block j: vf[2 mm] feeds o0 (d 0..31), vf[2 mm + 1] feeds o1 (d 32..63).
  // ds_read_b64_tr_b16 transposes within each group of 16 lanes: lane i's element j is
  // element i % 4 of the 8 bytes that lane 4 j + i / 4 of the group addressed.  With V
  // row-major in LDS, the lane (r = lq % 16 of its group) that addresses V[key0 + r / 4]
  // [d0 + 4 (r % 4) ..] hands element j of lane i the value V[key0 + j][d0 + i], which is
  // the A operand's (row d0 + i, k = j) for key0 = 16 mm + 4 lh (elements 0..3) and
  // 16 mm + 8 + 4 lh (elements 4..7), d0 = 16 (lq / 16) (+ 32 for o1).
  const int vrd = (4 * lh + ((lq & 15) >> 2)) * VR16 + 16 * (lq >> 4) + 4 * (lq & 3);
  auto read_v = [&](int j, half8 (&vf)[4]) {
    const _Float16* vb = &Vs[j & 1][vrd];
    auto tr = [&](int off) {
      typedef __attribute__((address_space(3))) short4v lds_short4v;
      return __builtin_bit_cast(half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)(vb + off)));
    };
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
#pragma unroll
      for (int o = 0; o < 2; ++o) {
        const half4 lo = tr(16 * mm * VR16 + 32 * o), hi = tr((16 * mm + 8) * VR16 + 32 * o);
        vf[2 * mm + o] = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    }
  };

  // Three-stage software pipeline over 32-key blocks.  Step kb issues the logits MFMAs
  // of block kb+2 and the P V MFMAs of block kb and computes the exponentials of block
  // kb+1 on the VALU: within a step the matrix work waits only for its LDS reads, never
  // for the exponentials, so a wave keeps MFMAs in flight while its softmax runs (this
  // kernel has only ~2.75 waves per SIMD to hide latency).  The branchy part of a
  // block's softmax (block maximum, lazy rescale, re-base: part_a) runs at the end of
  // the step that issued its logits.  A rescale there also scales the fp16
  // probabilities of the previous block, whose P V product is still to come (the
  // factor is a power of two while |m_run| <= 2048, so that scaling is exact); each
  // block's probability sum enters l_run with its P V product.  Block j's K sits in
  // Ks[j & 1] from the top of step j - 2, its V in Vs[j & 1] from the top of step j;
  // every buffer is rewritten two barriers after its last read.
  typedef _Float16 half2v __attribute__((ext_vector_type(2)));
  auto part_a = [&](int j, floatx16& s, float base, half8 (&pf_prev)[2], auto check_c) {
    if (decltype(check_c)::value && (j + 1) * KB > t) {  // only the last block is ragged
#pragma unroll
      for (int v = 0; v < 16; ++v)
        if (j * KB + (v >> 2) * 8 + lh * 4 + (v & 3) >= t) s[v] = -INFINITY;
    }
    // IEEE maximum: NaN-propagating, one v_maximum3_f32 per two logits
    float bmax = s[0];
#pragma unroll
    for (int v = 1; v < 16; ++v) bmax = __builtin_elementwise_maximum(bmax, s[v]);
    {
      const float2 p = swap_halves(bmax);
      bmax = __builtin_elementwise_maximum(p.x, p.y) + base;  // this block's maximum logit
    }
    // lazy rescaling (see kLazyLog2)
    if (!__all(bmax <= m_run + kLazyLog2)) {
      float mnew = fmaxf(m_run, bmax);
      if (fabsf(mnew) <= kBaseLimit) mnew = ceilf(mnew);
      const float alpha = softmax_exp2(m_run - mnew);  // 0 on the first block (m_run = -inf)
      l_run *= alpha;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        o0[v] *= alpha;
        o1[v] *= alpha;
      }
      const _Float16 ah = (_Float16)alpha;
      pf_prev[0] *= ah;
      pf_prev[1] *= ah;
      m_run = mnew;
      set_base();
    }
    // re-base the logits when the running maximum moved since they were issued (the
    // rescale above, and every block once |m_run| > 2048)
    const float shift = base - m_run;
    if (__any(shift != 0.f)) {
#pragma unroll
      for (int v = 0; v < 16; ++v) s[v] += shift;
    }
  };
  auto part_b = [&](const floatx16& s, half8 (&pf)[2]) {
#pragma unroll
    for (int v = 0; v < 16; ++v) pf[v >> 3][v & 7] = (_Float16)softmax_exp2(s[v]);
  };
  auto pv = [&](const half8 (&vf)[4], const half8 (&pf)[2]) {
    // this half-wave's share of the row sum of the fp16 probabilities the product uses,
    // two at a time in fp32
    const half2v ones = {(_Float16)1.f, (_Float16)1.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      l_run = __builtin_amdgcn_fdot2(half2v{pf[0][2 * i], pf[0][2 * i + 1]}, ones, l_run, false);
      l_run = __builtin_amdgcn_fdot2(half2v{pf[1][2 * i], pf[1][2 * i + 1]}, ones, l_run, false);
    }
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
      o0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[2 * mm], pf[mm], o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[2 * mm + 1], pf[mm], o1, 0, 0, 0);
    }
  };
  using Check = std::integral_constant<bool, true>;
  using NoCheck = std::integral_constant<bool, false>;

  // prologue: logits of blocks 0 and 1, exponentials of block 0; K(2) and V(0) in the
  // staging registers
  half8 kreg = load_block(kg, 0, Part{});
  store_k(0, kreg);
  if (nkb > 1) kreg = load_block(kg, 1, Part{});
  __syncthreads();
  set_base();
  float base_a = cur_base, base_b = 0.f;
  floatx16 sa, sb;
  {
    half8 kf[4];
    read_k(0, kf);
    sa = logits(kf);
  }
  half8 pfa[2] = {}, pfb[2] = {};
  part_a(0, sa, base_a, pfb, Check{});  // pfb is all zeros here
  if (nkb > 1) store_k(1, kreg);
  if (nkb > 2) kreg = load_block(kg, 2, Part{});
  half8 vreg = load_block(vg, 0, Part{});
  __syncthreads();
  if (nkb > 1) {
    base_b = cur_base;
    half8 kf[4];
    read_k(1, kf);
    sb = logits(kf);
  }
  part_b(sa, pfa);
  if (nkb > 1) part_a(1, sb, base_b, pfa, Check{});

  // step kb: logits of block kb+2 into s_new, P V of block kb with pf_use, exponentials
  // of block kb+1 (held in s_next) into pf_make.  kFull: every block named exists and
  // the blocks loaded are full.  Steps alternate between two register sets (no copies).
  auto step = [&](int kb, floatx16& s_new, float& b_new, const floatx16& s_next, half8 (&pf_use)[2],
                  half8 (&pf_make)[2], auto full_c) {
    constexpr bool kFull = decltype(full_c)::value;
    if (kFull || kb + 2 < nkb) store_k(kb & 1, kreg);
    store_v(kb & 1, vreg);
    if (kFull || kb + 3 < nkb) kreg = load_block(kg, kb + 3, std::integral_constant<bool, kFull>{});
    if (kFull || kb + 1 < nkb) vreg = load_block(vg, kb + 1, std::integral_constant<bool, kFull>{});
    __syncthreads();
    half8 kf[4], vf[4];
    if (kFull || kb + 2 < nkb) read_k(kb & 1, kf);
    read_v(kb, vf);
    if (kFull || kb + 2 < nkb) {
      b_new = cur_base;
      s_new = logits(kf);
    }
    pv(vf, pf_use);
    if (kFull || kb + 1 < nkb) part_b(s_next, pf_make);
    if constexpr (kFull) {
      part_a(kb + 2, s_new, b_new, pf_make, NoCheck{});
    } else {
      if (kb + 2 < nkb) part_a(kb + 2, s_new, b_new, pf_make, Check{});
    }
  };
  // A pair of whole steps loads K blocks kb+3, kb+4 and V blocks kb+1, kb+2 with the
  // full-block extent and skips the ragged mask on blocks kb+2, kb+3: it runs only while
  // all of them are full blocks (kb + 4 < t / KB), so a ragged last block always takes
  // the checked steps below and no load reads past key t - 1.
  const int nfull = t / KB;
  int kb = 0;
  for (; kb + 4 < nfull; kb += 2) {
    step(kb, sa, base_a, sb, pfa, pfb, Whole{});
    step(kb + 1, sb, base_b, sa, pfb, pfa, Whole{});
  }
  for (; kb < nkb; kb += 2) {
    step(kb, sa, base_a, sb, pfa, pfb, Part{});
    if (kb + 1 < nkb) step(kb + 1, sb, base_b, sa, pfb, pfa, Part{});
  }

  l_run = halves_sum(l_run);
  if (q < t) {
    const float inv = 1.f / l_run;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 a = make_float4(o0[4 * g] * inv, o0[4 * g + 1] * inv, o0[4 * g + 2] * inv, o0[4 * g + 3] * inv);
      const float4 b = make_float4(o1[4 * g] * inv, o1[4 * g + 1] * inv, o1[4 * g + 2] * inv, o1[4 * g + 3] * inv);
      const long long orow = out.base(bh) + (long long)q * out.st;
      st4<MUSC_DTYPE_F16>(og, (orow + 8 * g + 4 * lh) / 4, a);
      st4<MUSC_DTYPE_F16>(og, (orow + 32 + 8 * g + 4 * lh) / 4, b);
    }
  }
}

// Head-averaged attention probabilities, for the one block whose weights the
// caller reads (models/backbone/open_clip/transformer.py:331-333, averaged by
// nn.MultiheadAttention over heads): weights[b, i, j] = mean_h softmax_j(scale *
// q[b,h,i] . k[b,h,j]), fp32 logits and probabilities.
//
// Two passes on MFMA, both in the S^T = K Q^T layout (lane owns one query):
//   attn_wstats_kernel    one wave per (batch*head, 32 queries): running max and
//                         sum over all key blocks -> (max, 1/sum) per query, in
//                         the exp2 domain with the scale folded in.
//   attn_weights_kernel   one wave per (batch, 32 queries, kKR key blocks): for
//                         every head recomputes the logits of its key blocks,
//                         adds exp2(s - max) / sum into registers, then writes
//                         the averaged rows through an LDS transpose (each store
//                         instruction covers two 128-byte query-row segments).
// fp16 inputs use v_mfma_f32_32x32x16_f16 (products exact, fp32 accumulation);
// fp32 inputs use v_mfma_f32_32x32x2f32 with the same reduction-index split as
// attn_fwd_kernel.
template <int kDtype>
struct QFrag;
template <>
struct QFrag<MUSC_DTYPE_F16> {
  half8 v[4];
};
template <>
struct QFrag<MUSC_DTYPE_F32> {
  float4 v[8];
};

// Fragment of row `row` (zeros when row >= t) of a (t, 64) head matrix for lane
// half lh: fp16 -> halves 16m + 8lh .. +7 for m = 0..3; fp32 -> floats 8s + 4lh ..
// +3 for s = 0..7.
template <int kDtype>
__device__ inline QFrag<kDtype> load_frag(const void* base, long long head, long long st, int row, int t, int lh) {
  QFrag<kDtype> f;
  const bool ok = row < t;
  if constexpr (kDtype == MUSC_DTYPE_F16) {
    const _Float16* p = static_cast<const _Float16*>(base) + head + (long long)row * st + 8 * lh;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      half8 v = {};
      if (ok) v = *reinterpret_cast<const half8*>(p + 16 * m);
      f.v[m] = v;
    }
  } else {
    const float* p = static_cast<const float*>(base) + head + (long long)row * st + 4 * lh;
#pragma unroll
    for (int s = 0; s < 8; ++s) f.v[s] = ok ? *reinterpret_cast<const float4*>(p + 8 * s) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  return f;
}

// S^T tile (32 keys x 32 queries) of one key block: lane (lq, lh) gets query lq and
// keys (v/4)*8 + 4lh + v%4 of the block.
template <int kDtype>
__device__ inline floatx16 logits_t(const QFrag<kDtype>& kf, const QFrag<kDtype>& qf) {
  floatx16 s;
#pragma unroll
  for (int v = 0; v < 16; ++v) s[v] = 0.f;
  if constexpr (kDtype == MUSC_DTYPE_F16) {
#pragma unroll
    for (int m = 0; m < 4; ++m) s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf.v[m], qf.v[m], s, 0, 0, 0);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.v[j].x, qf.v[j].x, s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.v[j].y, qf.v[j].y, s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.v[j].z, qf.v[j].z, s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.v[j].w, qf.v[j].w, s, 0, 0, 0);
    }
  }
  return s;
}

// grid (ceil(t/32), batch*heads), one wave.  stats[bh*t + i] = (max, 1/sum).
template <int kDtype>
__global__ __launch_bounds__(kWave) void attn_wstats_kernel(const void* __restrict__ qg, const void* __restrict__ kg,
                                                            int t, float scale_log2, HeadLayout in,
                                                            float2* __restrict__ stats) {
  const int bh = blockIdx.y;
  const int lane = threadIdx.x, lq = lane & 31, lh = lane >> 5;
  const int query = blockIdx.x * 32 + lq;
  const long long head = in.base(bh), st = in.st;
  const QFrag<kDtype> qf = load_frag<kDtype>(qg, head, st, query, t, lh);
  const int nkb = (t + KB - 1) / KB;
  float m_run = -INFINITY, l_run = 0.f;
  QFrag<kDtype> kf = load_frag<kDtype>(kg, head, st, lq, t, lh);
  for (int kb = 0; kb < nkb; ++kb) {
    floatx16 s = logits_t<kDtype>(kf, qf);
    if (kb + 1 < nkb) kf = load_frag<kDtype>(kg, head, st, (kb + 1) * KB + lq, t, lh);
#pragma unroll
    for (int v = 0; v < 16; ++v) s[v] *= scale_log2;
    if ((kb + 1) * KB > t) {
#pragma unroll
      for (int v = 0; v < 16; ++v)
        if (kb * KB + (v >> 2) * 8 + lh * 4 + (v & 3) >= t) s[v] = -INFINITY;
    }
    float bmax = s[0];
#pragma unroll
    for (int v = 1; v < 16; ++v) bmax = fmaxf(bmax, s[v]);
    bmax = halves_max(bmax);
    const float mnew = fmaxf(m_run, bmax);
    float psum = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) psum += exp2f(s[v] - mnew);
    psum = halves_sum(psum);
    l_run = l_run * exp2f(m_run - mnew) + psum;
    m_run = mnew;
  }
  if (lh == 0 && query < t) stats[(long long)bh * t + query] = make_float2(m_run, 1.f / l_run);
}

// grid (ceil(t/32), ceil(nkb/kKR), batch), one wave.
template <int kDtype, int kKR>
__global__ __launch_bounds__(kWave) void attn_weights_kernel(const void* __restrict__ qg, const void* __restrict__ kg,
                                                             int heads, int t, float scale_log2, HeadLayout in,
                                                             const float2* __restrict__ stats,
                                                             float* __restrict__ weights) {
  __shared__ float tile[32][33];
  const int b = blockIdx.z;
  const int lane = threadIdx.x, lq = lane & 31, lh = lane >> 5;
  const int q0 = blockIdx.x * 32, query = q0 + lq;
  const int nkb = (t + KB - 1) / KB;
  const int kb0 = blockIdx.y * kKR;
  const int nr = min(kKR, nkb - kb0);
  floatx16 acc[kKR];
#pragma unroll
  for (int r = 0; r < kKR; ++r)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[r][v] = 0.f;
  for (int h = 0; h < heads; ++h) {
    const long long head = in.base(b * heads + h), st = in.st;
    const QFrag<kDtype> qf = load_frag<kDtype>(qg, head, st, query, t, lh);
    float mx = 0.f, il = 0.f;  // rows past t contribute nothing and are not written
    if (query < t) {
      const float2 st = stats[((long long)b * heads + h) * t + query];
      mx = st.x;
      il = st.y;
    }
#pragma unroll
    for (int r = 0; r < kKR; ++r) {
      if (r < nr) {
        const int kb = kb0 + r;
        const QFrag<kDtype> kf = load_frag<kDtype>(kg, head, st, kb * KB + lq, t, lh);
        const floatx16 s = logits_t<kDtype>(kf, qf);
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[r][v] += softmax_exp2(s[v] * scale_log2 - mx) * il;
      }
    }
  }
  const float inv_h = 1.f / (float)heads;
#pragma unroll
  for (int r = 0; r < kKR; ++r) {
    if (r < nr) {
      const int kb = kb0 + r;
      // tile[query][key] from the S^T registers, then 32 consecutive keys of two
      // query rows per store instruction
#pragma unroll
      for (int v = 0; v < 16; ++v) tile[lq][(v >> 2) * 8 + lh * 4 + (v & 3)] = acc[r][v] * inv_h;
      __syncthreads();
      const int key = kb * KB + lq;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = 2 * i + lh;
        if (q0 + row < t && key < t) weights[((long long)b * t + q0 + row) * t + key] = tile[row][lq];
      }
      __syncthreads();
    }
  }
}

}  // namespace attn
}  // namespace musc

using namespace musc;

namespace {

// Strides must keep every 16-byte vector access aligned and be non-negative.
inline bool layout_ok(const attn::HeadLayout& l, int dtype) {
  const long long unit = dtype == MUSC_DTYPE_F32 ? 4 : 8;
  return l.sb >= 0 && l.sh >= 0 && l.st >= attn::D && l.sb % unit == 0 && l.sh % unit == 0 && l.st % unit == 0;
}

int attention_fwd(const void* q, const void* k, const void* v, void* out, int dtype, int batch, int heads, int t,
                  int d, const attn::HeadLayout& in, const attn::HeadLayout& ol, float scale, hipStream_t stream) {
  if (!q || !k || !v || !out || batch < 1 || heads < 1 || t < 1) return MUSC_ERR_INVALID_ARG;
  if (dtype != MUSC_DTYPE_F32 && dtype != MUSC_DTYPE_F16) return MUSC_ERR_INVALID_ARG;
  if (d != attn::D) return MUSC_ERR_UNSUPPORTED;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
       reinterpret_cast<uintptr_t>(out)) % 16)
    return MUSC_ERR_INVALID_ARG;
  if (!layout_ok(in, dtype) || !layout_ok(ol, dtype)) return MUSC_ERR_INVALID_ARG;
  if ((long long)batch * heads > 65535) return MUSC_ERR_UNSUPPORTED;
  // K/V blocks are read through buffer resources whose extent and per-thread offsets are
  // 32-bit byte counts: a block of KB rows must span less than 2 GiB
  const long long elem = dtype == MUSC_DTYPE_F32 ? 4 : 2;
  if (((long long)(attn::KB - 1) * in.st + attn::D) * elem > 0x7fffffffLL) return MUSC_ERR_UNSUPPORTED;
  const float scale_log2 = scale * 1.4426950408889634f;
  const int nbh = batch * heads;
  const int tile = dtype == MUSC_DTYPE_F32 ? attn::QW * attn::WAVES32 : attn::QW * attn::WAVES;
  const long long units = (long long)((t + tile - 1) / tile) * nbh;
  const dim3 grid((unsigned)align_up((size_t)units, kXcds));
  if (dtype == MUSC_DTYPE_F32)
    hipLaunchKernelGGL(attn::attn_fwd_kernel, grid, dim3(attn::WAVES32 * kWave), 0, stream,
                       static_cast<const float*>(q), static_cast<const float*>(k), static_cast<const float*>(v),
                       static_cast<float*>(out), t, scale_log2, in, ol, nbh);
  else
    hipLaunchKernelGGL(attn::attn_fwd_f16_kernel, grid, dim3(attn::WAVES * kWave), 0, stream,
                       static_cast<const _Float16*>(q), static_cast<const _Float16*>(k),
                       static_cast<const _Float16*>(v), static_cast<_Float16*>(out), t, scale_log2, in, ol, nbh);
  return check_launch();
}

int attention_weights(const void* q, const void* k, int dtype, int batch, int heads, int t, int d,
                      const attn::HeadLayout& in, float scale, float* weights, void* workspace,
                      size_t workspace_bytes, hipStream_t stream) {
  if (!q || !k || !weights || batch < 1 || heads < 1 || t < 1) return MUSC_ERR_INVALID_ARG;
  if (dtype != MUSC_DTYPE_F32 && dtype != MUSC_DTYPE_F16) return MUSC_ERR_INVALID_ARG;
  if (d != attn::D) return MUSC_ERR_UNSUPPORTED;
  if (((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k)) % 16) != 0) return MUSC_ERR_INVALID_ARG;
  if (!layout_ok(in, dtype)) return MUSC_ERR_INVALID_ARG;
  if (batch > 65535 || (long long)batch * heads > 65535) return MUSC_ERR_UNSUPPORTED;
  const size_t need = align_up((size_t)batch * heads * t * sizeof(float2), 256);
  if (!workspace || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) % 8) != 0)
    return MUSC_ERR_WORKSPACE;
  float2* stats = static_cast<float2*>(workspace);
  const float scale_log2 = scale * 1.4426950408889634f;
  const int nqb = (t + 31) / 32, nkb = (t + attn::KB - 1) / attn::KB;
  const dim3 sgrid(nqb, batch * heads);
  if (dtype == MUSC_DTYPE_F32) {
    constexpr int kKR = 4;
    hipLaunchKernelGGL(attn::attn_wstats_kernel<MUSC_DTYPE_F32>, sgrid, dim3(kWave), 0, stream, q, k, t, scale_log2,
                       in, stats);
    hipLaunchKernelGGL((attn::attn_weights_kernel<MUSC_DTYPE_F32, kKR>), dim3(nqb, (nkb + kKR - 1) / kKR, batch),
                       dim3(kWave), 0, stream, q, k, heads, t, scale_log2, in, stats, weights);
  } else {
    constexpr int kKR = 4;
    hipLaunchKernelGGL(attn::attn_wstats_kernel<MUSC_DTYPE_F16>, sgrid, dim3(kWave), 0, stream, q, k, t, scale_log2,
                       in, stats);
    hipLaunchKernelGGL((attn::attn_weights_kernel<MUSC_DTYPE_F16, kKR>), dim3(nqb, (nkb + kKR - 1) / kKR, batch),
                       dim3(kWave), 0, stream, q, k, heads, t, scale_log2, in, stats, weights);
  }
  return check_launch();
}

attn::HeadLayout contiguous(int heads, int t) {
  return attn::HeadLayout{(long long)heads * t * attn::D, (long long)t * attn::D, attn::D, heads};
}

}  // namespace

extern "C" int musc_attention_fwd(const void* q, const void* k, const void* v, void* out, int dtype, int bh, int t,
                                  int d, float scale, hipStream_t stream) {
  if (bh < 1 || t < 1) return MUSC_ERR_INVALID_ARG;
  const attn::HeadLayout l = contiguous(1, t);
  return attention_fwd(q, k, v, out, dtype, bh, 1, t, d, l, l, scale, stream);
}

extern "C" int musc_attention_fwd_strided(const void* q, const void* k, const void* v, void* out, int dtype,
                                          int batch, int heads, int t, int d, long long in_sb, long long in_sh,
                                          long long in_st, long long out_sb, long long out_sh, long long out_st,
                                          float scale, hipStream_t stream) {
  if (heads < 1) return MUSC_ERR_INVALID_ARG;
  return attention_fwd(q, k, v, out, dtype, batch, heads, t, d, attn::HeadLayout{in_sb, in_sh, in_st, heads},
                       attn::HeadLayout{out_sb, out_sh, out_st, heads}, scale, stream);
}

extern "C" int musc_attention_weights_workspace_bytes(int batch, int heads, int t, size_t* out) {
  if (!out || batch < 1 || heads < 1 || t < 1) return MUSC_ERR_INVALID_ARG;
  *out = align_up((size_t)batch * heads * t * sizeof(float2), 256);
  return MUSC_OK;
}

extern "C" int musc_attention_weights(const void* q, const void* k, int dtype, int batch, int heads, int t, int d,
                                      float scale, float* weights, void* workspace, size_t workspace_bytes,
                                      hipStream_t stream) {
  if (batch < 1 || heads < 1 || t < 1) return MUSC_ERR_INVALID_ARG;
  return attention_weights(q, k, dtype, batch, heads, t, d, contiguous(heads, t), scale, weights, workspace,
                           workspace_bytes, stream);
}

extern "C" int musc_attention_weights_strided(const void* q, const void* k, int dtype, int batch, int heads, int t,
                                              int d, long long in_sb, long long in_sh, long long in_st, float scale,
                                              float* weights, void* workspace, size_t workspace_bytes,
                                              hipStream_t stream) {
  if (heads < 1) return MUSC_ERR_INVALID_ARG;
  return attention_weights(q, k, dtype, batch, heads, t, d, attn::HeadLayout{in_sb, in_sh, in_st, heads}, scale,
                           weights, workspace, workspace_bytes, stream);
}
