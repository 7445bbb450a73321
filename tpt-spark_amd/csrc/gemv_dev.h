// Device code of the fused dequant-GEMV (see k_gemv.hip for the design): weight-group loads,
// Q8_K / Q8_0 activation quantization (or, for F16 weights, the f32 activations) into LDS, group
// dots, and gemv_run, one workgroup's share of a GEMV.
#pragma once
#include "kernels.h"

namespace tpt {
namespace gemv {

constexpr int NT = 512;  // threads per workgroup
constexpr int NW = NT / WAVE;
constexpr int MAXB = 64 / NW;       // 256-element activation blocks per wave (K <= 16384)

__device__ __forceinline__ uint32_t bsel(uint32_t v, int i) { return (v >> (8 * i)) & 0xffu; }

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// ----------------------------------------------------------------- per-lane weight groups
// group g of a row = 64 weights: Q4_K (block g/4, qs bytes 32(g%4)..), Q6_K (block g/4, half
// (g/2)%2, column half g%2), Q8_0 (blocks 2g, 2g+1), F16 (the 16-byte runs 4i + g%4, i < 8, of
// the 512-byte run of 256 weights g/4: the four lanes of a run read 64 contiguous bytes per load)
template <int WT> struct Raw;
template <> struct Raw<TPT_TYPE_Q4_K> { uint4 h, a, b; };
template <> struct Raw<TPT_TYPE_Q6_K> { uint4 qa, qb, qh; uint2 sc; uint32_t d; };
template <> struct Raw<TPT_TYPE_Q8_0> { uint4 a0, a1, b0, b1; uint32_t d0, d1; };
template <> struct Raw<TPT_TYPE_Q5_K> { uint4 h, a, b, ha, hb; };
template <> struct Raw<TPT_TYPE_Q4_0> { uint4 a, b; uint32_t d0, d1; };
template <> struct Raw<TPT_TYPE_F16> { uint4 v[8]; };

// activation form of a weight type: Q8_0 rows for Q8_0 and Q4_0 weights, Q8_K for the k-quants,
// f32 for F16 weights (candle's QMatMul dequantizes F16 weights to f32 and multiplies in f32)
enum ActKind { ACT_Q8K = 0, ACT_Q80 = 1, ACT_F32 = 2 };
template <int WT> constexpr int act_kind() {
  return WT == TPT_TYPE_F16 ? ACT_F32 : WT == TPT_TYPE_Q8_0 || WT == TPT_TYPE_Q4_0 ? ACT_Q80 : ACT_Q8K;
}
template <int WT> constexpr bool act_q80() { return act_kind<WT>() == ACT_Q80; }

template <int WT>
__device__ __forceinline__ void load_raw(const uint8_t* row, int g, Raw<WT>& r);

template <>
__device__ __forceinline__ void load_raw<TPT_TYPE_Q4_K>(const uint8_t* row, int g,
                                                         Raw<TPT_TYPE_Q4_K>& r) {
  const uint8_t* blk = row + (size_t)(g >> 2) * 144;  // 144 = 9 x 16: blocks stay 16-aligned
  const int off = 16 + (g & 3) * 32;
  r.h = *(const uint4*)blk;
  r.a = *(const uint4*)(blk + off);
  r.b = *(const uint4*)(blk + off + 16);
}

template <>
__device__ __forceinline__ void load_raw<TPT_TYPE_Q6_K>(const uint8_t* row, int g,
                                                         Raw<TPT_TYPE_Q6_K>& r) {
  const uint8_t* blk = row + (size_t)(g >> 2) * 210;  // 2-byte aligned: unaligned vector loads
  const int p = (g >> 1) & 1, h = g & 1;
  r.qa = ldg_u<uint4>(blk + 64 * p + 16 * h);
  r.qb = ldg_u<uint4>(blk + 64 * p + 32 + 16 * h);
  r.qh = ldg_u<uint4>(blk + 128 + 32 * p + 16 * h);
  r.sc = ldg_u<uint2>(blk + 192 + 8 * p);
  r.d = ldg_u<uint16_t>(blk + 208);
}

template <>
__device__ __forceinline__ void load_raw<TPT_TYPE_Q8_0>(const uint8_t* row, int g,
                                                         Raw<TPT_TYPE_Q8_0>& r) {
  const uint8_t* b0 = row + (size_t)g * 68;
  r.d0 = ldg_u<uint16_t>(b0);
  r.a0 = ldg_u<uint4>(b0 + 2);
  r.a1 = ldg_u<uint4>(b0 + 18);
  r.d1 = ldg_u<uint16_t>(b0 + 34);
  r.b0 = ldg_u<uint4>(b0 + 36);
  r.b1 = ldg_u<uint4>(b0 + 52);
}

template <>
__device__ __forceinline__ void load_raw<TPT_TYPE_Q5_K>(const uint8_t* row, int g,
                                                         Raw<TPT_TYPE_Q5_K>& r) {
  const uint8_t* blk = row + (size_t)(g >> 2) * 176;  // 176 = 11 x 16: blocks stay 16-aligned
  r.h = *(const uint4*)blk;
  r.ha = *(const uint4*)(blk + 16);  // qh: the fifth bits of all four groups
  r.hb = *(const uint4*)(blk + 32);
  r.a = *(const uint4*)(blk + 48 + (g & 3) * 32);
  r.b = *(const uint4*)(blk + 64 + (g & 3) * 32);
}

template <>
__device__ __forceinline__ void load_raw<TPT_TYPE_Q4_0>(const uint8_t* row, int g,
                                                         Raw<TPT_TYPE_Q4_0>& r) {
  const uint8_t* b0 = row + (size_t)g * 36;  // blocks 2g, 2g + 1 (18 bytes: 2-byte aligned)
  r.d0 = ldg_u<uint16_t>(b0);
  r.a = ldg_u<uint4>(b0 + 2);
  r.d1 = ldg_u<uint16_t>(b0 + 18);
  r.b = ldg_u<uint4>(b0 + 20);
}

template <>
__device__ __forceinline__ void load_raw<TPT_TYPE_F16>(const uint8_t* row, int g,
                                                        Raw<TPT_TYPE_F16>& r) {
  // rows of K fp16 values, K a multiple of 256: 512-byte runs, 16-byte aligned
  const uint8_t* b = row + (size_t)(g >> 2) * 512 + 16 * (g & 3);
#pragma unroll
  for (int i = 0; i < 8; i++) r.v[i] = *(const uint4*)(b + 64 * i);
}

// ----------------------------------------------------------------- activation (LDS)
// LDS layout, quantized activations: qs int8[K] | d float[K/bs] | s16 int[K/16] | scratch
// float[NW] | rows.  f32 activations: xf float[K] | scratch float[NW] | rows.
struct Lds {
  int* q32;
  float* d;
  int* s16;
  float* xf;
  float* red;
  float* rows;
};

__host__ __device__ inline size_t lds_act_bytes(int K, int kind) {
  if (kind == ACT_F32) return 4 * (size_t)K + 4 * NW;
  const int nd = kind == ACT_Q80 ? K / QK8_0 : K / QK_K;
  return (size_t)K + 4 * nd + 4 * (K / 16) + 4 * NW;
}

__device__ __forceinline__ Lds lds_layout(char* smem, int K, int kind) {
  Lds l;
  l.q32 = (int*)smem;
  l.xf = (float*)smem;
  if (kind == ACT_F32) {
    l.d = nullptr;
    l.s16 = nullptr;
    l.red = (float*)(smem + 4 * (size_t)K);
  } else {
    l.d = (float*)(smem + K);
    const int nd = kind == ACT_Q80 ? K / QK8_0 : K / QK_K;
    l.s16 = (int*)(smem + K + 4 * nd);
    l.red = (float*)(smem + K + 4 * nd + 4 * (K / 16));
  }
  l.rows = l.red + NW;
  return l;
}

// f32 activations in LDS: element e of 256-run c sits at word 256c + (e ^ xf_swizzle(c)).  The
// reader lanes (run, quarter q) of one load take words 32i + 8q + 4h of four consecutive runs;
// flipping bits 2 and 5 by run puts those 16 four-word groups on distinct banks.  The flip
// stays inside each lane's own word set, and the prologue's float4 stores stay contiguous.
__device__ __forceinline__ int xf_swizzle(int c) { return ((c & 1) << 2) | ((c & 2) << 4); }

__device__ __forceinline__ void barrier_lds() {
  // LDS-only barrier: outstanding global loads (the prefetched weights) stay in flight.
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Activation preload.  Loads are unconditional (clamped block index) so the waitcnt pass can
// count exactly how many later loads may stay in flight; the norm weights are loaded only for
// an RMSNorm prologue (NORM).
//  * Q8_K activations (Q4_K / Q6_K weights), ROWS16: one 256-block per 16-lane DPP row -- lane l
//    of wave w holds elements 16(l%16) .. +15 of block 4(w + qi NW) + l/16, qi < MAXQ.
//  * Q8_0 activations: one float4 per lane per 256-element block, blocks w, w + NW, ...
constexpr int MAXQ = MAXB / 4;  // block quads per wave in the ROWS16 layout
constexpr int SSQL = kSsqMax / WAVE;  // RMSNorm partial sums per lane
struct XPre {
  float4 x[MAXB];
  float4 w[MAXB];
  float ssq[SSQL];
};

template <bool ROWS16, bool NORM>
__device__ __forceinline__ void preload_x(const GemvArgs& A, XPre& p) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int nb = A.K / 256;
  const float4* xs = (const float4*)A.x;
  const float4* ws = (const float4*)A.norm_w;
  if constexpr (NORM) {
    if (A.ssq_in) {
#pragma unroll
      for (int i = 0; i < SSQL; i++) p.ssq[i] = A.ssq_in[min(lane + i * WAVE, A.n_ssq - 1)];
    }
  }
  if constexpr (ROWS16) {
    const int k = lane >> 4, m = lane & 15;
#pragma unroll
    for (int qi = 0; qi < MAXQ; qi++) {
      int b = 4 * (wid + qi * NW) + k;
      if (b >= nb) b = nb - 1;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        p.x[qi * 4 + j] = xs[b * 64 + m * 4 + j];
        if constexpr (NORM) p.w[qi * 4 + j] = ws[b * 64 + m * 4 + j];
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < MAXB; i++) {
      int b = wid + i * NW;
      if (b >= nb) b = nb - 1;
      p.x[i] = xs[b * 64 + lane];
      if constexpr (NORM) p.w[i] = ws[b * 64 + lane];
    }
  }
}

// whether preload slot i of this lane holds a real block (not a clamped duplicate)
template <bool ROWS16>
__device__ __forceinline__ bool slot_valid(int i, int nb) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if constexpr (ROWS16) return 4 * (wid + (i >> 2) * NW) + (lane >> 4) < nb;
  else return wid + i * NW < nb;
}

// 1/m of rms_norm (candle_nn::ops::rms_norm: m = sqrt(sum(x^2)/dim + eps)).  With partial sums
// from the kernel that wrote x (A.ssq_in), every wave adds them in the same order (lane slots in
// sequence, then the lanes by DPP), so all waves hold the same m without a workgroup barrier.
// Otherwise every workgroup reduces the whole vector itself from the preloaded registers (each
// element is owned by exactly one lane of the workgroup).
template <bool ROWS16>
__device__ __forceinline__ float rms_denominator(const GemvArgs& A, const XPre& p, float* red) {
  const int tid = threadIdx.x, wid = tid >> 6;
  const int nb = A.K / 256;
  if (A.ssq_in) {
    const int lane = tid & 63;
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < SSQL; i++) t += lane + i * WAVE < A.n_ssq ? p.ssq[i] : 0.f;
    t = wave_sum_dpp(t);
    return sqrtf(t / (float)A.K + A.eps);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < MAXB; i++) {
    if (slot_valid<ROWS16>(i, nb)) {
      const float4 v = p.x[i];
      ss = fmaf(v.x, v.x, ss);
      ss = fmaf(v.y, v.y, ss);
      ss = fmaf(v.z, v.z, ss);
      ss = fmaf(v.w, v.w, ss);
    }
  }
  ss = wave_sum_dpp(ss);
  if ((tid & 63) == 0) red[wid] = ss;
  barrier_lds();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < NW; i++) t += red[i];
  return sqrtf(t / (float)A.K + A.eps);
}

// x / m correctly rounded from y = RN(1/m): q0 = RN(x y) is within an ulp of x/m, the remainder
// x - q0 m is exact in one fma, and RN(q0 + r y) is the correctly rounded quotient (Markstein's
// correction step; checked against the divide on 1e9 random pairs).  The sign of a zero
// quotient may differ, which no later step can see.
__device__ __forceinline__ float div_rn(float x, float m, float y) {
  const float q0 = x * y;
  return fmaf(fmaf(-q0, m, x), y, q0);
}
// candle's y = x / m * w with one true divide per workgroup (y = 1/m) instead of one per value
__device__ __forceinline__ float4 apply_norm(float4 v, float4 w, float m, float y) {
  v.x = div_rn(v.x, m, y) * w.x;
  v.y = div_rn(v.y, m, y) * w.y;
  v.z = div_rn(v.z, m, y) * w.z;
  v.w = div_rn(v.w, m, y) * w.w;
  return v;
}

// Q8_K quantization (BlockQ8K::from_float) in the ROWS16 layout: a 16-lane row reduces its
// block's max |x| with four DPP steps; the signed value at the first position holding it
// (element order: lane, then element) comes from the ballot of the lanes that hold it;
// iscale = -128/max, q = round-half-away(iscale * x) (the lower clamp never binds), d = 1/iscale.
// A lane's 16 values are exactly one per-16 group, so its q sum is that group's bsum.
// NM: 1 RMSNorm, 0 none, -1 as A.prologue says.
template <int NM = -1>
__device__ __forceinline__ void prologue_q8k(const GemvArgs& A, const XPre& p, const Lds& L) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int k = lane >> 4, m16 = lane & 15;
  const int nb = A.K / QK_K;
  float mn = 1.f, rm = 1.f;
  const bool norm = NM < 0 ? A.prologue == PRO_RMSNORM : NM == 1;
  if (norm) {
    mn = rms_denominator<true>(A, p, L.red);
    rm = 1.f / mn;
  }
#pragma unroll
  for (int qi = 0; qi < MAXQ; qi++) {
    const int b0 = 4 * (wid + qi * NW);
    if (b0 < nb) {  // uniform across the wave
      const int b = b0 + k;
      float e[16];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float4 v = norm ? apply_norm(p.x[qi * 4 + j], p.w[qi * 4 + j], mn, rm) : p.x[qi * 4 + j];
        e[4 * j] = v.x; e[4 * j + 1] = v.y; e[4 * j + 2] = v.z; e[4 * j + 3] = v.w;
      }
      float la = fabsf(e[0]);
#pragma unroll
      for (int i = 1; i < 16; i++) la = fmaxf(la, fabsf(e[i]));
      float amax = la;
      amax = fmaxf(amax, dpp_mov<0xB1>(amax));   // quad_perm [1,0,3,2]
      amax = fmaxf(amax, dpp_mov<0x4E>(amax));   // quad_perm [2,3,0,1]
      amax = fmaxf(amax, dpp_mov<0x141>(amax));  // row_half_mirror
      amax = fmaxf(amax, dpp_mov<0x140>(amax));  // row_mirror: the 16-lane row's max
      float mine = 0.f;
#pragma unroll
      for (int i = 15; i >= 0; i--) mine = fabsf(e[i]) == amax ? e[i] : mine;  // first hit wins
      const unsigned long long hit = __ballot(la == amax);
      const uint32_t bits = (uint32_t)(hit >> (16 * k)) & 0xffffu;
      const int src = 16 * k + (bits ? __builtin_ctz(bits) : 0);
      const float mx = __shfl(mine, src, WAVE);
      const bool nz = amax != 0.f;
      const float iscale = -128.f / (nz ? mx : 1.f);
      int pk[4];
      int qs = 0;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        int w = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const float r = __builtin_amdgcn_fmed3f(roundf(iscale * e[4 * j + c]), -128.f, 127.f);
          const int q = nz ? (int)r : 0;
          qs += q;
          w |= (q & 0xff) << (8 * c);
        }
        pk[j] = w;
      }
      if (b < nb) {
        *(int4*)(L.q32 + b * 64 + 4 * m16) = make_int4(pk[0], pk[1], pk[2], pk[3]);
        L.s16[b * 16 + m16] = qs;
        if (m16 == 0) L.d[b] = nz ? 1.f / iscale : 0.f;
      }
    }
  }
}

// Q8_0 activation quantization (BlockQ8_0::from_float): 8 lanes per 32-block.
template <int NM = -1>
__device__ __forceinline__ void prologue_q80(const GemvArgs& A, const XPre& p, const Lds& L) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int nb = A.K / 256;
  float m = 1.f, rm = 1.f;
  const bool norm = NM < 0 ? A.prologue == PRO_RMSNORM : NM == 1;
  if (norm) {
    m = rms_denominator<false>(A, p, L.red);
    rm = 1.f / m;
  }
#pragma unroll
  for (int i = 0; i < MAXB; i++) {
    const int c = wid + i * NW;
    if (c < nb) {
      const float4 v = norm ? apply_norm(p.x[i], p.w[i], m, rm) : p.x[i];
      float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
      amax = fmaxf(amax, dpp_mov<0xB1>(amax));   // max over 8 lanes
      amax = fmaxf(amax, dpp_mov<0x4E>(amax));
      amax = fmaxf(amax, dpp_mov<0x141>(amax));
      const float d = amax / 127.f;
      const float id = d != 0.f ? 1.f / d : 0.f;
      const float e[4] = {v.x, v.y, v.z, v.w};
      int packed = 0;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        float r = roundf(e[j] * id);
        r = fminf(fmaxf(r, -128.f), 127.f);
        packed |= ((int)r & 0xff) << (8 * j);
      }
      L.q32[c * 64 + lane] = packed;
      if ((lane & 7) == 0) L.d[c * 8 + (lane >> 3)] = h2f(f2h(d));  // stored as f16
    }
  }
}

// f32 activations (F16 weights): candle's rms_norm output, or x itself, stored unquantized.
template <int NM = -1>
__device__ __forceinline__ void prologue_f32(const GemvArgs& A, const XPre& p, const Lds& L) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int nb = A.K / 256;
  float m = 1.f, rm = 1.f;
  const bool norm = NM < 0 ? A.prologue == PRO_RMSNORM : NM == 1;
  if (norm) {
    m = rms_denominator<false>(A, p, L.red);
    rm = 1.f / m;
  }
#pragma unroll
  for (int i = 0; i < MAXB; i++) {
    const int c = wid + i * NW;
    if (c < nb) {
      const float4 v = norm ? apply_norm(p.x[i], p.w[i], m, rm) : p.x[i];
      *(float4*)(L.xf + 256 * c + ((4 * lane) ^ xf_swizzle(c))) = v;
    }
  }
}

// ----------------------------------------------------------------- activation slices
struct Act {
  int q[16];     // the group's 64 int8 activation values, packed
  float d0, d1;  // Q8_K: d0 = block d;  Q8_0: d of each 32-block
  int s[4];      // Q4_K: s[0], s[1] = sums over each 32;  Q6_K: per-16 sums of the 4 quads
};
// F16 weights: the group's 64 f32 activations, x[2i + h] = elements 32i + 8q + 4h .. + 3 of the run
struct ActF {
  float4 x[16];
};
template <int WT> struct ActOf { using T = Act; };
template <> struct ActOf<TPT_TYPE_F16> { using T = ActF; };

__device__ __forceinline__ void load_act_f(const Lds& L, int g, ActF& a) {
  const int c = g >> 2, q = g & 3, sw = xf_swizzle(c);
  const float* run = L.xf + 256 * c;
#pragma unroll
  for (int i = 0; i < 8; i++)
#pragma unroll
    for (int h = 0; h < 2; h++) a.x[2 * i + h] = *(const float4*)(run + ((32 * i + 8 * q + 4 * h) ^ sw));
}

template <int WT>
__device__ __forceinline__ void load_act(const Lds& L, int g, ActF& a) {
  load_act_f(L, g, a);
}

template <int WT>
__device__ __forceinline__ void load_act(const Lds& L, int g, Act& a) {
  if constexpr (WT == TPT_TYPE_Q4_K || WT == TPT_TYPE_Q5_K) {
    const int4* q = (const int4*)(L.q32 + 16 * g);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int4 v = q[i];
      a.q[4 * i] = v.x; a.q[4 * i + 1] = v.y; a.q[4 * i + 2] = v.z; a.q[4 * i + 3] = v.w;
    }
    a.d0 = L.d[g >> 2];
    const int4 bs = *(const int4*)(L.s16 + 4 * g);
    a.s[0] = bs.x + bs.y;
    a.s[1] = bs.z + bs.w;
  } else if constexpr (WT == TPT_TYPE_Q6_K) {
    const int b = g >> 2, p = (g >> 1) & 1, h = g & 1;
#pragma unroll
    for (int quad = 0; quad < 4; quad++) {
      const int4 v = *(const int4*)(L.q32 + (256 * b + 128 * p + 32 * quad + 16 * h) / 4);
      a.q[4 * quad] = v.x; a.q[4 * quad + 1] = v.y; a.q[4 * quad + 2] = v.z; a.q[4 * quad + 3] = v.w;
    }
    const int4 s0 = *(const int4*)(L.s16 + 16 * b + 8 * p), s1 = *(const int4*)(L.s16 + 16 * b + 8 * p + 4);
    // per-16 sums of elements 128p + 32quad + 16h: s16 index 8p + 2quad + h
    a.s[0] = h ? s0.y : s0.x;
    a.s[1] = h ? s0.w : s0.z;
    a.s[2] = h ? s1.y : s1.x;
    a.s[3] = h ? s1.w : s1.z;
    a.d0 = L.d[b];
  } else {
    const int4* q = (const int4*)(L.q32 + 16 * g);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int4 v = q[i];
      a.q[4 * i] = v.x; a.q[4 * i + 1] = v.y; a.q[4 * i + 2] = v.z; a.q[4 * i + 3] = v.w;
    }
    a.d0 = L.d[2 * g];
    a.d1 = L.d[2 * g + 1];
  }
}

// Q4_K x Q8_K for one group: vec_dot_q4k_q8k's per-block arithmetic restricted to the group's
// two sub-blocks, d_w*d_x * sum_j sc_j * sum(q4*q8)  -  dmin_w*d_x * sum_j m_j * bsum_j.
// get_scale_min_k4 for j0 = 2(g%4), j1 = j0 + 1 without branches: the scale bytes sit at byte
// offset 2(g%2) of the header dwords y = s[0..3], z = s[4..7], w = s[8..11].
__device__ __forceinline__ float dot_group(const Raw<TPT_TYPE_Q4_K>& r, const Act& a, int g) {
  const int sh = 16 * (g & 1);
  const uint32_t Y = r.h.y >> sh, Z = r.h.z >> sh, W = r.h.w >> sh;
  const bool hi = (g & 2) != 0;
  const int sc0 = hi ? (int)((W & 0xF) | (((Y >> 6) & 3) << 4)) : (int)(Y & 63);
  const int sc1 = hi ? (int)(((W >> 8) & 0xF) | (((Y >> 14) & 3) << 4)) : (int)((Y >> 8) & 63);
  const int m0 = hi ? (int)(((W >> 4) & 0xF) | (((Z >> 6) & 3) << 4)) : (int)(Z & 63);
  const int m1 = hi ? (int)(((W >> 12) & 0xF) | (((Z >> 14) & 3) << 4)) : (int)((Z >> 8) & 63);
  const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
  int s0 = 0, s1 = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    s0 = sdot4((int)(w[i] & 0x0F0F0F0Fu), a.q[i], s0);
    s1 = sdot4((int)((w[i] >> 4) & 0x0F0F0F0Fu), a.q[8 + i], s1);
  }
  // 6-bit scales times sums of at most 64 products of 4-bit and 8-bit values: 24-bit multiplies
  // are exact
  const int isum = __mul24(sc0, s0) + __mul24(sc1, s1);
  const int msum = __mul24(m0, a.s[0]) + __mul24(m1, a.s[1]);
  const float dd = h2f((uint16_t)(r.h.x & 0xffff)) * a.d0;
  const float dm = h2f((uint16_t)(r.h.x >> 16)) * a.d0;
  return dd * (float)isum - dm * (float)msum;
}

// Q5_K x Q8_K for one group: vec_dot_q5k_q8k's per-block arithmetic restricted to the group's
// two sub-blocks -- Q4_K's with the values nibble + 16 * (bit 2(g%4) or 2(g%4)+1 of qh[l]).
__device__ __forceinline__ float dot_group(const Raw<TPT_TYPE_Q5_K>& r, const Act& a, int g) {
  const int sh = 16 * (g & 1);
  const uint32_t Y = r.h.y >> sh, Z = r.h.z >> sh, W = r.h.w >> sh;
  const bool hi = (g & 2) != 0;
  const int sc0 = hi ? (int)((W & 0xF) | (((Y >> 6) & 3) << 4)) : (int)(Y & 63);
  const int sc1 = hi ? (int)(((W >> 8) & 0xF) | (((Y >> 14) & 3) << 4)) : (int)((Y >> 8) & 63);
  const int m0 = hi ? (int)(((W >> 4) & 0xF) | (((Z >> 6) & 3) << 4)) : (int)(Z & 63);
  const int m1 = hi ? (int)(((W >> 12) & 0xF) | (((Z >> 14) & 3) << 4)) : (int)((Z >> 8) & 63);
  const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
  const uint32_t qh[8] = {r.ha.x, r.ha.y, r.ha.z, r.ha.w, r.hb.x, r.hb.y, r.hb.z, r.hb.w};
  const int b0 = 2 * (g & 3);
  int s0 = 0, s1 = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const uint32_t v0 = (w[i] & 0x0F0F0F0Fu) | (((qh[i] >> b0) & 0x01010101u) << 4);
    const uint32_t v1 = ((w[i] >> 4) & 0x0F0F0F0Fu) | (((qh[i] >> (b0 + 1)) & 0x01010101u) << 4);
    s0 = sdot4((int)v0, a.q[i], s0);
    s1 = sdot4((int)v1, a.q[8 + i], s1);
  }
  // 6-bit scales times sums of at most 32 products of 5-bit and 8-bit values: exact in 24 bits
  const int isum = __mul24(sc0, s0) + __mul24(sc1, s1);
  const int msum = __mul24(m0, a.s[0]) + __mul24(m1, a.s[1]);
  const float dd = h2f((uint16_t)(r.h.x & 0xffff)) * a.d0;
  const float dm = h2f((uint16_t)(r.h.x >> 16)) * a.d0;
  return dd * (float)isum - dm * (float)msum;
}

// Q4_0 x Q8_0 for two blocks: vec_dot_q4_0_q8_0's (float)sumi * d_w * d_x per block, with
// sumi = sum (q - 8) y = sum q y - 8 sum y (the activation sums by dot products with ones).
__device__ __forceinline__ float dot_group(const Raw<TPT_TYPE_Q4_0>& r, const Act& a, int) {
  const uint32_t wa[4] = {r.a.x, r.a.y, r.a.z, r.a.w}, wb[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
  int s0 = 0, s1 = 0, t0 = 0, t1 = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {  // low nibbles: elements 4i.., high nibbles: 16 + 4i..
    s0 = sdot4((int)(wa[i] & 0x0F0F0F0Fu), a.q[i], s0);
    s0 = sdot4((int)((wa[i] >> 4) & 0x0F0F0F0Fu), a.q[4 + i], s0);
    s1 = sdot4((int)(wb[i] & 0x0F0F0F0Fu), a.q[8 + i], s1);
    s1 = sdot4((int)((wb[i] >> 4) & 0x0F0F0F0Fu), a.q[12 + i], s1);
  }
#pragma unroll
  for (int i = 0; i < 8; i++) {
    t0 = sdot4(0x01010101, a.q[i], t0);
    t1 = sdot4(0x01010101, a.q[8 + i], t1);
  }
  return ((float)(s0 - 8 * t0) * h2f((uint16_t)r.d0)) * a.d0 + ((float)(s1 - 8 * t1) * h2f((uint16_t)r.d1)) * a.d1;
}

// Q6_K x Q8_K for one group (half p, column half h): vec_dot_q6k_q8k's per-block arithmetic,
// d_w*d_x * sum_quad sc * (sum(q6*q8) - 32*bsum).
__device__ __forceinline__ float dot_group(const Raw<TPT_TYPE_Q6_K>& r, const Act& a, int g) {
  const int h = g & 1;
  const uint32_t qa[4] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w};
  const uint32_t qb[4] = {r.qb.x, r.qb.y, r.qb.z, r.qb.w};
  const uint32_t qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
  int d0 = 0, d1 = 0, d2 = 0, d3 = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t v0 = (qa[i] & 0x0F0F0F0Fu) | ((qh[i] & 0x03030303u) << 4);
    const uint32_t v1 = (qb[i] & 0x0F0F0F0Fu) | (((qh[i] >> 2) & 0x03030303u) << 4);
    const uint32_t v2 = ((qa[i] >> 4) & 0x0F0F0F0Fu) | (((qh[i] >> 4) & 0x03030303u) << 4);
    const uint32_t v3 = ((qb[i] >> 4) & 0x0F0F0F0Fu) | (((qh[i] >> 6) & 0x03030303u) << 4);
    d0 = sdot4((int)v0, a.q[i], d0);
    d1 = sdot4((int)v1, a.q[4 + i], d1);
    d2 = sdot4((int)v2, a.q[8 + i], d2);
    d3 = sdot4((int)v3, a.q[12 + i], d3);
  }
  // scales of quads 0..3 are bytes h, h+2, h+4, h+6 of the 8 loaded (sc[8p .. 8p+8))
  const uint32_t slo = r.sc.x >> (8 * h), shi = r.sc.y >> (8 * h);
  const int sc0 = (int8_t)(slo & 0xff), sc1 = (int8_t)((slo >> 16) & 0xff);
  const int sc2 = (int8_t)(shi & 0xff), sc3 = (int8_t)((shi >> 16) & 0xff);
  // |d - 32 s| < 2^18 and |sc| <= 128: 24-bit multiplies are exact
  const int isum = __mul24(sc0, d0 - 32 * a.s[0]) + __mul24(sc1, d1 - 32 * a.s[1]) +
                   __mul24(sc2, d2 - 32 * a.s[2]) + __mul24(sc3, d3 - 32 * a.s[3]);
  return (h2f((uint16_t)r.d) * a.d0) * (float)isum;
}

// Q8_0 x Q8_0 for two blocks: vec_dot_q8_0_q8_0's (sum_i * d_w) * d_x per block.
__device__ __forceinline__ float dot_group(const Raw<TPT_TYPE_Q8_0>& r, const Act& a, int) {
  const uint32_t wa[8] = {r.a0.x, r.a0.y, r.a0.z, r.a0.w, r.a1.x, r.a1.y, r.a1.z, r.a1.w};
  const uint32_t wb[8] = {r.b0.x, r.b0.y, r.b0.z, r.b0.w, r.b1.x, r.b1.y, r.b1.z, r.b1.w};
  int s0 = 0, s1 = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    s0 = sdot4((int)wa[i], a.q[i], s0);
    s1 = sdot4((int)wb[i], a.q[8 + i], s1);
  }
  return ((float)s0 * h2f((uint16_t)r.d0)) * a.d0 + ((float)s1 * h2f((uint16_t)r.d1)) * a.d1;
}

// F16 x f32 for one group: the dequantized weights (exact) times the f32 activations, f32 FMA
// in four chains, added as (c0 + c1) + (c2 + c3).  candle's f32 matmul order (the gemm crate's
// blocking) is not restated.
__device__ __forceinline__ float dot_group(const Raw<TPT_TYPE_F16>& r, const ActF& a, int) {
  float c[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const uint32_t w[4] = {r.v[i].x, r.v[i].y, r.v[i].z, r.v[i].w};
    const float4 x0 = a.x[2 * i], x1 = a.x[2 * i + 1];
    const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      c[i & 3] = fmaf(h2f((uint16_t)(w[j] & 0xffff)), xs[2 * j], c[i & 3]);
      c[i & 3] = fmaf(h2f((uint16_t)(w[j] >> 16)), xs[2 * j + 1], c[i & 3]);
    }
  }
  return (c[0] + c[1]) + (c[2] + c[3]);
}

// K or V cache elements ci, ci+1 (ci even): fp16 pair packed into one 32-bit store, or two f32
__device__ __forceinline__ void store_kv_pair(void* cache, int kv_type, size_t ci, float a, float b) {
  if (kv_type == TPT_TYPE_F32) {
    ((float*)cache)[ci] = a;
    ((float*)cache)[ci + 1] = b;
  } else {
    *(uint32_t*)((uint16_t*)cache + ci) = (uint32_t)f2h(a) | ((uint32_t)f2h(b) << 16);
  }
}

// ----------------------------------------------------------------- the kernel
// Launch geometry shared by host and device.
struct Geo {
  int rows_per_wg;  // contiguous rows per workgroup (whole row groups, even)
  int P;            // passes per row
};


// Does nothing between the first weight loads and the activation prologue (standalone launch).
struct NoHook {
  __device__ void operator()() const {}
};

// One workgroup's share of a GEMV: rows [wg * rows_per_wg, ...).  WT weight type; BPP
// super-blocks per row per pass (16, or fewer for short rows, then RPP = 16/BPP rows share a
// pass); RB row slots per step; NMAT matrices (2: gate|up, streamed one after the other: the
// workgroup's gate rows, then its up rows, as 2 rows_per_wg rows of one walk, so that at any
// step the waves read one contiguous window); KS-way split of the passes across
// waves; D steps in flight per wave; NORM: RMSNorm prologue; ONEPASS: one pass per row (the
// lane's activation slice is then the same at every step and is read from LDS once).  hook()
// runs after the activation and the first weight loads are issued, before the activation is
// quantized.
//
// Row totals: a row's LPR lanes first reduce in 16-lane DPP rows; the NPART partial sums of a
// row go to LDS and the epilogue adds them as (p0 + p1) + (p2 + p3) -- the bits a full
// lane_group_sum<LPR> would give, without LDS round trips inside the step loop.
template <int BPP> struct RowParts {
  static constexpr int LPR = 4 * BPP;
  static constexpr int N = LPR >= 16 ? LPR / 16 : 1;
};
template <int NPART>
__device__ __forceinline__ float row_total(const float* p) {
  if constexpr (NPART == 4) return (p[0] + p[1]) + (p[2] + p[3]);
  else if constexpr (NPART == 2) return p[0] + p[1];
  else return p[0];
}

template <int WT, int BPP, int RB, int NMAT, int KS, int D, bool NORM, bool ONEPASS, typename Hook>
__device__ __forceinline__ void gemv_run(const GemvArgs& A, const Geo& geo, int wg, char* smem,
                                         const Hook& hook) {
  constexpr int RPP = 16 / BPP;   // rows per pass
  constexpr int LPR = 4 * BPP;    // lanes per row
  constexpr int RG = RB * RPP;    // rows per row group
  constexpr int WR = NW / KS;     // waves per k-split
  constexpr int NPART = RowParts<BPP>::N;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int K = A.K, N = A.N;
  const int nb = K / QK_K;  // super-blocks (256 weights) per row
  const Lds L = lds_layout(smem, K, act_kind<WT>());
  const int RPW = geo.rows_per_wg;
  const int r0 = wg * RPW;
  constexpr bool PAIR = NMAT == 2;
  const int VR = PAIR ? 2 * RPW : RPW;  // rows of the walk: gate rows, then up rows
  const int rp = lane / LPR, sb = (lane / 4) % BPP, q = lane & 3;

  // this wave's row groups and passes
  const int ngrp = VR / RG;
  const int wr = wid / KS, ks = wid % KS;
  // row groups wr, wr + WR, ...: at any step the waves of a k-split read adjacent rows, so a
  // workgroup streams one contiguous window of the matrix
  const int ng = ngrp > wr ? (ngrp - wr + WR - 1) / WR : 0;
  const int pa = ks * geo.P / KS, pb = (ks + 1) * geo.P / KS;
  const int PP = pb - pa;
  const int S = ng * PP;


  // 2. weight steps in a ring of D register slots (slot d holds steps d, d + D, ...), the first
  //    D issued before the prologue
  Raw<WT> ring[D][RB];
  auto group_of = [&](int p, bool* valid) {  // this lane's weight group in pass p
    const int blk = p * BPP + sb;
    *valid = blk < nb;
    return 4 * (blk < nb ? blk : nb - 1) + q;
  };
  auto issue = [&](Raw<WT> (&buf)[RB], int s) {
    if (s >= S) s = S > 0 ? S - 1 : 0;  // past the end: re-read the last step (cache hits)
    const int pp = PP > 0 ? PP : 1;
    const int grp = wr + (s / pp) * WR, p = pa + s % pp;
    bool v;
    const int g = group_of(p, &v);
#pragma unroll
    for (int j = 0; j < RB; j++) {
      const int vr = (grp * RB + j) * RPP + rp;
      const bool up = PAIR && vr >= RPW;
      int row = r0 + (up ? vr - RPW : vr);
      if (row >= N) row = N - 1;
      load_raw<WT>((up ? A.w1 : A.w0) + (size_t)row * A.row_stride, g, buf[j]);
    }
  };
  // 0. the epilogue's own operands (residual, step position, argmax slot) are read before
  //    everything else: their latency then hides under the weight stream instead of following it
  const int nrows = min(RPW, N - r0);
  float pre_r = 0.f;  // EPI_RESID: resid of row tid
  int pos = 0, slot = 0;
  if (A.epilogue == EPI_RESID && tid < nrows) pre_r = A.resid[r0 + tid];
  if (A.epilogue == EPI_ROPE_QKV) pos = A.state ? A.state->pos : A.pos_host;
  if (A.epilogue == EPI_ARGMAX) slot = A.state ? A.state->parity : 0;
  // 1. activation values next: the loads complete in issue order, so the prologue below only
  //    waits for these, not for the weights issued after them
  XPre xp;
  preload_x<act_kind<WT>() == ACT_Q8K, NORM>(A, xp);
  // every activation load ahead of every weight load, and no prologue arithmetic among them:
  // the prologue then waits only for the former (left alone, the scheduler sinks some
  // activation loads below the weight loads, or hoists the first uses of x above them)
  __builtin_amdgcn_sched_barrier(0);
  // Long rows (two rows per step, K > 8192: the down GEMV's 56 KB activation) issue one step
  // ahead of the prologue and the rest behind it, so fewer weight bytes stand between the
  // activation loads and the prologue (8B decode +1%); shorter rows issue all D ahead.
  constexpr int PRE = RB == 2 ? 1 : D;
#pragma unroll
  for (int d = 0; d < PRE; d++) issue(ring[d], d);
  __builtin_amdgcn_sched_barrier(0);
  hook();
  if constexpr (act_kind<WT>() == ACT_F32) prologue_f32<NORM ? 1 : 0>(A, xp, L);
  else if constexpr (act_q80<WT>()) prologue_q80<NORM ? 1 : 0>(A, xp, L);
  else prologue_q8k<NORM ? 1 : 0>(A, xp, L);
#pragma unroll
  for (int d = PRE; d < D; d++) issue(ring[d], d);
  barrier_lds();

  // EPI_ROPE_QKV: the rotation of the thread's first (even, odd) row pair, issued behind the
  // first weight steps (the position arrived with the activation)
  float pre_c = 1.f, pre_s = 0.f;
  if (A.epilogue == EPI_ROPE_QKV && 2 * tid < nrows) {
    const int lrow = A.row0 + r0 + 2 * tid;
    if (lrow < A.qd + A.kd) {
      const int rr = lrow < A.qd ? lrow : lrow - A.qd;
      const size_t ti = (size_t)pos * (A.hd / 2) + ((rr % A.hd) >> 1);
      pre_c = A.rope_cos[ti];
      pre_s = A.rope_sin[ti];
    }
  }

  float acc[RB];
#pragma unroll
  for (int j = 0; j < RB; j++) acc[j] = 0.f;

  using ActT = typename ActOf<WT>::T;
  auto compute = [&](const Raw<WT> (&buf)[RB], int s, const ActT& act, int g, bool v) {
    const int grp = wr + (s / PP) * WR, p = pa + s % PP;
#pragma unroll
    for (int j = 0; j < RB; j++) {
      const float t = dot_group(buf[j], act, g);
      acc[j] += v ? t : 0.f;
    }
    if (p == pb - 1) {  // row group done: the row's partial sums to LDS
#pragma unroll
      for (int j = 0; j < RB; j++) {
        float t;
        int part = 0;
        if constexpr (LPR >= 16) {
          t = sum16(acc[j]);
          part = (lane % LPR) >> 4;
        } else {
          t = lane_group_sum<LPR>(acc[j]);
        }
        if (lane % (LPR >= 16 ? 16 : LPR) == 0)
          L.rows[((size_t)ks * VR + (grp * RB + j) * RPP + rp) * NPART + part] = t;
        acc[j] = 0.f;
      }
    }
  };

  if (S > 0) {
    if constexpr (ONEPASS) {  // this lane's activation slice is the same at every step
      bool v;
      const int g = group_of(pa, &v);
      ActT act;
      load_act<WT>(L, g, act);
      for (int s = 0; s < S; s += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
          if (s + d < S) compute(ring[d], s + d, act, g, v);
          issue(ring[d], s + d + D);  // unconditional: the slot's next step
        }
      }
    } else {
      for (int s = 0; s < S; s += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
          if (s + d < S) {
            bool v;
            const int g = group_of(pa + (s + d) % PP, &v);
            ActT act;
            load_act<WT>(L, g, act);
            compute(ring[d], s + d, act, g, v);
          }
          issue(ring[d], s + d + D);
        }
      }
    }
  }
  __syncthreads();

  // 3. epilogue over the workgroup's rows (first row / pair of each thread from the operands
  //    fetched up front)
  auto row_val = [&](int i, int m) {
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < KS; k++) t += row_total<NPART>(L.rows + ((size_t)k * VR + i + m * RPW) * NPART);
    return t;
  };
  switch (A.epilogue) {
    case EPI_STORE:
      for (int i = tid; i < nrows; i += NT) A.y[r0 + i] = row_val(i, 0);
      break;
    case EPI_RESID: {
      float ss = 0.f;  // sum of squares of the stored rows (A.ssq_out)
      for (int i = tid; i < nrows; i += NT) {
        float r;
        if (i == tid) r = pre_r;
        else r = A.resid[r0 + i];
        const float v = row_val(i, 0) + r;
        A.y[r0 + i] = v;
        ss = fmaf(v, v, ss);
      }
      if (A.ssq_out) {
        if (nrows <= WAVE) {  // the rows sit in wave 0
          if (wid == 0) {
            ss = wave_sum_dpp(ss);
            if (lane == 0) A.ssq_out[wg] = ss;
          }
        } else {
          ss = wave_sum_dpp(ss);
          float* red = L.red;  // free after the row totals were read
          __syncthreads();
          if (lane == 0) red[wid] = ss;
          __syncthreads();
          if (tid == 0) {
            float t = 0.f;
#pragma unroll
            for (int w = 0; w < NW; w++) t += red[w];
            A.ssq_out[wg] = t;
          }
        }
      }
    } break;
    case EPI_SWIGLU:
      for (int i = tid; i < nrows; i += NT) {
        const float g = row_val(i, 0);
        A.y[r0 + i] = silu_mul(g, row_val(i, NMAT - 1));
      }
      break;
    case EPI_ARGMAX: {
      unsigned long long best = 0;
      for (int i = tid; i < nrows; i += NT) {
        const float v = row_val(i, 0);
        if (A.y) A.y[r0 + i] = v;
        const unsigned long long key =
            ((unsigned long long)order_key(v) << 32) | (unsigned long long)(r0 + i);
        best = key > best ? key : best;
      }
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const unsigned long long ob = __shfl_xor(best, o, WAVE);
        best = ob > best ? ob : best;
      }
      // one atomic per workgroup: the waves' maxima meet in LDS (the row buffer is free now)
      unsigned long long* wbest = (unsigned long long*)L.q32;
      __syncthreads();
      if (lane == 0) wbest[wid] = best;
      __syncthreads();
      if (tid == 0) {
        unsigned long long b = 0;
#pragma unroll
        for (int w = 0; w < NW; w++) b = wbest[w] > b ? wbest[w] : b;
        if (b) atomicMax(A.amax + slot, b);
      }
    } break;
    case EPI_ROPE_QKV:
      // rows come in (even, odd) pairs; r0 and nrows are even
      for (int i = 2 * tid; i < nrows; i += 2 * NT) {
        const float x0 = row_val(i, 0), x1 = row_val(i + 1, 0);
        const int lrow = A.row0 + r0 + i;
        if (lrow < A.qd + A.kd) {
          const bool isq = lrow < A.qd;
          const int rr = isq ? lrow : lrow - A.qd;
          const size_t ti = (size_t)pos * (A.hd / 2) + ((rr % A.hd) >> 1);
          float cs, sn;
          if (i == 2 * tid) {
            cs = pre_c;
            sn = pre_s;
          } else {
            cs = A.rope_cos[ti];
            sn = A.rope_sin[ti];
          }
          // candle rope_i: dst[2i] = x0*cos - x1*sin; dst[2i+1] = x0*sin + x1*cos
          const float o0 = x0 * cs - x1 * sn, o1 = x0 * sn + x1 * cs;
          if (isq) {
            A.y[rr] = o0;
            A.y[rr + 1] = o1;
          } else {
            const size_t ci = ((size_t)(rr / A.hd) * A.max_ctx + pos) * A.hd + rr % A.hd;
            store_kv_pair(A.kcache, A.kv_type, ci, o0, o1);
          }
        } else {
          const int rr = lrow - A.qd - A.kd;
          const size_t ci = ((size_t)(rr / A.hd) * A.max_ctx + pos) * A.hd + rr % A.hd;
          store_kv_pair(A.vcache, A.kv_type, ci, x0, x1);
        }
      }
      break;
  }
}
}  // namespace gemv
}  // namespace tpt
