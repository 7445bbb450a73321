// Fused k-quant dequant-GEMV for bs=1 decode on gfx950.
//
// y[r] = sum_k W[r,k] * x[k], W in GGUF block layout (rows of K/256 super-blocks, uploaded
// unchanged), x fp32.  Replaces dequant_and_gemm (src-tauri/src/engine/wgpu_engine.rs:581-605:
// a full f32 dequant of W into a fresh buffer, then gemm.wgsl at M=1) and restates what the
// reference's CandleEngine computes on the CPU through candle 0.8.4 QMatMul:
//   k_quants::matmul -> BlockQ8K::from_float (activation quant) -> vec_dot_q4k_q8k /
//   vec_dot_q6k_q8k / vec_dot_q8_0_q8_0 (integer sums, f32 block scaling).
//
// Work layout (MI355X: 256 CUs, wave64, 160 KB LDS/CU, HBM3E):
//  * A lane owns a "group" of 64 weights: a quarter of a k-quant super-block (Q4_K: 32 qs bytes
//    + the block's 16-byte header; Q6_K: one (half, 16-column) slice: 2 x 16 ql bytes, 16 qh
//    bytes, its 8 scales and d; Q8_0: two 34-byte blocks).  A "pass" covers BPP super-blocks
//    of a row (4 lanes each); when a row has fewer than 16 super-blocks a pass covers
//    RPP = 16/BPP rows, so every lane of the wave has work.
//  * A wave runs RB rows in lockstep over a flattened sequence of (row group, pass) steps and
//    double-buffers them: the loads of step s+1 are in flight while step s is computed.  Loads
//    are unconditional (indices clamped into the matrix) so that the compiler never has to
//    wait on them one by one.  Workgroups own contiguous row ranges; the waves of a workgroup
//    split its row groups (and, for long rows, the passes: KS-way split of K).
//  * Prologue, once per workgroup: x (optionally RMS-normalised) is quantized exactly like
//    candle's CPU path into LDS -- Q8_K (per 256: signed max-abs value, iscale = -128/max,
//    round half away from zero, clamp 127, d = 1/iscale, per-16 sums) for k-quant weights,
//    Q8_0 (per 32: d = amax/127 rounded to f16, q = round(x/d)) for Q8_0 weights.  The x loads
//    are issued first and the first step's weight loads right after, so the prologue runs
//    under HBM latency.
//  * Integer dots use v_dot4_i32_i8; each group ends in f32 block scaling (candle's per-block
//    arithmetic), lanes accumulate in f32 and a row is reduced across its lanes once, with
//    DPP.  Row results go to LDS, and after a workgroup barrier the epilogue stores them:
//    plain, + residual, SiLU(gate)*up, interleaved RoPE + KV-cache append, or greedy argmax
//    (what follows the GEMV in run_forward_pass, wgpu_engine.rs:373-486).
#include <hip/hip_ext.h>

#include "kernels.h"

namespace tpt {

namespace {

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
// (g/2)%2, column half g%2), Q8_0 (blocks 2g, 2g+1)
template <int WT> struct Raw;
template <> struct Raw<TPT_TYPE_Q4_K> { uint4 h, a, b; };
template <> struct Raw<TPT_TYPE_Q6_K> { uint4 qa, qb, qh; uint2 sc; uint32_t d; };
template <> struct Raw<TPT_TYPE_Q8_0> { uint4 a0, a1, b0, b1; uint32_t d0, d1; };

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

// ----------------------------------------------------------------- activation (LDS)
// LDS layout: qs int8[K] | d float[K/bs] | s16 int[K/16] | scratch float[NW] | rows
struct Lds {
  int* q32;
  float* d;
  int* s16;
  float* red;
  float* rows;
};

__host__ __device__ inline size_t lds_act_bytes(int K, bool q80) {
  const int nd = q80 ? K / QK8_0 : K / QK_K;
  return (size_t)K + 4 * nd + 4 * (K / 16) + 4 * NW;
}

__device__ __forceinline__ Lds lds_layout(char* smem, int K, bool q80) {
  Lds l;
  l.q32 = (int*)smem;
  l.d = (float*)(smem + K);
  const int nd = q80 ? K / QK8_0 : K / QK_K;
  l.s16 = (int*)(smem + K + 4 * nd);
  l.red = (float*)(smem + K + 4 * nd + 4 * (K / 16));
  l.rows = l.red + NW;
  return l;
}

__device__ __forceinline__ void barrier_lds() {
  // LDS-only barrier: outstanding global loads (the prefetched weights) stay in flight.
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Activation preload: one float4 per lane per 256-element block, blocks b = wave, wave + NW,
// ...  Loads are unconditional (clamped block index, x itself as a dummy norm source) so the
// waitcnt pass can count exactly how many later loads may stay in flight.
struct XPre {
  float4 x[MAXB];
  float4 w[MAXB];
};

__device__ __forceinline__ void preload_x(const GemvArgs& A, XPre& p) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int nb = A.K / 256;
  const float4* xs = (const float4*)A.x;
  const float4* ws = (const float4*)(A.prologue == PRO_RMSNORM ? A.norm_w : A.x);
#pragma unroll
  for (int i = 0; i < MAXB; i++) {
    int b = wid + i * NW;
    if (b >= nb) b = nb - 1;
    p.x[i] = xs[b * 64 + lane];
    p.w[i] = ws[b * 64 + lane];
  }
}

// 1/m of rms_norm (candle_nn::ops::rms_norm: m = sqrt(sum(x^2)/dim + eps)).  Every workgroup
// reduces the whole vector itself from the preloaded registers (each element is owned by
// exactly one lane of the workgroup).
__device__ float rms_denominator(const GemvArgs& A, const XPre& p, float* red) {
  const int tid = threadIdx.x, wid = tid >> 6;
  const int nb = A.K / 256;
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < MAXB; i++) {
    if (wid + i * NW < nb) {
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

__device__ __forceinline__ float4 apply_norm(float4 v, float4 w, float m) {
  v.x = v.x / m * w.x;
  v.y = v.y / m * w.y;
  v.z = v.z / m * w.z;
  v.w = v.w / m * w.w;
  return v;
}

// Q8_K quantization of one 256-block per wave (BlockQ8K::from_float).  The blocks of a wave
// are independent, so their reductions interleave.
__device__ void prologue_q8k(const GemvArgs& A, const XPre& p, const Lds& L) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int nb = A.K / QK_K;
  float m = 1.f;
  const bool norm = A.prologue == PRO_RMSNORM;
  if (norm) m = rms_denominator(A, p, L.red);
#pragma unroll
  for (int i = 0; i < MAXB; i++) {
    const int b = wid + i * NW;
    if (b < nb) {
      const float4 v = norm ? apply_norm(p.x[i], p.w[i], m) : p.x[i];
      const float e[4] = {v.x, v.y, v.z, v.w};
      int qsum;
      float d;
      const int packed = q8k_block_wave(e, &qsum, &d);
      L.q32[b * 64 + lane] = packed;
      if ((lane & 3) == 0) L.s16[b * 16 + (lane >> 2)] = qsum;
      if (lane == 0) L.d[b] = d;
    }
  }
}

// Q8_0 activation quantization (BlockQ8_0::from_float): 8 lanes per 32-block.
__device__ void prologue_q80(const GemvArgs& A, const XPre& p, const Lds& L) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int nb = A.K / 256;
  float m = 1.f;
  const bool norm = A.prologue == PRO_RMSNORM;
  if (norm) m = rms_denominator(A, p, L.red);
#pragma unroll
  for (int i = 0; i < MAXB; i++) {
    const int c = wid + i * NW;
    if (c < nb) {
      const float4 v = norm ? apply_norm(p.x[i], p.w[i], m) : p.x[i];
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

// ----------------------------------------------------------------- activation slices
struct Act {
  int q[16];     // the group's 64 int8 activation values, packed
  float d0, d1;  // Q8_K: d0 = block d;  Q8_0: d of each 32-block
  int s[4];      // Q4_K: s[0], s[1] = sums over each 32;  Q6_K: per-16 sums of the 4 quads
};

template <int WT>
__device__ __forceinline__ void load_act(const Lds& L, int g, Act& a) {
  if constexpr (WT == TPT_TYPE_Q4_K) {
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
  const int isum = sc0 * s0 + sc1 * s1;
  const int msum = m0 * a.s[0] + m1 * a.s[1];
  const float dd = h2f((uint16_t)(r.h.x & 0xffff)) * a.d0;
  const float dm = h2f((uint16_t)(r.h.x >> 16)) * a.d0;
  return dd * (float)isum - dm * (float)msum;
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
  const int isum = sc0 * (d0 - 32 * a.s[0]) + sc1 * (d1 - 32 * a.s[1]) +
                   sc2 * (d2 - 32 * a.s[2]) + sc3 * (d3 - 32 * a.s[3]);
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

// ----------------------------------------------------------------- the kernel
// Launch geometry shared by host and device.
struct Geo {
  int rows_per_wg;  // contiguous rows per workgroup (whole row groups, even)
  int P;            // passes per row
};

// WT weight type; BPP super-blocks per row per pass (16, or fewer for short rows, then
// RPP = 16/BPP rows share a pass); RB row slots per step; NMAT matrices (2: gate|up);
// KS-way split of the passes across waves; D steps in flight per wave.
template <int WT, int BPP, int RB, int NMAT, int KS, int D>
__global__ void __launch_bounds__(NT, 2) gemv_q8_kernel(const GemvArgs A, const Geo geo) {
  constexpr int RPP = 16 / BPP;   // rows per pass
  constexpr int LPR = 4 * BPP;    // lanes per row
  constexpr int RG = RB * RPP;    // rows per row group
  constexpr int WR = NW / KS;     // waves per k-split
  extern __shared__ __align__(16) char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int K = A.K, N = A.N;
  const bool q80 = WT == TPT_TYPE_Q8_0;
  const int nb = K / QK_K;  // super-blocks (256 weights) per row
  const Lds L = lds_layout(smem, K, q80);
  const int RPW = geo.rows_per_wg;
  const int r0 = blockIdx.x * RPW;
  const int rp = lane / LPR, sb = (lane / 4) % BPP, q = lane & 3;

  // this wave's row groups and passes
  const int ngrp = RPW / RG;
  const int wr = wid / KS, ks = wid % KS;
  const int g0 = wr * ngrp / WR, g1 = (wr + 1) * ngrp / WR;
  const int pa = ks * geo.P / KS, pb = (ks + 1) * geo.P / KS;
  const int PP = pb - pa;
  const int S = (g1 - g0) * PP;

  // 1. activation values (issued first: see preload_x)
  XPre xp;
  preload_x(A, xp);

  // 2. the first D steps' weight loads, then the prologue under their latency.  Steps live in
  //    a ring of D register slots; slot d holds steps d, d + D, d + 2D, ...
  Raw<WT> ring[D][RB][NMAT];
  auto group_of = [&](int p, bool* valid) {  // this lane's weight group in pass p
    const int blk = p * BPP + sb;
    *valid = blk < nb;
    return 4 * (blk < nb ? blk : nb - 1) + q;
  };
  auto issue = [&](Raw<WT> (&buf)[RB][NMAT], int s) {
    if (s >= S) s = S > 0 ? S - 1 : 0;  // past the end: re-read the last step (cache hits)
    const int pp = PP > 0 ? PP : 1;
    const int grp = g0 + s / pp, p = pa + s % pp;
    bool v;
    const int g = group_of(p, &v);
#pragma unroll
    for (int j = 0; j < RB; j++) {
      int row = r0 + (grp * RB + j) * RPP + rp;
      if (row >= N) row = N - 1;
#pragma unroll
      for (int m = 0; m < NMAT; m++)
        load_raw<WT>((m == 0 ? A.w0 : A.w1) + (size_t)row * A.row_stride, g, buf[j][m]);
    }
  };
#pragma unroll
  for (int d = 0; d < D; d++) issue(ring[d], d);
  if constexpr (WT == TPT_TYPE_Q8_0) prologue_q80(A, xp, L);
  else prologue_q8k(A, xp, L);
  barrier_lds();

  float acc[RB][NMAT];
#pragma unroll
  for (int j = 0; j < RB; j++)
#pragma unroll
    for (int m = 0; m < NMAT; m++) acc[j][m] = 0.f;

  auto compute = [&](const Raw<WT> (&buf)[RB][NMAT], int s) {
    const int grp = g0 + s / PP, p = pa + s % PP;
    bool v;
    const int g = group_of(p, &v);
    Act act;
    load_act<WT>(L, g, act);
#pragma unroll
    for (int j = 0; j < RB; j++)
#pragma unroll
      for (int m = 0; m < NMAT; m++) {
        const float t = dot_group(buf[j][m], act, g);
        acc[j][m] += v ? t : 0.f;
      }
    if (p == pb - 1) {  // row group done: row totals to LDS
#pragma unroll
      for (int j = 0; j < RB; j++)
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
          const float t = lane_group_sum<LPR>(acc[j][m]);
          if (lane % LPR == 0) L.rows[((size_t)ks * RPW + (grp * RB + j) * RPP + rp) * NMAT + m] = t;
          acc[j][m] = 0.f;
        }
    }
  };

  if (S > 0) {
    for (int s = 0; s < S; s += D) {
#pragma unroll
      for (int d = 0; d < D; d++) {
        if (s + d < S) compute(ring[d], s + d);
        issue(ring[d], s + d + D);  // unconditional: the slot's next step
      }
    }
  }
  __syncthreads();

  // 3. epilogue over the workgroup's rows
  const int nrows = min(RPW, N - r0);
  int pos = 0;
  if (A.epilogue == EPI_ROPE_QKV) pos = A.state ? A.state->pos : A.pos_host;
  auto row_val = [&](int i, int m) {
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < KS; k++) t += L.rows[((size_t)k * RPW + i) * NMAT + m];
    return t;
  };
  switch (A.epilogue) {
    case EPI_STORE:
      for (int i = tid; i < nrows; i += NT) A.y[r0 + i] = row_val(i, 0);
      break;
    case EPI_RESID:
      for (int i = tid; i < nrows; i += NT) A.y[r0 + i] = row_val(i, 0) + A.resid[r0 + i];
      break;
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
        if (b) atomicMax(A.amax + (A.state ? A.state->parity : 0), b);
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
          const float cs = A.rope_cos[ti], sn = A.rope_sin[ti];
          // candle rope_i: dst[2i] = x0*cos - x1*sin; dst[2i+1] = x0*sin + x1*cos
          const float o0 = x0 * cs - x1 * sn, o1 = x0 * sn + x1 * cs;
          if (isq) {
            A.y[rr] = o0;
            A.y[rr + 1] = o1;
          } else {
            const size_t ci = ((size_t)(rr / A.hd) * A.max_ctx + pos) * A.hd + rr % A.hd;
            if (A.kv_type == TPT_TYPE_F32) {
              ((float*)A.kcache)[ci] = o0;
              ((float*)A.kcache)[ci + 1] = o1;
            } else {
              ((uint16_t*)A.kcache)[ci] = f2h(o0);
              ((uint16_t*)A.kcache)[ci + 1] = f2h(o1);
            }
          }
        } else {
          const int rr = lrow - A.qd - A.kd;
          const size_t ci = ((size_t)(rr / A.hd) * A.max_ctx + pos) * A.hd + rr % A.hd;
          if (A.kv_type == TPT_TYPE_F32) {
            ((float*)A.vcache)[ci] = x0;
            ((float*)A.vcache)[ci + 1] = x1;
          } else {
            ((uint16_t*)A.vcache)[ci] = f2h(x0);
            ((uint16_t*)A.vcache)[ci + 1] = f2h(x1);
          }
        }
      }
      break;
  }
}

// ----------------------------------------------------------------- fp32-activation variant
// y[r] = sum_k dequant(W)[r,k] * x[k] (dequantized exactly like the oracle, fp32 FMA).  One
// wave per row, x read through the vector cache.  Not on the parity path (candle quantizes
// activations); kept for the fp32-activation GEMV report.
// (The group layout and loads are the ones the Q8 kernel uses.)
template <int WT>
__device__ __forceinline__ void dequant64(const uint8_t* row, int g, float* y);

template <>
__device__ __forceinline__ void dequant64<TPT_TYPE_Q4_K>(const uint8_t* row, int g, float* y) {
  Raw<TPT_TYPE_Q4_K> r;
  load_raw<TPT_TYPE_Q4_K>(row, g, r);
  const int g4 = g & 3;
  int sc0, m0, sc1, m1;
  if (g4 < 2) {
    const int j0 = 2 * g4;
    sc0 = bsel(r.h.y, j0) & 63; m0 = bsel(r.h.z, j0) & 63;
    sc1 = bsel(r.h.y, j0 + 1) & 63; m1 = bsel(r.h.z, j0 + 1) & 63;
  } else {
    const int k = 2 * g4 - 4;
    sc0 = (bsel(r.h.w, k) & 0xF) | ((bsel(r.h.y, k) >> 6) << 4);
    m0 = (bsel(r.h.w, k) >> 4) | ((bsel(r.h.z, k) >> 6) << 4);
    sc1 = (bsel(r.h.w, k + 1) & 0xF) | ((bsel(r.h.y, k + 1) >> 6) << 4);
    m1 = (bsel(r.h.w, k + 1) >> 4) | ((bsel(r.h.z, k + 1) >> 6) << 4);
  }
  const float d = h2f((uint16_t)(r.h.x & 0xffff)), dmin = h2f((uint16_t)(r.h.x >> 16));
  const float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
  const float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
  const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
  for (int i = 0; i < 32; i++) {
    const uint32_t byte = bsel(w[i >> 2], i & 3);
    y[i] = d1 * (float)(byte & 0xF) - mm1;
    y[32 + i] = d2 * (float)(byte >> 4) - mm2;
  }
}

template <>
__device__ __forceinline__ void dequant64<TPT_TYPE_Q6_K>(const uint8_t* row, int g, float* y) {
  // group (p, h): elements 128p + 32quad + 16h + i, quad = 0..3, i < 16; y holds them quad-major
  Raw<TPT_TYPE_Q6_K> r;
  load_raw<TPT_TYPE_Q6_K>(row, g, r);
  const int h = g & 1;
  const float d = h2f((uint16_t)r.d);
  const uint32_t qa[4] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w};
  const uint32_t qb[4] = {r.qb.x, r.qb.y, r.qb.z, r.qb.w};
  const uint32_t qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
  const float sc[4] = {(float)(int8_t)bsel(r.sc.x, h), (float)(int8_t)bsel(r.sc.x, h + 2),
                       (float)(int8_t)bsel(r.sc.y, h), (float)(int8_t)bsel(r.sc.y, h + 2)};
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const uint32_t a = bsel(qa[i >> 2], i & 3), b = bsel(qb[i >> 2], i & 3);
    const uint32_t hh = bsel(qh[i >> 2], i & 3);
    const int q0 = (int)((a & 0xF) | ((hh & 3) << 4)) - 32;
    const int q1 = (int)((b & 0xF) | (((hh >> 2) & 3) << 4)) - 32;
    const int q2 = (int)((a >> 4) | (((hh >> 4) & 3) << 4)) - 32;
    const int q3 = (int)((b >> 4) | (((hh >> 6) & 3) << 4)) - 32;
    y[i] = d * sc[0] * (float)q0;
    y[16 + i] = d * sc[1] * (float)q1;
    y[32 + i] = d * sc[2] * (float)q2;
    y[48 + i] = d * sc[3] * (float)q3;
  }
}

template <>
__device__ __forceinline__ void dequant64<TPT_TYPE_Q8_0>(const uint8_t* row, int g, float* y) {
  Raw<TPT_TYPE_Q8_0> r;
  load_raw<TPT_TYPE_Q8_0>(row, g, r);
  const float d0 = h2f((uint16_t)r.d0), d1 = h2f((uint16_t)r.d1);
  const uint32_t wa[8] = {r.a0.x, r.a0.y, r.a0.z, r.a0.w, r.a1.x, r.a1.y, r.a1.z, r.a1.w};
  const uint32_t wb[8] = {r.b0.x, r.b0.y, r.b0.z, r.b0.w, r.b1.x, r.b1.y, r.b1.z, r.b1.w};
#pragma unroll
  for (int i = 0; i < 32; i++) {
    y[i] = d0 * (float)(int8_t)bsel(wa[i >> 2], i & 3);
    y[32 + i] = d1 * (float)(int8_t)bsel(wb[i >> 2], i & 3);
  }
}

// element offset (within the row) of the e-th value dequant64 produces for group g
template <int WT>
__device__ __forceinline__ int elem_of(int g, int e) {
  if constexpr (WT == TPT_TYPE_Q6_K) {
    const int b = g >> 2, p = (g >> 1) & 1, h = g & 1;
    return 256 * b + 128 * p + 32 * (e >> 4) + 16 * h + (e & 15);
  } else {
    return 64 * g + e;
  }
}

template <int WT>
__global__ void __launch_bounds__(256) gemv_f32_kernel(const uint8_t* __restrict__ w,
                                                       const float* __restrict__ x,
                                                       float* __restrict__ y, int K, int N,
                                                       size_t row_stride) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= N) return;
  const uint8_t* rp = w + (size_t)row * row_stride;
  float acc = 0.f;
  for (int g = lane; g < K / 64; g += 64) {
    float v[64];
    dequant64<WT>(rp, g, v);
#pragma unroll
    for (int e = 0; e < 64; e++) acc = fmaf(v[e], x[elem_of<WT>(g, e)], acc);
  }
  acc = wave_sum(acc);
  if (lane == 0) y[row] = acc;
}

// ----------------------------------------------------------------- launch
template <int WT, int BPP, int RB, int NMAT, int KS, int D>
int launch_cfg(const tpt_ctx* ctx, const GemvArgs& a, int wg_per_cu, hipStream_t s,
               hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr) {
  Geo geo;
  const int nb = a.K / QK_K;
  geo.P = (nb + BPP - 1) / BPP;
  if (KS > geo.P) return fail(TPT_ERR_INVALID, "gemv: K split larger than the passes per row");
  const int ncu = ctx && ctx->n_cu > 0 ? ctx->n_cu : 256;
  const int cap = ncu * (wg_per_cu > 0 ? wg_per_cu : 1);
  const int rg = RB * (16 / BPP);
  const int unit = rg >= 2 ? rg : 2;  // whole row groups, even row ranges (RoPE pairs)
  int rpw = (a.N + cap - 1) / cap;
  rpw = (rpw + unit - 1) / unit * unit;
  geo.rows_per_wg = rpw;
  const int grid = (a.N + rpw - 1) / rpw;
  const size_t lds = lds_act_bytes(a.K, WT == TPT_TYPE_Q8_0) + 4 * (size_t)KS * rpw * NMAT;
  if (lds > 65536) return fail(TPT_ERR_UNSUPPORTED, "gemv: too many rows per workgroup for LDS");
  if (ev0 || ev1)  // the dispatch itself timestamps the events (no packets between kernels)
    hipExtLaunchKernelGGL((gemv_q8_kernel<WT, BPP, RB, NMAT, KS, D>), dim3((unsigned)grid), dim3(NT), lds, s,
                          ev0, ev1, 0, a, geo);
  else
    hipLaunchKernelGGL((gemv_q8_kernel<WT, BPP, RB, NMAT, KS, D>), dim3((unsigned)grid), dim3(NT), lds, s, a, geo);
  TPT_HIP(hipGetLastError());
  return TPT_OK;
}

// Launch shape by matrix shape: BPP from the row length (short rows share a pass), RB rows per
// step, D steps in flight per wave, one workgroup per CU.
template <int WT, int NMAT, int RB, int D>
int by_bpp(const tpt_ctx* ctx, const GemvArgs& a, hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
  const int nb = a.K / QK_K;
  if (nb >= 16) return launch_cfg<WT, 16, RB, NMAT, 1, D>(ctx, a, 1, s, e0, e1);
  if (nb >= 8) return launch_cfg<WT, 8, RB, NMAT, 1, D>(ctx, a, 1, s, e0, e1);
  if (nb >= 4) return launch_cfg<WT, 4, RB, NMAT, 1, D>(ctx, a, 1, s, e0, e1);
  if (nb >= 2) return launch_cfg<WT, 2, RB, NMAT, 1, D>(ctx, a, 1, s, e0, e1);
  return launch_cfg<WT, 1, RB, NMAT, 1, D>(ctx, a, 1, s, e0, e1);
}

template <int WT, int NMAT>
int dispatch_shape(const tpt_ctx* ctx, const GemvArgs& a, hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
  if constexpr (NMAT == 2) return by_bpp<WT, 2, 1, 2>(ctx, a, s, e0, e1);
  else {
    if (a.K > 8192) return by_bpp<WT, 1, 2, 2>(ctx, a, s, e0, e1);  // long rows: two rows per step
    return by_bpp<WT, 1, 1, 2>(ctx, a, s, e0, e1);
  }
}

}  // namespace

int launch_gemv_q8(const tpt_ctx* ctx, int wtype, const GemvArgs& a, hipStream_t s, hipEvent_t ev0,
                   hipEvent_t ev1) {
  if (a.K <= 0 || a.N <= 0 || a.K % 256) return fail(TPT_ERR_INVALID, "gemv: K must be a positive multiple of 256, N > 0");
  if (a.K > 64 * 256) return fail(TPT_ERR_UNSUPPORTED, "gemv: K > 16384 not supported");
  if (!a.w0 || !a.x) return fail(TPT_ERR_INVALID, "gemv: null weight/activation pointer");
  if (a.prologue == PRO_RMSNORM && !a.norm_w) return fail(TPT_ERR_INVALID, "gemv: rmsnorm prologue needs norm weights");
  if (a.epilogue == EPI_SWIGLU && !a.w1) return fail(TPT_ERR_INVALID, "gemv: swiglu needs two matrices");
  if (a.epilogue == EPI_ROPE_QKV && ((a.N & 1) || (a.row0 & 1) || (a.hd & 1)))
    return fail(TPT_ERR_INVALID, "gemv: rope epilogue needs even row counts");
  const bool two = a.epilogue == EPI_SWIGLU;
  switch (wtype) {
    case TPT_TYPE_Q4_K: return two ? dispatch_shape<TPT_TYPE_Q4_K, 2>(ctx, a, s, ev0, ev1) : dispatch_shape<TPT_TYPE_Q4_K, 1>(ctx, a, s, ev0, ev1);
    case TPT_TYPE_Q6_K: return two ? dispatch_shape<TPT_TYPE_Q6_K, 2>(ctx, a, s, ev0, ev1) : dispatch_shape<TPT_TYPE_Q6_K, 1>(ctx, a, s, ev0, ev1);
    case TPT_TYPE_Q8_0: return two ? dispatch_shape<TPT_TYPE_Q8_0, 2>(ctx, a, s, ev0, ev1) : dispatch_shape<TPT_TYPE_Q8_0, 1>(ctx, a, s, ev0, ev1);
  }
  return fail(TPT_ERR_UNSUPPORTED, "gemv: weight type must be Q4_K, Q6_K or Q8_0");
}

int launch_gemv_f32(int wtype, const uint8_t* w, const float* x, float* y, int K, int N,
                    hipStream_t s) {
  if (K <= 0 || N <= 0 || K % 256) return fail(TPT_ERR_INVALID, "gemv_f32: K must be a positive multiple of 256");
  const size_t rs = row_bytes(wtype, K);
  const dim3 grid((unsigned)((N + 3) / 4));
  switch (wtype) {
    case TPT_TYPE_Q4_K: hipLaunchKernelGGL(gemv_f32_kernel<TPT_TYPE_Q4_K>, grid, dim3(256), 0, s, w, x, y, K, N, rs); break;
    case TPT_TYPE_Q6_K: hipLaunchKernelGGL(gemv_f32_kernel<TPT_TYPE_Q6_K>, grid, dim3(256), 0, s, w, x, y, K, N, rs); break;
    case TPT_TYPE_Q8_0: hipLaunchKernelGGL(gemv_f32_kernel<TPT_TYPE_Q8_0>, grid, dim3(256), 0, s, w, x, y, K, N, rs); break;
    default: return fail(TPT_ERR_UNSUPPORTED, "gemv_f32: weight type must be Q4_K, Q6_K or Q8_0");
  }
  TPT_HIP(hipGetLastError());
  return TPT_OK;
}

}  // namespace tpt
