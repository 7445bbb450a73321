// Fused k-quant dequant-GEMV for bs=1 decode on gfx950.
//
// y[r] = sum_k W[r,k] * x[k], W in GGUF block layout (rows of K/256 super-blocks, uploaded
// unchanged), x fp32.  Replaces dequant_and_gemm (src-tauri/src/engine/wgpu_engine.rs:581-605:
// a full f32 dequant of W into a fresh buffer, then gemm.wgsl at M=1) and restates what the
// reference's CandleEngine computes on the CPU through candle 0.8.4 QMatMul:
//   k_quants::matmul -> BlockQ8K::from_float (activation quant) -> vec_dot_q4k_q8k /
//   vec_dot_q6k_q8k / vec_dot_q8_0_q8_0 (integer sums, f32 block scaling).
//
// Layout of the work (MI355X: 256 CUs, wave64, 160 KB LDS/CU, HBM3E):
//  * A persistent grid of ~1 workgroup per CU (512 threads = 8 waves).  Each wave owns a
//    contiguous range of rows, so a row's K/256 super-blocks stream as one contiguous run.
//  * Prologue, once per workgroup: the activation (optionally RMS-normalised first) is
//    quantized exactly like candle's CPU path into LDS: Q8_K (per 256: signed max-abs value,
//    iscale = -128/max, round half away from zero, clamp 127, d = 1/iscale, per-16 sums) for
//    k-quant weights, Q8_0 (per 32: d = amax/127 stored as f16, q = round(x/d)) for Q8_0.
//    The weight loads of each wave's first rows are issued before it, so the prologue runs
//    under HBM latency.
//  * Lanes: a "group" is 64 weights (Q4_K: 32 qs bytes of one super-block + its 16-byte
//    header; Q6_K: one (pass, half) slice of a super-block; Q8_0: two blocks).  LPR lanes
//    share a row, each lane owns GPL groups, and keeps its activation slice in registers for
//    every row it visits.  Integer dots use v_dot4_i32_i8; each group ends in f32 block
//    scaling; lanes reduce with cross-lane shuffles.
//  * Epilogues fuse what follows the GEMV in run_forward_pass (wgpu_engine.rs:373-486):
//    residual add, interleaved RoPE + fp16 KV-cache append, SiLU(gate)*up, greedy argmax.
#include "kernels.h"

namespace tpt {

namespace {

constexpr int NT = 512;  // threads per workgroup
constexpr int NW = NT / WAVE;

// ----------------------------------------------------------------- activation in registers
struct Act {
  int q[16];    // 64 int8 activation values of this lane's group, packed
  float d0, d1; // Q8_K: d0 = block d;  Q8_0: d of each 32-block
  int s[4];     // Q4_K: s[0], s[1] = sums over each 32;  Q6_K: per-16 sums of the 4 quads
};

__device__ __forceinline__ uint32_t bsel(uint32_t v, int i) { return (v >> (8 * i)) & 0xffu; }

// ----------------------------------------------------------------- raw weight slices
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
  const uint8_t* blk = row + (size_t)(g >> 2) * 210;  // 2-byte aligned: unaligned loads
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

// Q4_K x Q8_K for one group: restates vec_dot_q4k_q8k's per-block arithmetic
// (d_w*d_x * sum_j sc_j * sum(q4*q8)  -  dmin_w*d_x * sum_j m_j * bsum_j).
__device__ __forceinline__ float dot_group(const Raw<TPT_TYPE_Q4_K>& r, const Act& a, int g) {
  const int g4 = g & 3;
  // get_scale_min_k4 for j0 = 2*g4 and j1 = j0 + 1 (scales bytes: h.y = s[0..3],
  // h.z = s[4..7], h.w = s[8..11])
  int sc0, m0, sc1, m1;
  if (g4 < 2) {
    const int j0 = 2 * g4;
    sc0 = bsel(r.h.y, j0) & 63;
    m0 = bsel(r.h.z, j0) & 63;
    sc1 = bsel(r.h.y, j0 + 1) & 63;
    m1 = bsel(r.h.z, j0 + 1) & 63;
  } else {
    const int k = 2 * g4 - 4;
    sc0 = (bsel(r.h.w, k) & 0xF) | ((bsel(r.h.y, k) >> 6) << 4);
    m0 = (bsel(r.h.w, k) >> 4) | ((bsel(r.h.z, k) >> 6) << 4);
    sc1 = (bsel(r.h.w, k + 1) & 0xF) | ((bsel(r.h.y, k + 1) >> 6) << 4);
    m1 = (bsel(r.h.w, k + 1) >> 4) | ((bsel(r.h.z, k + 1) >> 6) << 4);
  }
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

// Q6_K x Q8_K for one group (pass p, half h): vec_dot_q6k_q8k's per-block arithmetic,
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
  const uint32_t slo = r.sc.x, shi = r.sc.y;
  const int sc0 = (int8_t)bsel(slo, h), sc1 = (int8_t)bsel(slo, h + 2);
  const int sc2 = (int8_t)bsel(shi, h), sc3 = (int8_t)bsel(shi, h + 2);
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

// ----------------------------------------------------------------- prologue (LDS)
// LDS layout: qs int8[K] | d float[K/bs] | s16 int[K/16] | scratch float[NW]
struct Lds {
  int* q32;
  float* d;
  int* s16;
  float* red;
};

__device__ __forceinline__ Lds lds_layout(char* smem, int K, bool q80) {
  Lds l;
  l.q32 = (int*)smem;
  l.d = (float*)(smem + K);
  const int nd = q80 ? K / QK8_0 : K / QK_K;
  l.s16 = (int*)(smem + K + 4 * nd);
  l.red = (float*)(smem + K + 4 * nd + 4 * (K / 16));
  return l;
}

__device__ __forceinline__ float eps_of(const GemvArgs& A) { return A.eps; }

__device__ __forceinline__ void barrier_lds() {
  // LDS-only barrier: outstanding global loads (the prefetched weights) stay in flight.
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Activation preload: the x (and RMSNorm weight) values a wave quantizes -- one float4 per lane
// per 256-element block, blocks b = wave, wave + NW, ... -- are loaded BEFORE the weight
// prefetch is issued: vmcnt retires loads in issue order, so the prologue must not wait
// behind the weights.
template <int MAXB>
struct XPre {
  float4 x[MAXB];
  float4 w[MAXB];
};

template <int MAXB>
__device__ __forceinline__ void preload_x(const GemvArgs& A, XPre<MAXB>& p) {
  // unconditional loads (indices clamped, a dummy source when there is no norm) so that the
  // waitcnt pass can count exactly how many later loads may stay in flight
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
template <int MAXB>
__device__ float rms_denominator(const GemvArgs& A, const XPre<MAXB>& p, float* red) {
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
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[wid] = ss;
  barrier_lds();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < NW; i++) t += red[i];
  return sqrtf(t / (float)A.K + eps_of(A));
}

// Q8_K quantization of one 256-block per wave iteration (BlockQ8K::from_float).
template <int MAXB>
__device__ void prologue_q8k(const GemvArgs& A, const XPre<MAXB>& p, const Lds& L) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int nb = A.K / QK_K;
  float m = 1.f;
  const bool norm = A.prologue == PRO_RMSNORM;
  if (norm) m = rms_denominator<MAXB>(A, p, L.red);
#pragma unroll
  for (int i = 0; i < MAXB; i++) {
    const int b = wid + i * NW;
    if (b >= nb) break;
    float4 v = p.x[i];
    if (norm) {
      const float4 w = p.w[i];
      v.x = v.x / m * w.x;
      v.y = v.y / m * w.y;
      v.z = v.z / m * w.z;
      v.w = v.w / m * w.w;
    }
    // the signed value of largest |x|, first occurrence winning ties
    float amax = fabsf(v.x), mx = v.x;
    int idx = lane * 4;
    if (fabsf(v.y) > amax) { amax = fabsf(v.y); mx = v.y; idx = lane * 4 + 1; }
    if (fabsf(v.z) > amax) { amax = fabsf(v.z); mx = v.z; idx = lane * 4 + 2; }
    if (fabsf(v.w) > amax) { amax = fabsf(v.w); mx = v.w; idx = lane * 4 + 3; }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float oa = __shfl_xor(amax, o, WAVE);
      const float om = __shfl_xor(mx, o, WAVE);
      const int oi = __shfl_xor(idx, o, WAVE);
      if (oa > amax || (oa == amax && oi < idx)) { amax = oa; mx = om; idx = oi; }
    }
    int packed = 0, qsum = 0;
    float d = 0.f;
    if (amax != 0.f) {
      const float iscale = -128.f / mx;
      const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        float r = roundf(iscale * e[j]);
        r = fminf(r, 127.f);
        r = fmaxf(r, -128.f);
        const int q = (int)r;
        qsum += q;
        packed |= (q & 0xff) << (8 * j);
      }
      d = 1.f / iscale;
    }
    L.q32[b * 64 + lane] = packed;
    qsum += __shfl_xor(qsum, 1, WAVE);
    qsum += __shfl_xor(qsum, 2, WAVE);
    if ((lane & 3) == 0) L.s16[b * 16 + (lane >> 2)] = qsum;
    if (lane == 0) L.d[b] = d;
  }
}

// Q8_0 activation quantization (BlockQ8_0::from_float): 8 lanes per 32-block.
template <int MAXB>
__device__ void prologue_q80(const GemvArgs& A, const XPre<MAXB>& p, const Lds& L) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int nb = A.K / 256;
  float m = 1.f;
  const bool norm = A.prologue == PRO_RMSNORM;
  if (norm) m = rms_denominator<MAXB>(A, p, L.red);
#pragma unroll
  for (int i = 0; i < MAXB; i++) {
    const int c = wid + i * NW;
    if (c >= nb) break;
    float4 v = p.x[i];
    if (norm) {
      const float4 w = p.w[i];
      v.x = v.x / m * w.x;
      v.y = v.y / m * w.y;
      v.z = v.z / m * w.z;
      v.w = v.w / m * w.w;
    }
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, WAVE));
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

template <int WT>
__device__ __forceinline__ void load_act(const Lds& L, int g, Act& a) {
  if constexpr (WT == TPT_TYPE_Q4_K) {
#pragma unroll
    for (int i = 0; i < 16; i++) a.q[i] = L.q32[16 * g + i];
    a.d0 = L.d[g >> 2];
    a.s[0] = L.s16[4 * g] + L.s16[4 * g + 1];
    a.s[1] = L.s16[4 * g + 2] + L.s16[4 * g + 3];
  } else if constexpr (WT == TPT_TYPE_Q6_K) {
    const int b = g >> 2, p = (g >> 1) & 1, h = g & 1;
#pragma unroll
    for (int quad = 0; quad < 4; quad++) {
      const int e0 = 256 * b + 128 * p + 32 * quad + 16 * h;
#pragma unroll
      for (int i = 0; i < 4; i++) a.q[4 * quad + i] = L.q32[e0 / 4 + i];
      a.s[quad] = L.s16[e0 / 16];
    }
    a.d0 = L.d[b];
  } else {
#pragma unroll
    for (int i = 0; i < 16; i++) a.q[i] = L.q32[16 * g + i];
    a.d0 = L.d[2 * g];
    a.d1 = L.d[2 * g + 1];
  }
}

// ----------------------------------------------------------------- the kernel
template <int LPR, int GPL, int NMAT>
struct Shape {
  static constexpr int RPW = WAVE / LPR;  // rows per wave pass (one per lane slot)
  static constexpr int RB = GPL >= 3 ? 1 : (GPL == 2 || NMAT == 2) ? 2 : 4;  // passes/chunk
  static constexpr int MAXB = (LPR * GPL / 4 + NW - 1) / NW;  // 256-blocks per wave (prologue)
};

template <int WT, int LPR, int GPL, int NMAT>
__global__ void __launch_bounds__(NT) gemv_q8_kernel(const GemvArgs A) {
  using S = Shape<LPR, GPL, NMAT>;
  constexpr int RPW = S::RPW, RB = S::RB, MAXB = S::MAXB;
  extern __shared__ __align__(16) char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int slot = lane / LPR, lr = lane % LPR;
  const int K = A.K, N = A.N, G = K / 64;
  const Lds L = lds_layout(smem, K, WT == TPT_TYPE_Q8_0);

  // contiguous chunk range of this wave; a chunk = RB*RPW consecutive rows
  const long units = (N + RPW - 1) / RPW;
  const long chunks = (units + RB - 1) / RB;
  const long W = (long)gridDim.x * NW, gw = (long)blockIdx.x * NW + wid;
  const long c_begin = gw * chunks / W, c_end = (gw + 1) * chunks / W;

  // 1. activation values this wave quantizes (issued first: see preload_x)
  XPre<MAXB> xp;
  preload_x<MAXB>(A, xp);
  int pos = 0;
  if (A.epilogue == EPI_ROPE_QKV) pos = A.state ? A.state->pos : A.pos_host;

  // 2. weight prefetch of the first chunk
  Raw<WT> raw[RB][GPL][NMAT];
  auto issue = [&](long c) {
#pragma unroll
    for (int r = 0; r < RB; r++) {
      long row = (c * RB + r) * RPW + slot;
      if (row >= N) row = N - 1;  // clamp: loads stay in bounds, result discarded
#pragma unroll
      for (int j = 0; j < GPL; j++) {
        int g = lr + j * LPR;
        if (g >= G) g = G - 1;
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
          const uint8_t* base = (m == 0 ? A.w0 : A.w1) + (size_t)row * A.row_stride;
          load_raw<WT>(base, g, raw[r][j][m]);
        }
      }
    }
  };
  issue(c_begin < c_end ? c_begin : (chunks > 0 ? chunks - 1 : 0));  // unconditional (see preload_x)

  // 3. activation quantization into LDS (runs under the prefetch's latency)
  if constexpr (WT == TPT_TYPE_Q8_0) prologue_q80<MAXB>(A, xp, L);
  else prologue_q8k<MAXB>(A, xp, L);
  barrier_lds();

  Act act[GPL];
#pragma unroll
  for (int j = 0; j < GPL; j++) {
    const int g = lr + j * LPR;
    load_act<WT>(L, g < G ? g : G - 1, act[j]);
  }

  unsigned long long best = 0;
  for (long c = c_begin; c < c_end; c++) {
    // epilogue inputs of this chunk, loaded before the next chunk's weights are issued
    // (unconditionally, from a dummy address when unused)
    float ein0[RB], ein1[RB];
#pragma unroll
    for (int r = 0; r < RB; r++) {
      long row = (c * RB + r) * RPW + slot;
      if (row >= N) row = N - 1;
      const float* p0 = A.x;
      const float* p1 = A.x;
      if (A.epilogue == EPI_RESID) {
        p0 = A.resid + row;
      } else if (A.epilogue == EPI_ROPE_QKV) {
        const int lrow = A.row0 + (int)row;
        const int rr = lrow < A.qd ? lrow : lrow - A.qd;
        const size_t ti = (size_t)pos * (A.hd / 2) + ((rr % A.hd) >> 1);
        p0 = A.rope_cos + ti;
        p1 = A.rope_sin + ti;
      }
      ein0[r] = *p0;
      ein1[r] = *p1;
    }

    float acc[RB][NMAT];
#pragma unroll
    for (int r = 0; r < RB; r++)
#pragma unroll
      for (int m = 0; m < NMAT; m++) {
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < GPL; j++) {
          const int g = lr + j * LPR;
          const float v = dot_group(raw[r][j][m], act[j], g);
          if ((j + 1) * LPR <= G || g < G) s += v;
        }
        acc[r][m] = group_sum<LPR>(s);
      }
    issue(c + 1 < c_end ? c + 1 : c);  // next rows' loads overlap this chunk's epilogue

#pragma unroll
    for (int r = 0; r < RB; r++) {
      const long row = (c * RB + r) * RPW + slot;
      const bool valid = row < N && lr == 0;
      switch (A.epilogue) {
        case EPI_STORE:
          if (valid) A.y[row] = acc[r][0];
          break;
        case EPI_RESID:
          if (valid) A.y[row] = acc[r][0] + ein0[r];
          break;
        case EPI_SWIGLU:
          if (valid) {
            const float g = acc[r][0];
            A.y[row] = g / (1.f + expf(-g)) * acc[r][NMAT - 1];
          }
          break;
        case EPI_ARGMAX:
          if (valid) {
            if (A.y) A.y[row] = acc[r][0];
            const unsigned long long key =
                ((unsigned long long)order_key(acc[r][0]) << 32) | (unsigned long long)row;
            best = key > best ? key : best;
          }
          break;
        case EPI_ROPE_QKV: {
          // rows come in (even, odd) pairs: consecutive passes when RPW == 1, adjacent slots
          // (lanes l and l + LPR) otherwise.
          float partner;
          bool first;
          if constexpr (RPW == 1 && RB == 1) {
            partner = 0.f;  // unreachable: the host rejects RoPE for this layout
            first = true;
          } else if constexpr (RPW == 1) {
            partner = acc[r ^ 1][0];
            first = (r & 1) == 0;
          } else {
            partner = __shfl_xor(acc[r][0], LPR, WAVE);
            first = (slot & 1) == 0;
          }
          if (valid) {
            const int lrow = A.row0 + (int)row;
            const float self = acc[r][0];
            const float x0 = first ? self : partner, x1 = first ? partner : self;
            if (lrow < A.qd + A.kd) {
              const bool isq = lrow < A.qd;
              const int rr = isq ? lrow : lrow - A.qd;
              const float cs = ein0[r], sn = ein1[r];
              // candle rope_i: dst[2i] = x0*cos - x1*sin; dst[2i+1] = x0*sin + x1*cos
              const float out = first ? (x0 * cs - x1 * sn) : (x0 * sn + x1 * cs);
              if (isq) {
                A.y[rr] = out;
              } else {
                const size_t ci = ((size_t)(rr / A.hd) * A.max_ctx + pos) * A.hd + rr % A.hd;
                if (A.kv_type == TPT_TYPE_F32) ((float*)A.kcache)[ci] = out;
                else ((uint16_t*)A.kcache)[ci] = f2h(out);
              }
            } else {
              const int rr = lrow - A.qd - A.kd;
              const size_t ci = ((size_t)(rr / A.hd) * A.max_ctx + pos) * A.hd + rr % A.hd;
              if (A.kv_type == TPT_TYPE_F32) ((float*)A.vcache)[ci] = self;
              else ((uint16_t*)A.vcache)[ci] = f2h(self);
            }
          }
        } break;
      }
    }
  }
  if (A.epilogue == EPI_ARGMAX) {
    // wave max of the 64-bit keys, one atomic per wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const unsigned long long ob = __shfl_xor(best, o, WAVE);
      best = ob > best ? ob : best;
    }
    if (lane == 0 && best) {
      unsigned long long* slot_p = A.amax + (A.state ? A.state->parity : 0);
      atomicMax(slot_p, best);
    }
  }
}

// ----------------------------------------------------------------- fp32-activation variant
// y[r] = sum_k dequant(W)[r,k] * x[k] (dequantized exactly like the oracle, fp32 FMA).  One
// wave per row, x read through the vector cache.  Not on the parity path (candle quantizes
// activations); kept for the fp32-activation GEMV report.
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

template <int WT, int LPR, int GPL, int NMAT>
int launch_one(const tpt_ctx* ctx, const GemvArgs& a, hipStream_t s) {
  const bool q80 = WT == TPT_TYPE_Q8_0;
  const size_t lds = (size_t)a.K + 4 * (q80 ? a.K / QK8_0 : a.K / QK_K) + 4 * (a.K / 16) + 4 * NW;
  constexpr int RPW = Shape<LPR, GPL, NMAT>::RPW, RB = Shape<LPR, GPL, NMAT>::RB;
  const long chunks = ((a.N + RPW - 1) / RPW + RB - 1) / RB;
  long grid = (chunks + NW - 1) / NW;
  const long cap = ctx && ctx->n_cu > 0 ? ctx->n_cu : 256;
  if (grid > cap) grid = cap;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL((gemv_q8_kernel<WT, LPR, GPL, NMAT>), dim3((unsigned)grid), dim3(NT), lds, s, a);
  TPT_HIP(hipGetLastError());
  return TPT_OK;
}

template <int WT, int NMAT>
int dispatch_layout(const tpt_ctx* ctx, const GemvArgs& a, hipStream_t s) {
  const int G = a.K / 64;
  if (G >= 64) {
    const int gpl = (G + 63) / 64;
    switch (gpl) {
      case 1: return launch_one<WT, 64, 1, NMAT>(ctx, a, s);
      case 2: return launch_one<WT, 64, 2, NMAT>(ctx, a, s);
      case 3:
      case 4:
        if constexpr (NMAT == 1) {
          if (a.epilogue == EPI_ROPE_QKV) return fail(TPT_ERR_UNSUPPORTED, "gemv: RoPE epilogue needs K <= 8192");
          return gpl == 3 ? launch_one<WT, 64, 3, 1>(ctx, a, s) : launch_one<WT, 64, 4, 1>(ctx, a, s);
        }
        return fail(TPT_ERR_UNSUPPORTED, "gemv: two-matrix epilogue needs K <= 8192");
      default: return fail(TPT_ERR_UNSUPPORTED, "gemv: K > 16384 not supported");
    }
  }
  if (G >= 32) return G == 32 ? launch_one<WT, 32, 1, NMAT>(ctx, a, s) : launch_one<WT, 32, 2, NMAT>(ctx, a, s);
  if (G >= 16) return G == 16 ? launch_one<WT, 16, 1, NMAT>(ctx, a, s) : launch_one<WT, 16, 2, NMAT>(ctx, a, s);
  if (G >= 8) return G == 8 ? launch_one<WT, 8, 1, NMAT>(ctx, a, s) : launch_one<WT, 8, 2, NMAT>(ctx, a, s);
  if (G >= 4) return G == 4 ? launch_one<WT, 4, 1, NMAT>(ctx, a, s) : launch_one<WT, 4, 2, NMAT>(ctx, a, s);
  return fail(TPT_ERR_UNSUPPORTED, "gemv: K must be a multiple of 256 (>= 256)");
}

}  // namespace

int launch_gemv_q8(const tpt_ctx* ctx, int wtype, const GemvArgs& a, hipStream_t s) {
  if (a.K <= 0 || a.N <= 0 || a.K % 256) return fail(TPT_ERR_INVALID, "gemv: K must be a positive multiple of 256, N > 0");
  if (!a.w0 || !a.x) return fail(TPT_ERR_INVALID, "gemv: null weight/activation pointer");
  if (a.prologue == PRO_RMSNORM && !a.norm_w) return fail(TPT_ERR_INVALID, "gemv: rmsnorm prologue needs norm weights");
  if (a.epilogue == EPI_SWIGLU && !a.w1) return fail(TPT_ERR_INVALID, "gemv: swiglu needs two matrices");
  if (a.epilogue == EPI_ROPE_QKV && ((a.N & 1) || (a.row0 & 1) || (a.hd & 1)))
    return fail(TPT_ERR_INVALID, "gemv: rope epilogue needs even row counts");
  const bool two = a.epilogue == EPI_SWIGLU;
  switch (wtype) {
    case TPT_TYPE_Q4_K: return two ? dispatch_layout<TPT_TYPE_Q4_K, 2>(ctx, a, s) : dispatch_layout<TPT_TYPE_Q4_K, 1>(ctx, a, s);
    case TPT_TYPE_Q6_K: return two ? dispatch_layout<TPT_TYPE_Q6_K, 2>(ctx, a, s) : dispatch_layout<TPT_TYPE_Q6_K, 1>(ctx, a, s);
    case TPT_TYPE_Q8_0: return two ? dispatch_layout<TPT_TYPE_Q8_0, 2>(ctx, a, s) : dispatch_layout<TPT_TYPE_Q8_0, 1>(ctx, a, s);
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
