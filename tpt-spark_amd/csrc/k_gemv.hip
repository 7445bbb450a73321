// Fused dequant-GEMV (k-quant, Q8_0 / Q4_0 and F16 weights) for bs=1 decode on gfx950.
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
//    bytes, its 8 scales and d; Q8_0: two 34-byte blocks; F16: 128 bytes, as eight 16-byte
//    runs interleaved with the other three lanes of the 256 weights).  A "pass" covers BPP super-blocks
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
//    Q8_0 (per 32: d = amax/127 rounded to f16, q = round(x/d)) for Q8_0 weights.  F16 weights
//    are candle's dequantize-then-f32-matmul: x (or its RMSNorm) stays f32 in LDS and the
//    group dot is 64 f32 FMAs over the exactly widened weights.  The x loads
//    are issued first and the first step's weight loads right after, so the prologue runs
//    under HBM latency.
//  * Integer dots use v_dot4_i32_i8; each group ends in f32 block scaling (candle's per-block
//    arithmetic), lanes accumulate in f32 and a row is reduced across its lanes once, with
//    DPP.  Row results go to LDS, and after a workgroup barrier the epilogue stores them:
//    plain, + residual, SiLU(gate)*up, interleaved RoPE + KV-cache append, or greedy argmax
//    (what follows the GEMV in run_forward_pass, wgpu_engine.rs:373-486).
#include <hip/hip_ext.h>

#include "kernels.h"


#include "gemv_dev.h"

namespace tpt {

namespace {

using namespace gemv;

template <int WT, int BPP, int RB, int NMAT, int KS, int D, bool NORM, bool ONEPASS>
__global__ void __launch_bounds__(NT, 1) gemv_q8_kernel(const GemvArgs A, const Geo geo) {
  extern __shared__ __align__(16) char smem[];
  gemv_run<WT, BPP, RB, NMAT, KS, D, NORM, ONEPASS>(A, geo, blockIdx.x, smem, NoHook());
}

// The launch of one instantiation (ev0/ev1: dispatch-stamped events, hipExtLaunchKernelGGL).
template <int WT, int BPP, int RB, int NMAT, int KS, int D, bool NORM, bool ONEPASS>
void launch_inst(const GemvArgs& a, const Geo& geo, int grid, size_t lds, hipStream_t s, hipEvent_t ev0,
                 hipEvent_t ev1) {
  if (ev0 || ev1)
    hipExtLaunchKernelGGL((gemv_q8_kernel<WT, BPP, RB, NMAT, KS, D, NORM, ONEPASS>), dim3((unsigned)grid),
                          dim3(NT), lds, s, ev0, ev1, 0, a, geo);
  else
    hipLaunchKernelGGL((gemv_q8_kernel<WT, BPP, RB, NMAT, KS, D, NORM, ONEPASS>), dim3((unsigned)grid),
                       dim3(NT), lds, s, a, geo);
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

template <>
__device__ __forceinline__ void dequant64<TPT_TYPE_Q5_K>(const uint8_t* row, int g, float* y) {
  // as Q4_K, values nibble + 16 * bit of qh[l]
  Raw<TPT_TYPE_Q5_K> r;
  load_raw<TPT_TYPE_Q5_K>(row, g, r);
  const int j0 = 2 * (g & 3);
  auto s = [&](int k) {  // scales byte k: header bytes 4 + k
    return (int)bsel(k < 4 ? r.h.y : k < 8 ? r.h.z : r.h.w, k & 3);
  };
  int sc[2], mn[2];
#pragma unroll
  for (int t = 0; t < 2; t++) {
    const int j = j0 + t;
    if (j < 4) {
      sc[t] = s(j) & 63;
      mn[t] = s(j + 4) & 63;
    } else {
      sc[t] = (s(j + 4) & 0xF) | ((s(j - 4) >> 6) << 4);
      mn[t] = (s(j + 4) >> 4) | ((s(j) >> 6) << 4);
    }
  }
  const float d = h2f((uint16_t)(r.h.x & 0xffff)), dmin = h2f((uint16_t)(r.h.x >> 16));
  const float d1 = d * (float)sc[0], mm1 = dmin * (float)mn[0];
  const float d2 = d * (float)sc[1], mm2 = dmin * (float)mn[1];
  const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
  const uint32_t qh[8] = {r.ha.x, r.ha.y, r.ha.z, r.ha.w, r.hb.x, r.hb.y, r.hb.z, r.hb.w};
#pragma unroll
  for (int i = 0; i < 32; i++) {
    const uint32_t byte = bsel(w[i >> 2], i & 3), hb = bsel(qh[i >> 2], i & 3);
    y[i] = d1 * (float)((byte & 0xF) + (((hb >> j0) & 1) << 4)) - mm1;
    y[32 + i] = d2 * (float)((byte >> 4) + (((hb >> (j0 + 1)) & 1) << 4)) - mm2;
  }
}

template <>
__device__ __forceinline__ void dequant64<TPT_TYPE_F16>(const uint8_t* row, int g, float* y) {
  const uint4* p = (const uint4*)(row + (size_t)g * 128);  // 64 contiguous weights
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const uint4 v = p[i];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      y[8 * i + 2 * j] = h2f((uint16_t)(w[j] & 0xffff));
      y[8 * i + 2 * j + 1] = h2f((uint16_t)(w[j] >> 16));
    }
  }
}

template <>
__device__ __forceinline__ void dequant64<TPT_TYPE_Q4_0>(const uint8_t* row, int g, float* y) {
  Raw<TPT_TYPE_Q4_0> r;
  load_raw<TPT_TYPE_Q4_0>(row, g, r);
  const float d0 = h2f((uint16_t)r.d0), d1 = h2f((uint16_t)r.d1);
  const uint32_t wa[4] = {r.a.x, r.a.y, r.a.z, r.a.w}, wb[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const uint32_t ba = bsel(wa[i >> 2], i & 3), bb = bsel(wb[i >> 2], i & 3);
    y[i] = (float)((int)(ba & 0xF) - 8) * d0;
    y[16 + i] = (float)((int)(ba >> 4) - 8) * d0;
    y[32 + i] = (float)((int)(bb & 0xF) - 8) * d1;
    y[48 + i] = (float)((int)(bb >> 4) - 8) * d1;
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
// grid_out: when given, only the workgroup count is computed (nothing is launched)
template <int WT, int BPP, int RB, int NMAT, int KS, int D>
int launch_cfg(const tpt_ctx* ctx, const GemvArgs& a, int wg_per_cu, hipStream_t s,
               hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr, int* grid_out = nullptr) {
  Geo geo;
  const int nb = a.K / QK_K;
  geo.P = (nb + BPP - 1) / BPP;
  if (KS > geo.P) return fail(TPT_ERR_INVALID, "gemv: K split larger than the passes per row");
  const int ncu = ctx && ctx->n_cu > 0 ? ctx->n_cu : 256;
  const int cap = ncu * (wg_per_cu > 0 ? wg_per_cu : 1);
  const int rg = RB * (16 / BPP);
  const int unit = rg >= 2 ? rg : 2;  // whole row groups, even row ranges (RoPE pairs)
  int rpw = (a.N + cap - 1) / cap;
  // very short Q4_K matrices (fewer than 8 rows per CU): 16 rows per workgroup, so that fewer
  // workgroups each fetch the whole activation (4096->1024: 64 instead of 256, same time); the
  // heavier Q6_K and Q8_0 rows keep every CU (4096->1024 measured 5-10% slower on 64)
  if (rpw < 8 && a.K <= 8192 && NMAT == 1 && WT == TPT_TYPE_Q4_K) rpw = 16;
  rpw = (rpw + unit - 1) / unit * unit;
  geo.rows_per_wg = rpw;
  const int grid = (a.N + rpw - 1) / rpw;
  const size_t lds = lds_act_bytes(a.K, act_kind<WT>()) + 4 * (size_t)KS * rpw * NMAT * RowParts<BPP>::N;
  if (lds > 65536)
    return fail(TPT_ERR_UNSUPPORTED, act_kind<WT>() == ACT_F32
                                         ? "gemv: F16 weights need K * 4 bytes of LDS (K <= 15360)"
                                         : "gemv: too many rows per workgroup for LDS");
  if (grid_out) {
    *grid_out = grid;
    return TPT_OK;
  }
  const bool norm = a.prologue == PRO_RMSNORM, one = geo.P == KS;  // one pass per k-split wave
  if (norm && one) launch_inst<WT, BPP, RB, NMAT, KS, D, true, true>(a, geo, grid, lds, s, ev0, ev1);
  else if (norm) launch_inst<WT, BPP, RB, NMAT, KS, D, true, false>(a, geo, grid, lds, s, ev0, ev1);
  else if (one) launch_inst<WT, BPP, RB, NMAT, KS, D, false, true>(a, geo, grid, lds, s, ev0, ev1);
  else launch_inst<WT, BPP, RB, NMAT, KS, D, false, false>(a, geo, grid, lds, s, ev0, ev1);
  TPT_HIP(hipGetLastError());
  return TPT_OK;
}

// Launch shape by matrix shape: BPP from the row length (short rows share a pass), RB rows per
// step, D steps in flight per wave, one workgroup per CU.
template <int WT, int NMAT, int RB, int D>
int by_bpp(const tpt_ctx* ctx, const GemvArgs& a, hipStream_t s, hipEvent_t e0, hipEvent_t e1, int* g) {
  const int nb = a.K / QK_K;
  if (nb >= 16) return launch_cfg<WT, 16, RB, NMAT, 1, D>(ctx, a, 1, s, e0, e1, g);
  if (nb >= 8) return launch_cfg<WT, 8, RB, NMAT, 1, D>(ctx, a, 1, s, e0, e1, g);
  if (nb >= 4) return launch_cfg<WT, 4, RB, NMAT, 1, D>(ctx, a, 1, s, e0, e1, g);
  if (nb >= 2) return launch_cfg<WT, 2, RB, NMAT, 1, D>(ctx, a, 1, s, e0, e1, g);
  return launch_cfg<WT, 1, RB, NMAT, 1, D>(ctx, a, 1, s, e0, e1, g);
}

template <int WT, int NMAT>
int dispatch_shape(const tpt_ctx* ctx, const GemvArgs& a, hipStream_t s, hipEvent_t e0, hipEvent_t e1,
                   int* g) {
  if constexpr (NMAT == 2) return by_bpp<WT, 2, 1, 2>(ctx, a, s, e0, e1, g);
  else if constexpr (WT == TPT_TYPE_F16) return by_bpp<WT, 1, 1, 2>(ctx, a, s, e0, e1, g);  // 128 B per group
  else {
    // Q6_K and Q8_0 (five and six loads per lane and step, against Q4_K's three): one step in
    // flight per wave, one row per step (4096->14336: Q8_0 18.1 -> 14.3 us, Q6_K 12.2 -> 11.7 us;
    // two steps or two rows per step were slower at every shape)
    if constexpr (WT == TPT_TYPE_Q6_K || WT == TPT_TYPE_Q8_0) return by_bpp<WT, 1, 1, 1>(ctx, a, s, e0, e1, g);
    // Q4_K and the rest: two steps in flight; long rows two rows per step
    if (a.K > 8192) return by_bpp<WT, 1, 2, 2>(ctx, a, s, e0, e1, g);
    return by_bpp<WT, 1, 1, 2>(ctx, a, s, e0, e1, g);
  }
}

int dispatch_type(const tpt_ctx* ctx, int wtype, const GemvArgs& a, hipStream_t s, hipEvent_t ev0,
                  hipEvent_t ev1, int* g) {
  const bool two = a.epilogue == EPI_SWIGLU;
  switch (wtype) {
    case TPT_TYPE_Q4_K: return two ? dispatch_shape<TPT_TYPE_Q4_K, 2>(ctx, a, s, ev0, ev1, g) : dispatch_shape<TPT_TYPE_Q4_K, 1>(ctx, a, s, ev0, ev1, g);
    case TPT_TYPE_Q6_K: return two ? dispatch_shape<TPT_TYPE_Q6_K, 2>(ctx, a, s, ev0, ev1, g) : dispatch_shape<TPT_TYPE_Q6_K, 1>(ctx, a, s, ev0, ev1, g);
    case TPT_TYPE_Q8_0: return two ? dispatch_shape<TPT_TYPE_Q8_0, 2>(ctx, a, s, ev0, ev1, g) : dispatch_shape<TPT_TYPE_Q8_0, 1>(ctx, a, s, ev0, ev1, g);
    case TPT_TYPE_Q5_K: return two ? dispatch_shape<TPT_TYPE_Q5_K, 2>(ctx, a, s, ev0, ev1, g) : dispatch_shape<TPT_TYPE_Q5_K, 1>(ctx, a, s, ev0, ev1, g);
    case TPT_TYPE_Q4_0: return two ? dispatch_shape<TPT_TYPE_Q4_0, 2>(ctx, a, s, ev0, ev1, g) : dispatch_shape<TPT_TYPE_Q4_0, 1>(ctx, a, s, ev0, ev1, g);
    case TPT_TYPE_F16: return two ? dispatch_shape<TPT_TYPE_F16, 2>(ctx, a, s, ev0, ev1, g) : dispatch_shape<TPT_TYPE_F16, 1>(ctx, a, s, ev0, ev1, g);
  }
  return fail(TPT_ERR_UNSUPPORTED, "gemv: weight type must be Q4_K, Q5_K, Q6_K, Q8_0, Q4_0 or F16");
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
  if (a.prologue == PRO_RMSNORM && a.ssq_in && (a.n_ssq < 1 || a.n_ssq > kSsqMax))
    return fail(TPT_ERR_INVALID, "gemv: rmsnorm partial sums must number 1 .. 256");
  return dispatch_type(ctx, wtype, a, s, ev0, ev1, nullptr);
}

int gemv_grid(const tpt_ctx* ctx, int wtype, const GemvArgs& a) {
  if (a.K <= 0 || a.N <= 0 || a.K % 256 || a.K > 64 * 256) return 0;
  int g = 0;
  if (dispatch_type(ctx, wtype, a, nullptr, nullptr, nullptr, &g) != TPT_OK) return 0;
  return g;
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
    case TPT_TYPE_Q5_K: hipLaunchKernelGGL(gemv_f32_kernel<TPT_TYPE_Q5_K>, grid, dim3(256), 0, s, w, x, y, K, N, rs); break;
    case TPT_TYPE_Q4_0: hipLaunchKernelGGL(gemv_f32_kernel<TPT_TYPE_Q4_0>, grid, dim3(256), 0, s, w, x, y, K, N, rs); break;
    case TPT_TYPE_F16: hipLaunchKernelGGL(gemv_f32_kernel<TPT_TYPE_F16>, grid, dim3(256), 0, s, w, x, y, K, N, rs); break;
    default: return fail(TPT_ERR_UNSUPPORTED, "gemv_f32: weight type must be Q4_K, Q5_K, Q6_K, Q8_0, Q4_0 or F16");
  }
  TPT_HIP(hipGetLastError());
  return TPT_OK;
}

}  // namespace tpt
