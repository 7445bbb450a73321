// Prefill GEMM on MFMA: Y[M,N] = X[M,K] . W[N,K]^T with W in GGUF Q4_K blocks (uploaded
// unchanged), for M >= 16 tokens at once.
//
// Replaces the prefill of the reference engines: WgpuEngine runs one whole forward pass per
// prompt position through dequant_and_gemm + gemm.wgsl at M=1 (wgpu_engine.rs:254-261,
// 581-605); CandleEngine runs a batched forward whose QMatMul quantizes every activation row
// to Q8_K and takes integer dot products (candle_engine.rs:272-273; candle 0.8.4
// k_quants::matmul).  Two modes:
//  * GEMM_Q8K (the model's prefill): candle's arithmetic.  The activation arrives as Q8_K rows
//    (int8 q, f32 d per 256, per-16 sums); the weight tile is decoded into LDS as the exact
//    integers sc_j * q (<= 63 * 15, exact in fp16).  One MFMA chain covers at most 128
//    elements, so every partial sum is an integer below 2^24 and exact in f32; the two halves
//    of a super-block add with one rounding, as (float)isum does in candle.  The mins term
//    sum_j m_j * bsum_j is one more K=16 MFMA (per-16 sums <= 2032 and mins <= 63: exact).
//    Per block, in f32 as candle: y += (d_w * d_x) * isum - (dmin_w * d_x) * msum.
//  * GEMM_F16: the tile is dequantized into LDS as fp16 (d*sc*q - dmin*m rounded to fp16), the
//    activation is fp16, one fp32 MFMA chain over all of K.
// Tiling (MI355X: 160 KB LDS, wave64, v_mfma_f32_32x32x16_f16): 256 threads, a 128 x 128 tile
// of Y per workgroup, each wave 64 x 64 (2 x 2 MFMA tiles), K stepped one super-block (256) at
// a time through LDS; the next step's global loads are issued before the current step's MFMAs.
#include <hip/hip_ext.h>

#include "kernels.h"

namespace tpt {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int GT = 256;          // threads per workgroup
constexpr int BM = 128, BN = 128, BK = 256;
constexpr int LDK = BK + 8;      // fp16 per LDS row (16 B pad: conflict-free 16-byte reads)
constexpr int LDG = 16 + 8;      // per-16 sums / mins row

struct GemmSmem {
  _Float16 a[BM][LDK];
  _Float16 b[BN][LDK];
  _Float16 a16[BM][LDG];  // Q8K: activation per-16 sums of the block
  _Float16 b16[BN][LDG];  // Q8K: weight mins, each repeated for its two 16-element halves
  float dx[BM];           // Q8K: activation block scale
  float dw[BN], dm[BN];   // Q8K: weight d, dmin
};

// registers one thread stages for a K-step: 128 activation values and half a weight block
template <int MODE> struct Stage;
template <> struct Stage<GEMM_Q8K> {
  uint4 a[8];   // 128 int8
  uint4 a16;    // 8 per-16 sums (int16)
  float dx;     // block scale
  uint4 h;      // weight block header
  uint4 q[4];   // 64 qs bytes (half a block)
};
template <> struct Stage<GEMM_F16> {
  uint4 a[16];  // 128 fp16
  uint4 h;
  uint4 q[4];
};

__device__ __forceinline__ void get_scale_min(const uint4& h, int j, int* sc, int* m) {
  // get_scale_min_k4 (ggml/candle): scales bytes s[0..11] are h.y, h.z, h.w
  const uint32_t Y = h.y, Z = h.z, W = h.w;
  if (j < 4) {
    *sc = (Y >> (8 * j)) & 63;
    *m = (Z >> (8 * j)) & 63;
  } else {
    const int k = j - 4;
    *sc = ((W >> (8 * k)) & 0xF) | (((Y >> (8 * k + 6)) & 3) << 4);
    *m = ((W >> (8 * k + 4)) & 0xF) | (((Z >> (8 * k + 6)) & 3) << 4);
  }
}

template <int MODE>
__device__ __forceinline__ void stage_load(const GemmArgs& g, int m0, int n0, int kb, Stage<MODE>& st) {
  const int tid = threadIdx.x, r = tid >> 1, hf = tid & 1;
  int m = m0 + r;
  if (m >= g.M) m = g.M - 1;
  int n = n0 + r;
  if (n >= g.N) n = g.N - 1;
  if constexpr (MODE == GEMM_Q8K) {
    const uint4* src = (const uint4*)(g.aq + (size_t)m * g.K + (size_t)kb * 256 + 128 * hf);
#pragma unroll
    for (int i = 0; i < 8; i++) st.a[i] = src[i];
    st.a16 = *(const uint4*)(g.as16 + (size_t)m * (g.K / 16) + kb * 16 + 8 * hf);
    st.dx = g.ad[(size_t)m * (g.K / 256) + kb];
  } else {
    const uint4* src = (const uint4*)(g.af + (size_t)m * g.K + (size_t)kb * 256 + 128 * hf);
#pragma unroll
    for (int i = 0; i < 16; i++) st.a[i] = src[i];
  }
  const uint8_t* blk = g.w + (size_t)n * g.w_stride + (size_t)kb * 144;
  st.h = *(const uint4*)blk;
  const uint4* qs = (const uint4*)(blk + 16 + 64 * hf);
#pragma unroll
  for (int i = 0; i < 4; i++) st.q[i] = qs[i];
}

template <int MODE>
__device__ __forceinline__ void stage_store(const Stage<MODE>& st, GemmSmem& s) {
  const int tid = threadIdx.x, r = tid >> 1, hf = tid & 1;
  // activation row r, elements 128 hf .. +128
  if constexpr (MODE == GEMM_Q8K) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t w[4] = {st.a[i].x, st.a[i].y, st.a[i].z, st.a[i].w};
      half8 lo, hi;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const _Float16 v0 = (_Float16)(int8_t)(w[j] & 0xff), v1 = (_Float16)(int8_t)((w[j] >> 8) & 0xff);
        const _Float16 v2 = (_Float16)(int8_t)((w[j] >> 16) & 0xff), v3 = (_Float16)(int8_t)(w[j] >> 24);
        if (j < 2) { lo[4 * j] = v0; lo[4 * j + 1] = v1; lo[4 * j + 2] = v2; lo[4 * j + 3] = v3; }
        else { hi[4 * j - 8] = v0; hi[4 * j - 7] = v1; hi[4 * j - 6] = v2; hi[4 * j - 5] = v3; }
      }
      *(half8*)&s.a[r][128 * hf + 16 * i] = lo;
      *(half8*)&s.a[r][128 * hf + 16 * i + 8] = hi;
    }
    const uint32_t b[4] = {st.a16.x, st.a16.y, st.a16.z, st.a16.w};
    half8 v;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      v[2 * j] = (_Float16)(int16_t)(b[j] & 0xffff);
      v[2 * j + 1] = (_Float16)(int16_t)(b[j] >> 16);
    }
    *(half8*)&s.a16[r][8 * hf] = v;
    if (hf == 0) s.dx[r] = st.dx;
  } else {
#pragma unroll
    for (int i = 0; i < 16; i++) *(uint4*)&s.a[r][128 * hf + 8 * i] = st.a[i];
  }
  // weight row r, groups g = 2 hf, 2 hf + 1 (elements 128 hf .. +128): qs[32g + l] holds element
  // 64g + l (low nibble, sub-block 2g) and 64g + 32 + l (high nibble, sub-block 2g + 1)
  const float d = h2f((uint16_t)(st.h.x & 0xffff)), dmin = h2f((uint16_t)(st.h.x >> 16));
#pragma unroll
  for (int gg = 0; gg < 2; gg++) {
    const int g = 2 * hf + gg;
    int sc0, m0, sc1, m1;
    get_scale_min(st.h, 2 * g, &sc0, &m0);
    get_scale_min(st.h, 2 * g + 1, &sc1, &m1);
    const uint4 q0 = st.q[2 * gg], q1 = st.q[2 * gg + 1];
    const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    const int e0 = 64 * g;
#pragma unroll
    for (int c = 0; c < 4; c++) {  // 8 consecutive elements per half8 store
      half8 lo, hi;
#pragma unroll
      for (int t = 0; t < 8; t++) {
        const uint32_t byte = (w[2 * c + t / 4] >> (8 * (t % 4))) & 0xff;
        const int ql = byte & 0xF, qh = byte >> 4;
        if constexpr (MODE == GEMM_Q8K) {
          lo[t] = (_Float16)(sc0 * ql);
          hi[t] = (_Float16)(sc1 * qh);
        } else {
          const float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
          const float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
          lo[t] = (_Float16)(d1 * (float)ql - mm1);
          hi[t] = (_Float16)(d2 * (float)qh - mm2);
        }
      }
      *(half8*)&s.b[r][e0 + 8 * c] = lo;
      *(half8*)&s.b[r][e0 + 32 + 8 * c] = hi;
    }
    if constexpr (MODE == GEMM_Q8K) {
      // mins of sub-blocks 2g, 2g + 1, each for its two 16-element halves (16-sums 8g .. 8g+3)
      s.b16[r][4 * g] = (_Float16)m0;
      s.b16[r][4 * g + 1] = (_Float16)m0;
      s.b16[r][4 * g + 2] = (_Float16)m1;
      s.b16[r][4 * g + 3] = (_Float16)m1;
    }
  }
  if constexpr (MODE == GEMM_Q8K) {
    if (hf == 0) {
      s.dw[r] = d;
      s.dm[r] = dmin;
    }
  }
}

template <int MODE>
__global__ void __launch_bounds__(GT, 1) gemm_q4k_kernel(const GemmArgs g) {
  __shared__ GemmSmem s;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid >> 1, wn = wid & 1;  // wave tile: rows 64 wm .., cols 64 wn ..
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int nkb = g.K / 256;
  const int lr = lane & 31, lk = 8 * (lane >> 5);  // MFMA operand lane mapping

  floatx16 out[2][2];
  floatx16 acc0[2][2], acc1[2][2], accm[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      out[i][j] = floatx16{};
      acc0[i][j] = floatx16{};
      acc1[i][j] = floatx16{};
      accm[i][j] = floatx16{};
    }

  Stage<MODE> st;
  stage_load<MODE>(g, m0, n0, 0, st);
  for (int kb = 0; kb < nkb; kb++) {
    __syncthreads();  // the previous step's MFMAs are done with the LDS tiles
    stage_store<MODE>(st, s);
    __syncthreads();
    // next step's loads in flight during the MFMAs (unconditional: the last step re-reads itself)
    stage_load<MODE>(g, m0, n0, kb + 1 < nkb ? kb + 1 : kb, st);

#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      half8 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; i++) a[i] = *(const half8*)&s.a[64 * wm + 32 * i + lr][kk + lk];
#pragma unroll
      for (int j = 0; j < 2; j++) b[j] = *(const half8*)&s.b[64 * wn + 32 * j + lr][kk + lk];
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
          if constexpr (MODE == GEMM_Q8K) {
            if (kk < 128) acc0[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc0[i][j], 0, 0, 0);
            else acc1[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc1[i][j], 0, 0, 0);
          } else {
            out[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], out[i][j], 0, 0, 0);
          }
        }
    }
    if constexpr (MODE == GEMM_Q8K) {
      half8 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; i++) a[i] = *(const half8*)&s.a16[64 * wm + 32 * i + lr][lk];
#pragma unroll
      for (int j = 0; j < 2; j++) b[j] = *(const half8*)&s.b16[64 * wn + 32 * j + lr][lk];
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
          accm[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], floatx16{}, 0, 0, 0);
          // per block, candle's f32 arithmetic: y += (d_w d_x) isum - (dmin_w d_x) msum
          const int col = 64 * wn + 32 * j + lr;
          const float dw = s.dw[col], dm = s.dm[col];
#pragma unroll
          for (int e = 0; e < 16; e++) {
            const int row = 64 * wm + 32 * i + (e / 4) * 8 + (lane >> 5) * 4 + (e % 4);
            const float dx = s.dx[row];
            const float isum = acc0[i][j][e] + acc1[i][j][e];
            const float dd = dw * dx, ddm = dm * dx;
            const float v = dd * isum - ddm * accm[i][j][e];
            out[i][j][e] = out[i][j][e] + v;
          }
          acc0[i][j] = floatx16{};
          acc1[i][j] = floatx16{};
        }
    }
  }

  // epilogue: y[m][n] = out (+ resid[m][n])
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int n = n0 + 64 * wn + 32 * j + lr;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int m = m0 + 64 * wm + 32 * i + (e / 4) * 8 + (lane >> 5) * 4 + (e % 4);
        if (m < g.M && n < g.N) {
          float v = out[i][j][e];
          if (g.resid) v = v + g.resid[(size_t)m * g.ldr + n];
          g.y[(size_t)m * g.ldy + n] = v;
        }
      }
    }
}

// One workgroup (4 waves) per activation row: optional SwiGLU (candle: silu(w1 x) * (w3 x)),
// optional rms_norm (m = sqrt(sum(x^2)/K + eps), y = x / m * w), then per 256-block the Q8_K
// quantization of BlockQ8K::from_float (the GEMV prologue's arithmetic) or fp16 conversion.
__global__ void __launch_bounds__(256) act_prep_kernel(const ActPrepArgs a) {
  __shared__ float red[4];
  const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int K = a.K, nb = K / 256;
  const float4* xr = (const float4*)(a.x + (size_t)m * a.ldx);
  const float4* ur = a.x2 ? (const float4*)(a.x2 + (size_t)m * a.ldx) : nullptr;
  auto value = [&](int i) {  // element group i (4 floats) after SwiGLU
    float4 v = xr[i];
    if (ur) {
      const float4 u = ur[i];
      v.x = silu_mul(v.x, u.x);
      v.y = silu_mul(v.y, u.y);
      v.z = silu_mul(v.z, u.z);
      v.w = silu_mul(v.w, u.w);
    }
    return v;
  };
  float rms = 1.f;
  if (a.norm_w) {
    float ss = 0.f;
    for (int i = tid; i < K / 4; i += 256) {
      const float4 v = value(i);
      ss = fmaf(v.x, v.x, ss);
      ss = fmaf(v.y, v.y, ss);
      ss = fmaf(v.z, v.z, ss);
      ss = fmaf(v.w, v.w, ss);
    }
    ss = wave_sum_dpp(ss);
    if (lane == 0) red[wid] = ss;
    __syncthreads();
    rms = sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)K + a.eps);
  }
  const float4* nw = (const float4*)a.norm_w;
  for (int b = wid; b < nb; b += 4) {
    float4 v = value(b * 64 + lane);
    if (nw) {
      const float4 w = nw[b * 64 + lane];
      v.x = v.x / rms * w.x;
      v.y = v.y / rms * w.y;
      v.z = v.z / rms * w.z;
      v.w = v.w / rms * w.w;
    }
    const float e[4] = {v.x, v.y, v.z, v.w};
    if (a.mode == GEMM_Q8K) {
      int qsum;
      float d;
      const int packed = q8k_block_wave(e, &qsum, &d);
      ((int*)(a.aq + (size_t)m * K + (size_t)b * 256))[lane] = packed;
      if ((lane & 3) == 0) a.as16[(size_t)m * (K / 16) + b * 16 + (lane >> 2)] = (int16_t)qsum;
      if (lane == 0) a.ad[(size_t)m * nb + b] = d;
    } else {
      uint2 h;
      h.x = (uint32_t)f2h(e[0]) | ((uint32_t)f2h(e[1]) << 16);
      h.y = (uint32_t)f2h(e[2]) | ((uint32_t)f2h(e[3]) << 16);
      ((uint2*)(a.af + (size_t)m * K + (size_t)b * 256))[lane] = h;
    }
  }
}

}  // namespace

int launch_act_prep(const ActPrepArgs& a, hipStream_t s) {
  if (a.M <= 0 || a.K <= 0 || a.K % 256 || a.ldx < a.K || a.ldx % 4) return fail(TPT_ERR_INVALID, "act_prep: bad shape");
  if (!a.x) return fail(TPT_ERR_INVALID, "act_prep: null input");
  if (a.mode == GEMM_Q8K ? (!a.aq || !a.ad || !a.as16) : !a.af) return fail(TPT_ERR_INVALID, "act_prep: null output");
  hipLaunchKernelGGL(act_prep_kernel, dim3((unsigned)a.M), dim3(256), 0, s, a);
  TPT_HIP(hipGetLastError());
  return TPT_OK;
}

int launch_gemm_q4k(const GemmArgs& g, hipStream_t s) { return launch_gemm_q4k_timed(g, s, nullptr, nullptr); }

int launch_gemm_q4k_timed(const GemmArgs& g, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  if (g.M <= 0 || g.N <= 0 || g.K <= 0 || g.K % 256) return fail(TPT_ERR_INVALID, "gemm: K must be a positive multiple of 256, M and N positive");
  if (!g.w || !g.y) return fail(TPT_ERR_INVALID, "gemm: null weight/output pointer");
  if (g.mode == GEMM_Q8K && (!g.aq || !g.ad || !g.as16)) return fail(TPT_ERR_INVALID, "gemm: Q8_K mode needs q, d and per-16 sums");
  if (g.mode == GEMM_F16 && !g.af) return fail(TPT_ERR_INVALID, "gemm: F16 mode needs fp16 activations");
  if ((g.w_stride % 16) || ((uintptr_t)g.w % 16)) return fail(TPT_ERR_INVALID, "gemm: weight rows must be 16-byte aligned");
  const dim3 grid((unsigned)((g.N + BN - 1) / BN), (unsigned)((g.M + BM - 1) / BM));
  if (g.mode == GEMM_Q8K) hipExtLaunchKernelGGL(gemm_q4k_kernel<GEMM_Q8K>, grid, dim3(GT), 0, s, ev0, ev1, 0, g);
  else hipExtLaunchKernelGGL(gemm_q4k_kernel<GEMM_F16>, grid, dim3(GT), 0, s, ev0, ev1, 0, g);
  TPT_HIP(hipGetLastError());
  return TPT_OK;
}

}  // namespace tpt
