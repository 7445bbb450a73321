// Split-K (flash-decoding) GQA attention for one query position over an fp16 KV cache.
//
// Replaces the three-pass attention.wgsl (src-tauri/src/engine/shaders/attention.wgsl:31-170,
// dispatch_attention wgpu_engine.rs:666-726: scores materialised in f32 for every head and
// position, then softmax, then P.V) and restates what candle's quantized_llama computes on the
// CPU for a decode step: repeat_kv (head h reads kv head h / (Nq/Nkv)),
// att = (q . k) * f32(1/sqrt(hd)), softmax_last_dim, att . v.
//
// Cache layout [Nkv][L_stride][hd] fp16 (one layer): the K and V rows of a kv head are
// contiguous over positions, so a chunk of positions streams as one contiguous run.
// Grid (n_chunks, Nkv), 256 threads.  A workgroup reads each K and V row of its chunk once
// and serves all G = Nq/Nkv query heads of the group:
//   phase 1: 16 lanes per position (hd/16 dims each) dot the G queries, scores -> LDS;
//   phase 2: chunk max per head, p = exp(s - max), partial o = sum p*v and l = sum p;
//   merge:   the last workgroup of a kv head (atomic counter) combines the chunks with the
//            log-sum-exp rule and writes o; it also returns the counter to zero.
#include "kernels.h"

namespace tpt {
namespace {

constexpr int ANT = 256;
constexpr int ANW = ANT / WAVE;
constexpr int CL_MAX = 1024;  // positions per chunk held in LDS

template <int HD>
__device__ __forceinline__ void load_half_slice(const uint16_t* p, float* out) {
  constexpr int DPL = HD / 16;
  if constexpr (DPL == 8) {
    const uint4 v = *(const uint4*)p;
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      out[2 * i] = h2f((uint16_t)(w[i] & 0xffff));
      out[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
    }
  } else if constexpr (DPL == 6) {
    const uint32_t* q = (const uint32_t*)p;
    const uint32_t w[3] = {q[0], q[1], q[2]};
#pragma unroll
    for (int i = 0; i < 3; i++) {
      out[2 * i] = h2f((uint16_t)(w[i] & 0xffff));
      out[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
    }
  } else {
    static_assert(DPL == 4, "head_dim must be 64, 96 or 128");
    const uint2 v = *(const uint2*)p;
    const uint32_t w[2] = {v.x, v.y};
#pragma unroll
    for (int i = 0; i < 2; i++) {
      out[2 * i] = h2f((uint16_t)(w[i] & 0xffff));
      out[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
    }
  }
}

template <int HD, int G>
__global__ void __launch_bounds__(ANT) attn_decode_kernel(const AttnArgs a, const float scale) {
  constexpr int DPL = HD / 16;
  constexpr int PSTRIDE = HD + 2;  // partial record: o[HD], m, l
  __shared__ float s_sc[G][CL_MAX];
  __shared__ float s_red[ANW][G];
  __shared__ float s_o[16][G][HD];
  __shared__ float s_l[16][G];
  __shared__ int s_last;

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int li = lane & 15, pg = wid * 4 + (lane >> 4);  // position group 0..15
  const int kvh = blockIdx.y, chunk = blockIdx.x, nch = gridDim.x;
  const int L = a.state ? a.state->pos + 1 : a.L_host;
  int CL = (L + nch - 1) / nch;
  CL = (CL + 15) & ~15;
  if (CL > CL_MAX) CL = CL_MAX;  // the caller sizes n_chunks so that this never binds
  const int p0 = chunk * CL;
  const int p1 = min(L, p0 + CL);

  const uint16_t* K = a.kc + (size_t)kvh * a.L_stride * HD + li * DPL;
  const uint16_t* V = a.vc + (size_t)kvh * a.L_stride * HD + li * DPL;

  float q[G][DPL];
#pragma unroll
  for (int h = 0; h < G; h++)
#pragma unroll
    for (int e = 0; e < DPL; e++) q[h][e] = a.q[(size_t)(kvh * G + h) * HD + li * DPL + e];

  // phase 1: scores
  float mloc[G];
#pragma unroll
  for (int h = 0; h < G; h++) mloc[h] = -INFINITY;
  for (int p = p0 + pg; p < p1; p += 16) {
    float k[DPL];
    load_half_slice<HD>(K + (size_t)p * HD, k);
#pragma unroll
    for (int h = 0; h < G; h++) {
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < DPL; e++) s = fmaf(q[h][e], k[e], s);
      s = group_sum<16>(s) * scale;
      mloc[h] = fmaxf(mloc[h], s);
      if (li == 0) s_sc[h][p - p0] = s;
    }
  }
#pragma unroll
  for (int h = 0; h < G; h++) {
    const float m = wave_max(mloc[h]);
    if (lane == 0) s_red[wid][h] = m;
  }
  __syncthreads();
  float M[G];
#pragma unroll
  for (int h = 0; h < G; h++) {
    M[h] = s_red[0][h];
#pragma unroll
    for (int w = 1; w < ANW; w++) M[h] = fmaxf(M[h], s_red[w][h]);
  }

  // phase 2: p = exp(s - M), o = sum p v, l = sum p
  float o[G][DPL], l[G];
#pragma unroll
  for (int h = 0; h < G; h++) {
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < DPL; e++) o[h][e] = 0.f;
  }
  for (int p = p0 + pg; p < p1; p += 16) {
    float v[DPL];
    load_half_slice<HD>(V + (size_t)p * HD, v);
#pragma unroll
    for (int h = 0; h < G; h++) {
      const float w = expf(s_sc[h][p - p0] - M[h]);
      l[h] += w;
#pragma unroll
      for (int e = 0; e < DPL; e++) o[h][e] = fmaf(w, v[e], o[h][e]);
    }
  }
#pragma unroll
  for (int h = 0; h < G; h++) {
#pragma unroll
    for (int e = 0; e < DPL; e++) s_o[pg][h][li * DPL + e] = o[h][e];
    if (li == 0) s_l[pg][h] = l[h];
  }
  __syncthreads();

  float* part = a.part + ((size_t)kvh * nch + chunk) * G * PSTRIDE;
  for (int i = tid; i < G * HD; i += ANT) {
    const int h = i / HD, d = i % HD;
    float s = 0.f;
#pragma unroll
    for (int g = 0; g < 16; g++) s += s_o[g][h][d];
    part[h * PSTRIDE + d] = s;
  }
  if (tid < G) {
    float s = 0.f;
#pragma unroll
    for (int g = 0; g < 16; g++) s += s_l[g][tid];
    part[tid * PSTRIDE + HD] = M[tid];
    part[tid * PSTRIDE + HD + 1] = s;
  }

  // merge: the last chunk of this kv head to finish combines all chunks
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(&a.counters[kvh], 1u) == (unsigned)(nch - 1);
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  const float* pk = a.part + (size_t)kvh * nch * G * PSTRIDE;
  // chunk weights exp(m_c - Mmax) per head, reusing s_sc as scratch [G][nch]
  for (int h = wid; h < G; h += ANW) {
    float mm = -INFINITY;
    for (int c = lane; c < nch; c += WAVE) mm = fmaxf(mm, pk[((size_t)c * G + h) * PSTRIDE + HD]);
    mm = wave_max(mm);
    float ssum = 0.f;
    for (int c = lane; c < nch; c += WAVE) {
      const float* rec = pk + ((size_t)c * G + h) * PSTRIDE;
      const float w = expf(rec[HD] - mm);
      s_sc[h][c] = w;
      ssum = fmaf(w, rec[HD + 1], ssum);
    }
    ssum = wave_sum(ssum);
    if (lane == 0) s_red[0][h] = ssum;
  }
  __syncthreads();
  for (int i = tid; i < G * HD; i += ANT) {
    const int h = i / HD, d = i % HD;
    float s = 0.f;
    for (int c = 0; c < nch; c++) s = fmaf(s_sc[h][c], pk[((size_t)c * G + h) * PSTRIDE + d], s);
    a.o[(size_t)(kvh * G + h) * HD + d] = s / s_red[0][h];
  }
  if (tid == 0) a.counters[kvh] = 0u;
}

template <int HD>
int launch_hd(const AttnArgs& a, float scale, hipStream_t s) {
  const dim3 grid((unsigned)a.n_chunks, (unsigned)a.nkv);
  switch (a.nq / a.nkv) {
    case 1: hipLaunchKernelGGL((attn_decode_kernel<HD, 1>), grid, dim3(ANT), 0, s, a, scale); break;
    case 2: hipLaunchKernelGGL((attn_decode_kernel<HD, 2>), grid, dim3(ANT), 0, s, a, scale); break;
    case 4: hipLaunchKernelGGL((attn_decode_kernel<HD, 4>), grid, dim3(ANT), 0, s, a, scale); break;
    case 8: hipLaunchKernelGGL((attn_decode_kernel<HD, 8>), grid, dim3(ANT), 0, s, a, scale); break;
    default: return fail(TPT_ERR_UNSUPPORTED, "attention: Nq/Nkv must be 1, 2, 4 or 8");
  }
  TPT_HIP(hipGetLastError());
  return TPT_OK;
}

}  // namespace

int attn_part_floats(int nq, int nkv, int hd, int n_chunks) {
  return nkv * n_chunks * (nq / nkv) * (hd + 2);
}

int attn_default_chunks(int L, int nkv) {
  int n = (L + 63) / 64;
  const int cap = 1024 / (nkv > 0 ? nkv : 1);
  if (n > cap) n = cap;
  const int need = (L + CL_MAX - 1) / CL_MAX;
  if (n < need) n = need;
  return n < 1 ? 1 : n;
}

int launch_attn_decode(const AttnArgs& a, hipStream_t s) {
  if (a.nq <= 0 || a.nkv <= 0 || a.nq % a.nkv) return fail(TPT_ERR_INVALID, "attention: bad head counts");
  if (a.n_chunks <= 0 || a.n_chunks > 4096) return fail(TPT_ERR_INVALID, "attention: bad chunk count");
  if (!a.state && (a.L_host <= 0 || a.L_host > a.L_stride))
    return fail(TPT_ERR_INVALID, "attention: L must be in [1, L_stride]");
  if (!a.state && (a.L_host + a.n_chunks - 1) / a.n_chunks > CL_MAX)
    return fail(TPT_ERR_INVALID, "attention: too few chunks for this length");
  if (a.n_chunks > CL_MAX) return fail(TPT_ERR_INVALID, "attention: too many chunks");
  const float scale = (float)(1.0 / __builtin_sqrt((double)a.hd));
  switch (a.hd) {
    case 64: return launch_hd<64>(a, scale, s);
    case 96: return launch_hd<96>(a, scale, s);
    case 128: return launch_hd<128>(a, scale, s);
  }
  return fail(TPT_ERR_UNSUPPORTED, "attention: head_dim must be 64, 96 or 128");
}

}  // namespace tpt
