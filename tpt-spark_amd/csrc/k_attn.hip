// Split-K (flash-decoding) GQA attention for one query position over an fp16 or f32 KV cache.
//
// Replaces the three-pass attention.wgsl (src-tauri/src/engine/shaders/attention.wgsl:31-170,
// dispatch_attention wgpu_engine.rs:666-726: scores materialised in f32 for every head and
// position, then softmax, then P.V) and restates what candle's quantized_llama computes on the
// CPU for a decode step: repeat_kv (head h reads kv head h / (Nq/Nkv)),
// att = (q . k) * f32(1/sqrt(hd)), softmax_last_dim, att . v.
//
// Cache layout [Nkv][L_stride][hd], element type fp16 (the default) or f32 (candle keeps an f32
// cache): the K and V rows of a kv head are contiguous over positions, so a chunk of positions
// streams as one contiguous run.  Two kernels:
//  * attn_partial, grid (n_chunks, Nkv), 256 threads.  A workgroup reads each K and V row of its
//    chunk once and serves all G = Nq/Nkv query heads of the group.  LPP lanes (16 B each)
//    share a position and reduce with DPP; every thread keeps U rows in flight (loads are
//    unconditional, positions past the chunk re-read its last row), and the first round's V
//    rows are loaded together with its K rows (a chunk of up to R*U positions is one round
//    trip).
//    Scores go to LDS; after the chunk max, p = exp(s - max) is formed once per (head,
//    position) and summed; then o = sum p v.  The record (o unnormalised, max, sum) goes to
//    the partial buffer.  Chunks of up to 64 positions (the decode partition up to 4096
//    positions with 8 kv heads) take attn_partial1: the chunk's K and V rows, scores and
//    probabilities stay in registers, two workgroup barriers instead of four.  With one query
//    head per kv head the long chunks' rounds are software-pipelined (the next round's rows
//    requested before the current round's arithmetic).
//  * attn_merge, one workgroup per 32 output dims: combines the chunk records with the
//    log-sum-exp rule; its first chunk loads are issued before the chunk weights are known.  The kernel boundary orders the two, so
//    no device-wide fence or arrival counter is needed.
#include "attn_dev.h"

namespace tpt {
namespace {

using namespace attn;

constexpr int ANT = 256;
constexpr int ANW = ANT / WAVE;
constexpr int CL_MAX = 1024;   // positions per chunk held in LDS
constexpr int NCH_MAX = 256;   // chunks per kv head
constexpr int MT = 32;         // output dims per merge workgroup
constexpr int MSETS = ANT / MT;

template <typename T, int HD, int G, int U, bool PIPE>
__global__ void __launch_bounds__(ANT) attn_partial_kernel(const AttnArgs a, const float scale) {
  constexpr int LPP = KvTraits<T>::LPP;   // lanes per position
  constexpr int EPL = HD / LPP;           // elements per lane
  constexpr int R = ANT / LPP;            // positions per round
  // U: rounds whose loads are in flight together (R*U >= the chunk length when it is short)
  constexpr int PSTRIDE = HD + 2;         // partial record: o[HD], m, l
  __shared__ float s_p[G][CL_MAX];        // scores, then p = exp(s - max)
  __shared__ float s_red[ANW][G];
  __shared__ float s_o[R][G][HD];
  __shared__ float s_l[G];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int li = tid % LPP, pg = tid / LPP;  // lane in position, position group 0..R-1
  const int kvh = blockIdx.y, chunk = blockIdx.x, nch = gridDim.x, t = blockIdx.z;
  // The chunk's rows are known at launch; the live length L (from the step state on the
  // decode path) only masks: q and the first round's K and V rows are requested before L is
  // read, so no load waits for it (a chunk past L discards what it fetched).
  const int CL = a.chunk_len;
  const int p0 = chunk * CL;
  const int plast = min(p0 + CL, a.L_stride) - 1;  // clamped loads stay inside the cache

  const T* K = (const T*)a.kc + (size_t)kvh * a.L_stride * HD + li * EPL;
  const T* V = (const T*)a.vc + (size_t)kvh * a.L_stride * HD + li * EPL;

  float q[G][EPL];
#pragma unroll
  for (int h = 0; h < G; h++)
#pragma unroll
    for (int e = 0; e < EPL; e++) q[h][e] = a.q[(size_t)t * a.ldq + (size_t)(kvh * G + h) * HD + li * EPL + e];
  float k0[U][EPL], vpre[U][EPL];
#pragma unroll
  for (int u = 0; u < U; u++) load_row<EPL>(K + (size_t)min(p0 + u * R + pg, plast) * HD, k0[u]);
#pragma unroll
  for (int u = 0; u < U; u++) load_row<EPL>(V + (size_t)min(p0 + u * R + pg, plast) * HD, vpre[u]);

  const int L = (a.state ? a.state->pos + 1 : a.L_host) + t;
  const int p1 = min(L, p0 + CL);
  const int n = p1 - p0;
  if (n <= 0) return;  // a chunk past the live length: the merge does not read its record

  // Rounds of R*U positions.  PIPE: software-pipelined, the next round's rows requested before
  // the current round's arithmetic (two register buffers, the first holding the preloaded
  // round), so a long chunk pays its load latency about once per phase rather than once per
  // round; otherwise each later round loads, then computes.  Same arithmetic in the same order.
  auto load_rows = [&](const T* base_ptr, float (&buf)[U][EPL], int base) {
#pragma unroll
    for (int u = 0; u < U; u++) load_row<EPL>(base_ptr + (size_t)min(base + u * R + pg, plast) * HD, buf[u]);
  };

  // phase 1: scores
  float mloc[G];
#pragma unroll
  for (int h = 0; h < G; h++) mloc[h] = -INFINITY;
  auto score_round = [&](const float (&k)[U][EPL], int base) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int p = base + u * R + pg;
#pragma unroll
      for (int h = 0; h < G; h++) {
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; e++) s = fmaf(q[h][e], k[u][e], s);
        s = lane_group_sum<LPP>(s) * scale;
        if (p < p1) {
          mloc[h] = fmaxf(mloc[h], s);
          if (li == 0) s_p[h][p - p0] = s;
        }
      }
    }
  };
  if constexpr (PIPE) {
    float k1[U][EPL];
    for (int base = p0; base < p1; base += 2 * R * U) {
      if (base + R * U < p1) load_rows(K, k1, base + R * U);
      score_round(k0, base);
      if (base + R * U >= p1) break;
      if (base + 2 * R * U < p1) load_rows(K, k0, base + 2 * R * U);
      score_round(k1, base + R * U);
    }
  } else {
    for (int base = p0; base < p1; base += R * U) {
      float k[U][EPL];
      if (base == p0) {
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
          for (int e = 0; e < EPL; e++) k[u][e] = k0[u][e];
      } else {
        load_rows(K, k, base);
      }
      score_round(k, base);
    }
  }
#pragma unroll
  for (int h = 0; h < G; h++) {
    const float m = wave_max_dpp(mloc[h]);
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
  __syncthreads();  // s_red is reused below

  // p = exp(s - M) once per (head, position); l = sum p
#pragma unroll
  for (int h = 0; h < G; h++) {
    float ls = 0.f;
    for (int j = tid; j < n; j += ANT) {
      const float w = expf(s_p[h][j] - M[h]);
      s_p[h][j] = w;
      ls += w;
    }
    ls = wave_sum_dpp(ls);
    if (lane == 0) s_red[wid][h] = ls;
  }
  __syncthreads();
  if (tid < G) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < ANW; w++) t += s_red[w][tid];
    s_l[tid] = t;
  }

  // phase 2: o = sum p v
  float o[G][EPL];
#pragma unroll
  for (int h = 0; h < G; h++)
#pragma unroll
    for (int e = 0; e < EPL; e++) o[h][e] = 0.f;
  auto pv_round = [&](const float (&vv)[U][EPL], int base) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int p = base + u * R + pg;
      if (p < p1) {
#pragma unroll
        for (int h = 0; h < G; h++) {
          const float w = s_p[h][p - p0];
#pragma unroll
          for (int e = 0; e < EPL; e++) o[h][e] = fmaf(w, vv[u][e], o[h][e]);
        }
      }
    }
  };
  if constexpr (PIPE) {
    float v1[U][EPL];
    for (int base = p0; base < p1; base += 2 * R * U) {
      if (base + R * U < p1) load_rows(V, v1, base + R * U);
      pv_round(vpre, base);
      if (base + R * U >= p1) break;
      if (base + 2 * R * U < p1) load_rows(V, vpre, base + 2 * R * U);
      pv_round(v1, base + R * U);
    }
  } else {
    for (int base = p0; base < p1; base += R * U) {
      float vv[U][EPL];
      if (base == p0) {
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
          for (int e = 0; e < EPL; e++) vv[u][e] = vpre[u][e];
      } else {
        load_rows(V, vv, base);
      }
      pv_round(vv, base);
    }
  }
#pragma unroll
  for (int h = 0; h < G; h++)
#pragma unroll
    for (int e = 0; e < EPL; e++) s_o[pg][h][li * EPL + e] = o[h][e];
  __syncthreads();

  float* part = a.part + (((size_t)t * gridDim.y + kvh) * nch + chunk) * G * PSTRIDE;
  for (int i = tid; i < G * HD; i += ANT) {
    const int h = i / HD, d = i % HD;
    float s = 0.f;
#pragma unroll
    for (int g = 0; g < R; g++) s += s_o[g][h][d];
    part[h * PSTRIDE + d] = s;
  }
  if (tid < G) {
    part[tid * PSTRIDE + HD] = M[tid];  // -inf for an empty chunk (its l is 0)
    part[tid * PSTRIDE + HD + 1] = s_l[tid];
  }
}

// The same record in one pass when the chunk fits the registers (chunk_len <= R*U): every thread
// keeps the scores of its U positions, forms p = exp(s - max) for them once the chunk max is
// known and accumulates p and p*v at once.  Two workgroup barriers (the max, then the record's
// sums over position groups) instead of four, and no score round trip through LDS.
template <typename T, int HD, int G, int U>
__global__ void __launch_bounds__(ANT) attn_partial1_kernel(const AttnArgs a, const float scale) {
  constexpr int LPP = KvTraits<T>::LPP;
  constexpr int EPL = HD / LPP;
  constexpr int R = ANT / LPP;
  constexpr int PSTRIDE = HD + 2;
  __shared__ float s_red[ANW][G];
  __shared__ float s_l[ANW][G];
  __shared__ float s_o[R][G][HD];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int li = tid % LPP, pg = tid / LPP;
  const int kvh = blockIdx.y, chunk = blockIdx.x, nch = gridDim.x, t = blockIdx.z;
  const int CL = a.chunk_len;
  const int p0 = chunk * CL;
  const int plast = min(p0 + CL, a.L_stride) - 1;
  const T* K = (const T*)a.kc + (size_t)kvh * a.L_stride * HD + li * EPL;
  const T* V = (const T*)a.vc + (size_t)kvh * a.L_stride * HD + li * EPL;

  float q[G][EPL];
#pragma unroll
  for (int h = 0; h < G; h++)
#pragma unroll
    for (int e = 0; e < EPL; e++) q[h][e] = a.q[(size_t)t * a.ldq + (size_t)(kvh * G + h) * HD + li * EPL + e];
  float kk[U][EPL], vv[U][EPL];
#pragma unroll
  for (int u = 0; u < U; u++) load_row<EPL>(K + (size_t)min(p0 + u * R + pg, plast) * HD, kk[u]);
#pragma unroll
  for (int u = 0; u < U; u++) load_row<EPL>(V + (size_t)min(p0 + u * R + pg, plast) * HD, vv[u]);

  const int L = (a.state ? a.state->pos + 1 : a.L_host) + t;
  const int p1 = min(L, p0 + CL);
  if (p1 <= p0) return;  // a chunk past the live length: the merge does not read its record

  float sc[U][G], mloc[G];
#pragma unroll
  for (int h = 0; h < G; h++) mloc[h] = -INFINITY;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const bool live = p0 + u * R + pg < p1;
#pragma unroll
    for (int h = 0; h < G; h++) {
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; e++) d = fmaf(q[h][e], kk[u][e], d);
      sc[u][h] = lane_group_sum<LPP>(d) * scale;
      if (live) mloc[h] = fmaxf(mloc[h], sc[u][h]);
    }
  }
#pragma unroll
  for (int h = 0; h < G; h++) {
    const float m = wave_max_dpp(mloc[h]);
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

  float o[G][EPL], ls[G];
#pragma unroll
  for (int h = 0; h < G; h++) {
    ls[h] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; e++) o[h][e] = 0.f;
  }
#pragma unroll
  for (int u = 0; u < U; u++) {
    if (p0 + u * R + pg < p1) {
#pragma unroll
      for (int h = 0; h < G; h++) {
        const float w = expf(sc[u][h] - M[h]);
        ls[h] += w;
#pragma unroll
        for (int e = 0; e < EPL; e++) o[h][e] = fmaf(w, vv[u][e], o[h][e]);
      }
    }
  }
  // the LPP lanes of a position group hold the same sums: count each group once
#pragma unroll
  for (int h = 0; h < G; h++) {
    const float l = wave_sum_dpp(li == 0 ? ls[h] : 0.f);
    if (lane == 0) s_l[wid][h] = l;
  }
#pragma unroll
  for (int h = 0; h < G; h++)
#pragma unroll
    for (int e = 0; e < EPL; e++) s_o[pg][h][li * EPL + e] = o[h][e];
  __syncthreads();

  float* part = a.part + (((size_t)t * gridDim.y + kvh) * nch + chunk) * G * PSTRIDE;
  for (int i = tid; i < G * HD; i += ANT) {
    const int h = i / HD, d = i % HD;
    float s = 0.f;
#pragma unroll
    for (int g = 0; g < R; g++) s += s_o[g][h][d];
    part[h * PSTRIDE + d] = s;
  }
  if (tid < G) {
    float l = 0.f;
#pragma unroll
    for (int w = 0; w < ANW; w++) l += s_l[w][tid];
    part[tid * PSTRIDE + HD] = M[tid];
    part[tid * PSTRIDE + HD + 1] = l;
  }
}

// o[h][d] = sum_c w_c o_c[h][d] / sum_c w_c l_c with w_c = exp(m_c - max_c m_c).  Workgroup:
// 32 consecutive output dims of one head; thread (set, j) sums chunks set, set + 8, ...
template <int HD, int G>
__global__ void __launch_bounds__(ANT) attn_merge_kernel(const float* __restrict__ part,
                                                         float* __restrict__ out, int nch, int ldo,
                                                         const StepState* state, int L_host, int CL) {
  constexpr int PSTRIDE = HD + 2;
  constexpr int TILES = G * HD / MT;  // merge workgroups per kv head
  __shared__ float s_w[NCH_MAX];
  __shared__ float s_acc[MSETS][MT];
  __shared__ float s_l;
  const int tid = threadIdx.x, lane = tid & 63;
  const int kvh = blockIdx.x / TILES, d0 = (blockIdx.x % TILES) * MT, t = blockIdx.y;
  const int nkv = gridDim.x / TILES;
  const int h = d0 / HD, dh = d0 % HD;
  out += (size_t)t * ldo;
  const float* pk = part + ((size_t)t * nkv + kvh) * nch * G * PSTRIDE + (size_t)h * PSTRIDE;
  const int j = tid % MT, set = tid / MT;
  const float* src = pk + dh + j;
  // first 8 chunks of this thread's set, issued before the weights (clamped: always in bounds)
  float v0[8];
#pragma unroll
  for (int i = 0; i < 8; i++) v0[i] = src[(size_t)min(set + i * MSETS, nch - 1) * G * PSTRIDE];
  // chunks that hold positions of this query (the others wrote no record)
  const int L = (state ? state->pos + 1 : L_host) + t;
  nch = min(nch, (L + CL - 1) / CL);
  if (tid < WAVE) {
    // each chunk's max and sum in one round trip (at most NCH_MAX / WAVE chunks per lane)
    constexpr int CPL = NCH_MAX / WAVE;
    float mv[CPL], lv[CPL];
#pragma unroll
    for (int i = 0; i < CPL; i++) {
      const int c = lane + i * WAVE;
      const float* rec = pk + (size_t)min(c, nch - 1) * G * PSTRIDE;
      mv[i] = rec[HD];
      lv[i] = rec[HD + 1];
    }
    float mm = -INFINITY;
#pragma unroll
    for (int i = 0; i < CPL; i++)
      if (lane + i * WAVE < nch) mm = fmaxf(mm, mv[i]);
    mm = wave_max_dpp(mm);
    float ls = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; i++) {
      const int c = lane + i * WAVE;
      if (c < nch) {
        const float w = expf(mv[i] - mm);
        s_w[c] = w;
        ls = fmaf(w, lv[i], ls);
      }
    }
    ls = wave_sum_dpp(ls);
    if (lane == 0) s_l = ls;
  }
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int c = set + i * MSETS;
    if (c < nch) s = fmaf(s_w[c], v0[i], s);
  }
  int c = set + 8 * MSETS;
  for (; c + 7 * MSETS < nch; c += 8 * MSETS) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = src[(size_t)(c + i * MSETS) * G * PSTRIDE];
#pragma unroll
    for (int i = 0; i < 8; i++) s = fmaf(s_w[c + i * MSETS], v[i], s);
  }
  for (; c < nch; c += MSETS) s = fmaf(s_w[c], src[(size_t)c * G * PSTRIDE], s);
  s_acc[set][j] = s;
  __syncthreads();
  if (tid < MT) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < MSETS; i++) t += s_acc[i][tid];
    out[(size_t)(kvh * G + h) * HD + dh + tid] = t / s_l;
  }
}

template <typename T, int HD, int G>
int launch_g(const AttnArgs& a, float scale, hipStream_t s) {
  const dim3 grid((unsigned)a.n_chunks, (unsigned)a.nkv, (unsigned)a.nqb);
  constexpr int R = ANT / KvTraits<T>::LPP;
  constexpr int U1 = 64 / R;  // one-pass form: chunks of up to 64 positions
  static_assert(U1 * R >= 4 * R, "chunks of up to four rounds take the one-pass form");
  if (a.chunk_len <= U1 * R)
    hipLaunchKernelGGL((attn_partial1_kernel<T, HD, G, U1>), grid, dim3(ANT), 0, s, a, scale);
  else if constexpr (G == 1) {
    // one query head per kv head (MHA): few registers per round, so the pipelined form pays;
    // grids of more than two workgroups per CU take rounds of 4R (hd 96, 32 heads: 32768
    // positions 84 -> 71 us with 4R, 16384 positions 41.6 -> 39.4 us with 8R)
    if ((long)a.n_chunks * a.nkv * a.nqb > 512)
      hipLaunchKernelGGL((attn_partial_kernel<T, HD, G, 4, true>), grid, dim3(ANT), 0, s, a, scale);
    else
      hipLaunchKernelGGL((attn_partial_kernel<T, HD, G, 8, true>), grid, dim3(ANT), 0, s, a, scale);
  } else
    hipLaunchKernelGGL((attn_partial_kernel<T, HD, G, 8, false>), grid, dim3(ANT), 0, s, a, scale);
  TPT_HIP(hipGetLastError());
  hipLaunchKernelGGL((attn_merge_kernel<HD, G>), dim3((unsigned)(a.nkv * G * HD / MT), (unsigned)a.nqb),
                     dim3(ANT), 0, s, (const float*)a.part, a.o, a.n_chunks, a.ldo, a.state, a.L_host,
                     a.chunk_len);
  TPT_HIP(hipGetLastError());
  return TPT_OK;
}

template <typename T, int HD>
int launch_hd(const AttnArgs& a, float scale, hipStream_t s) {
  switch (a.nq / a.nkv) {
    case 1: return launch_g<T, HD, 1>(a, scale, s);
    case 2: return launch_g<T, HD, 2>(a, scale, s);
    case 4: return launch_g<T, HD, 4>(a, scale, s);
    case 8: return launch_g<T, HD, 8>(a, scale, s);
  }
  return fail(TPT_ERR_UNSUPPORTED, "attention: Nq/Nkv must be 1, 2, 4 or 8");
}

template <typename T>
int launch_t(const AttnArgs& a, float scale, hipStream_t s) {
  switch (a.hd) {
    case 64: return launch_hd<T, 64>(a, scale, s);
    case 96: return launch_hd<T, 96>(a, scale, s);
    case 128: return launch_hd<T, 128>(a, scale, s);
  }
  return fail(TPT_ERR_UNSUPPORTED, "attention: head_dim must be 64, 96 or 128");
}

}  // namespace

int attn_part_floats(int nq, int nkv, int hd, int n_chunks) {
  return nkv * n_chunks * (nq / nkv) * (hd + 2);
}

// Chunks per kv head: about 64 positions per workgroup while the grid is small, at most 512
// workgroups in total, and never more than CL_MAX positions per chunk.
int attn_default_chunks(int L, int nkv) {
  int n = (L + 63) / 64;
  int cap = 512 / (nkv > 0 ? nkv : 1);
  if (cap < 1) cap = 1;
  if (n > cap) n = cap;
  const int need = (L + CL_MAX - 1) / CL_MAX;
  if (n < need) n = need;
  if (n > NCH_MAX) n = NCH_MAX;
  return n < 1 ? 1 : n;
}

int attn_max_len() { return CL_MAX * NCH_MAX; }

int attn_chunk_len(int L, int n_chunks) {
  int cl = (L + n_chunks - 1) / n_chunks;
  return (cl + 15) & ~15;
}

int launch_attn_decode(const AttnArgs& a, hipStream_t s) {
  if (a.nq <= 0 || a.nkv <= 0 || a.nq % a.nkv) return fail(TPT_ERR_INVALID, "attention: bad head counts");
  if (a.n_chunks <= 0 || a.n_chunks > NCH_MAX) return fail(TPT_ERR_INVALID, "attention: chunk count must be in [1, 256]");
  if (!a.state && (a.L_host <= 0 || a.L_host > a.L_stride))
    return fail(TPT_ERR_INVALID, "attention: L must be in [1, L_stride]");
  if (a.chunk_len <= 0 || a.chunk_len % 16 || a.chunk_len > CL_MAX)
    return fail(TPT_ERR_INVALID, "attention: chunk length must be a multiple of 16 in [16, 1024]");
  if (!a.state && (long)a.chunk_len * a.n_chunks < a.L_host)
    return fail(TPT_ERR_INVALID, "attention: chunks do not cover the length");
  if (a.nqb < 1 || (a.nqb > 1 && (a.state || a.ldq < a.nq * a.hd || a.ldo < a.nq * a.hd)))
    return fail(TPT_ERR_INVALID, "attention: bad query batch");
  if (!a.state && a.L_host + a.nqb - 1 > a.L_stride)
    return fail(TPT_ERR_INVALID, "attention: queries past the cache");
  if (!a.state && (long)a.chunk_len * a.n_chunks < a.L_host + a.nqb - 1)
    return fail(TPT_ERR_INVALID, "attention: chunks do not cover the last query");
  if (a.kv_type != TPT_TYPE_F16 && a.kv_type != TPT_TYPE_F32)
    return fail(TPT_ERR_UNSUPPORTED, "attention: KV cache type must be F16 or F32");
  const float scale = (float)(1.0 / __builtin_sqrt((double)a.hd));
  return a.kv_type == TPT_TYPE_F32 ? launch_t<float>(a, scale, s) : launch_t<uint16_t>(a, scale, s);
}

}  // namespace tpt
