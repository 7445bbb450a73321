// Persistent decode step for bs=1 Llama decode on gfx950: the token embedding and every decoder
// layer of one decode step in ONE launch of one 512-thread workgroup per compute unit.
//
// It computes what the multi-kernel decode step computes (run_forward_pass,
// src-tauri/src/engine/wgpu_engine.rs:339-490, with the residual adds candle's quantized_llama
// has): per layer
//   QKV    RMSNorm -> Q|K|V GEMV -> RoPE on q and k -> q buffer, k and v appended to the cache
//   ATT    split-K GQA attention over the cache: per (kv head, chunk) a partial record; the last
//          chunk of a kv head to finish merges the records (log-sum-exp) into the output
//   WO     x += Wo . attention
//   GU     h = silu(W1 . RMSNorm(x)) * (W3 . RMSNorm(x))
//   DN     x += W2 . h
// with the same per-row arithmetic as the standalone kernels (the GEMV rows are bit-identical
// to k_gemv.hip's: same lane groups, same Q8_K activation quantization, same reductions).
//
// Why one launch: at bs=1 every phase is a short HBM stream (8B shape: 14 MB QKV, 9 MB Wo, 66 MB
// gate|up, 33 MB down per layer), and separate kernels each pay their launch ramp, prologue and
// drain (measured 58 us per layer as six kernels against 22 us of streaming at 6 TB/s).  Here
// the phases of the whole step are separated by grid barriers instead, and every workgroup
// issues its first weight loads of the next phase BEFORE it waits at the barrier (weights do not
// depend on the activations), so HBM keeps streaming through the barrier.
//
// Grid barrier: every workgroup owns one flag in its own 128-byte line; arriving writes the
// epoch to it, waiting polls all flags with one thread per flag (measured 1.6 us per barrier on
// 256 CUs, against 3.9 us for a single contended counter).  Every wait is bounded: a wait that
// exceeds kSpinLimit polls sets the error word and releases the workgroup (and, through its
// poisoned flag, everybody waiting on it), so a launch always drains; the host reports the error.
//
// Memory coherence: the eight XCDs' L2 caches are not coherent with each other, so data that one
// workgroup writes and another reads in the same launch (residual x, q, this position's K/V
// rows, attention records and output, the FFN hidden vector) is written with agent-scope stores
// (global_store sc1) and read with agent-scope loads (buffer_load sc1), after the writer's
// s_waitcnt vmcnt(0) and before its barrier arrival.  Weights, norms, RoPE tables and cache rows
// of earlier positions were written before the launch and are read normally.
#include <algorithm>
#include <atomic>

#include "kernels.h"

#include "attn_dev.h"
#include "gemv_dev.h"

namespace tpt {
namespace {

using namespace gemv;

// ------------------------------------------------------------------ address spaces and state
// Each phase is its own non-inlined function, register-allocated on its own (inlined into one
// layer loop, the compiler hoists every phase's loop-invariant lane arithmetic out of the loop and
// runs out of registers).  Inside them, global memory is reached only through pointers typed
// address_space(1) (global_load / global_store) or buffer descriptors: a generic pointer would
// compile to flat instructions, which also count against the LDS counter, so every LDS wait would
// wait for the weight loads in flight.  The launch arguments are copied to LDS at kernel start and
// read from there (LDS reads never wait for global loads either).
#define GLB __attribute__((address_space(1)))
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

template <class T>
__device__ __forceinline__ const GLB T* cg(const T* p) { return (const GLB T*)p; }
template <class T>
__device__ __forceinline__ GLB T* gp(T* p) { return (GLB T*)p; }

struct Ctl {
  int dead;        // a barrier wait of this workgroup timed out
  int pos;
  uint32_t tok;
  unsigned base;   // barrier epoch before this launch's first arrival
};
__shared__ __align__(16) unsigned char s_args[sizeof(DecodeArgs)];  // DecodeArgs, copied at start
__shared__ Ctl s_c;
#define s_a (*(DecodeArgs*)s_args)
extern __shared__ __align__(16) char smem[];

// ------------------------------------------------------------------ agent-scope accesses
constexpr int kSC1 = 16;  // raw-buffer cache-policy bit that sets sc1 on gfx950
typedef __amdgpu_buffer_rsrc_t Rsrc;

// The descriptor must sit in scalar registers; pointers read from LDS are not provably uniform,
// so they are made so (readfirstlane) -- else every buffer access becomes a waterfall loop.
__device__ __forceinline__ Rsrc rsrc(const void* p, size_t bytes) {
  const uint64_t u = (uint64_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  const int n = __builtin_amdgcn_readfirstlane(bytes > 0x7fffffffull ? 0x7fffffff : (int)bytes);
  return __builtin_amdgcn_make_buffer_rsrc((void*)(((uint64_t)hi << 32) | lo), (short)0, n, 0x00020000);
}
__device__ __forceinline__ float ldb(Rsrc r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kSC1));
}
// (element VALUES are converted: clang lowers __builtin_bit_cast of an ext-vector element
// lvalue v[i] as a load from the vector's base address, i.e. always element 0)
__device__ __forceinline__ float4 u4f(u32x4 v) {
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}
__device__ __forceinline__ float4 ldb4(Rsrc r, uint32_t off) {
  return u4f(__builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kSC1));
}
__device__ __forceinline__ unsigned ld_flag(const GLB unsigned* p) {
  return __hip_atomic_load(const_cast<GLB unsigned*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_u(GLB unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_f(GLB float* p, float v) {
  st_u((GLB unsigned*)p, __builtin_bit_cast(unsigned, v));
}
__device__ __forceinline__ void wait_mem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ __forceinline__ float4 ldg4(const GLB float* p) {  // plain load (read-only data)
  return u4f(*(const GLB u32x4*)p);
}

// One K or V row slice of EPL elements (KT = fp16 bits or f32) through an agent-scope load.
template <typename KT, int EPL>
__device__ __forceinline__ void ld_row(Rsrc r, uint32_t off, float* out) {
  constexpr int B = EPL * (int)sizeof(KT);
  uint32_t w[4];
  if constexpr (B == 16) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kSC1);
    w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
  } else if constexpr (B == 12) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b96(r, off, 0, kSC1);
    w[0] = v[0]; w[1] = v[1]; w[2] = v[2];
  } else {
    static_assert(B == 8, "row slices of 8, 12 or 16 bytes");
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kSC1);
    w[0] = v[0]; w[1] = v[1];
  }
  if constexpr (sizeof(KT) == 2) {
#pragma unroll
    for (int i = 0; i < B / 4; i++) {
      out[2 * i] = h2f((uint16_t)(w[i] & 0xffff));
      out[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
    }
  } else {
#pragma unroll
    for (int i = 0; i < B / 4; i++) out[i] = __uint_as_float(w[i]);
  }
}

// ------------------------------------------------------------------ grid barrier
constexpr unsigned kSpinLimit = 1u << 20;  // polls (~0.5 us each) before a wait gives up
constexpr int kFlagStride = 32;            // words: one flag per 128-byte line

// Called by every thread after its last store of the phase; returns the arrival count.
__device__ __forceinline__ unsigned grid_arrive(unsigned e) {
  wait_mem();      // this thread's stores are performed at agent scope
  barrier_lds();   // ... and so are every other thread's
  e++;
  if (threadIdx.x == 0)
    st_u(gp(s_a.flags) + blockIdx.x * kFlagStride, s_c.dead ? 0xffffffffu : s_c.base + e);
  return e;
}

// Waits until every workgroup has made e arrivals (one poll thread per workgroup flag).
__device__ __forceinline__ void grid_wait(unsigned e) {
  const unsigned target = s_c.base + e;
  if (!s_c.dead && threadIdx.x < gridDim.x) {
    const GLB unsigned* f = gp(s_a.flags) + threadIdx.x * kFlagStride;
    const GLB unsigned* err = gp(s_a.err);
    unsigned spins = 0;
    while (ld_flag(f) < target) {
      if (++spins >= kSpinLimit) {
        __hip_atomic_fetch_or(gp(s_a.err), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_c.dead = 1;
        break;
      }
      if ((spins & 255) == 0 && ld_flag(err)) {
        s_c.dead = 1;
        break;
      }
    }
  }
  barrier_lds();
  // a workgroup that gave up poisons its flag: nobody waits on it again
  if (s_c.dead && threadIdx.x == 0) st_u(gp(s_a.flags) + blockIdx.x * kFlagStride, 0xffffffffu);
}

// ------------------------------------------------------------------ GEMV phase
// One workgroup's rows of a Q4_K GEMV (KS = 1: a wave owns whole rows), split so that the first
// D steps' weight loads can be issued before the grid barrier that releases the activation.
// Same lane groups, step order and reductions as gemv_run (gemv_dev.h).
__device__ __forceinline__ void load_q4k(const GLB uint8_t* row, int g, Raw<TPT_TYPE_Q4_K>& r) {
  const GLB uint8_t* blk = row + (size_t)(g >> 2) * 144;  // 144 = 9 x 16: blocks stay 16-aligned
  const int off = 16 + (g & 3) * 32;
  const u32x4 h = *(const GLB u32x4*)blk;
  const u32x4 a = *(const GLB u32x4*)(blk + off);
  const u32x4 b = *(const GLB u32x4*)(blk + off + 16);
  r.h = make_uint4(h[0], h[1], h[2], h[3]);
  r.a = make_uint4(a[0], a[1], a[2], a[3]);
  r.b = make_uint4(b[0], b[1], b[2], b[3]);
}

template <int BPP, int RB, int NMAT, int D>
struct Phase {
  static constexpr int WT = TPT_TYPE_Q4_K;  // D: steps in flight per wave
  static constexpr int RPP = 16 / BPP;    // rows per pass
  static constexpr int LPR = 4 * BPP;     // lanes per row
  static constexpr int RG = RB * RPP;     // rows per row group
  Raw<WT> ring[D][RB][NMAT];
  const GLB uint8_t* w0;
  const GLB uint8_t* w1;
  size_t stride;
  int N, r0, rpw, nb, P, S, rp, sb, q, wid;

  __device__ __forceinline__ void init(const GLB uint8_t* a0, const GLB uint8_t* a1, size_t row_stride,
                                       int K, int n, int rows_per_wg) {
    const int lane = threadIdx.x & 63;
    w0 = a0;
    w1 = a1;
    stride = row_stride;
    N = n;
    rpw = rows_per_wg;
    r0 = blockIdx.x * rows_per_wg;
    nb = K / QK_K;
    P = (nb + BPP - 1) / BPP;
    rp = lane / LPR;
    sb = (lane / 4) % BPP;
    q = lane & 3;
    wid = threadIdx.x >> 6;
    const int ngrp = rpw / RG;
    const int ng = ngrp > wid ? (ngrp - wid + NW - 1) / NW : 0;
    S = r0 < N ? ng * P : 0;
  }
  __device__ __forceinline__ int group_of(int p, bool* valid) const {
    const int blk = p * BPP + sb;
    *valid = blk < nb;
    return 4 * (blk < nb ? blk : nb - 1) + q;
  }
  __device__ __forceinline__ void issue(Raw<WT> (&buf)[RB][NMAT], int s) const {
    if (s >= S) s = S > 0 ? S - 1 : 0;  // past the end: re-read the last step (cache hits)
    const int grp = wid + (s / P) * NW, p = s % P;
    bool v;
    const int g = group_of(p, &v);
#pragma unroll
    for (int j = 0; j < RB; j++) {
      int row = r0 + (grp * RB + j) * RPP + rp;
      if (row >= N) row = N - 1;
#pragma unroll
      for (int m = 0; m < NMAT; m++) load_q4k((m == 0 ? w0 : w1) + (size_t)row * stride, g, buf[j][m]);
    }
  }
  __device__ __forceinline__ void issue_first() {
#pragma unroll
    for (int d = 0; d < D; d++) issue(ring[d], d);
  }
  // Activation values (xl(i) = float4 i of x) -> optional RMSNorm -> Q8_K into LDS, in the
  // preload layout of the standalone kernel (one 256-block per 16-lane DPP row).
  template <bool NORM, class XL>
  __device__ __forceinline__ void prologue(const GemvArgs& A, const GLB float* norm_w, const Lds& L,
                                           const XL& xl) const {
    const int lane = threadIdx.x & 63;
    const int k = lane >> 4, m = lane & 15;
    const int nbk = A.K / 256;
    XPre p;
#pragma unroll
    for (int qi = 0; qi < MAXQ; qi++) {
      int b = 4 * (wid + qi * NW) + k;
      if (b >= nbk) b = nbk - 1;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        p.x[qi * 4 + j] = xl(b * 64 + m * 4 + j);
        if constexpr (NORM) p.w[qi * 4 + j] = ldg4(norm_w + 4 * (b * 64 + m * 4 + j));
        else p.w[qi * 4 + j] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    prologue_q8k(A, p, L);
    barrier_lds();
  }
  // All steps; row totals to L.rows[row * NMAT + m]; ends with a workgroup barrier.
  __device__ __forceinline__ void run(const Lds& L) {
    const int lane = threadIdx.x & 63;
    float acc[RB][NMAT];
#pragma unroll
    for (int j = 0; j < RB; j++)
#pragma unroll
      for (int m = 0; m < NMAT; m++) acc[j][m] = 0.f;
    auto compute = [&](const Raw<WT> (&buf)[RB][NMAT], int s) {
      const int grp = wid + (s / P) * NW, p = s % P;
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
      if (p == P - 1) {
#pragma unroll
        for (int j = 0; j < RB; j++)
#pragma unroll
          for (int m = 0; m < NMAT; m++) {
            const float t = lane_group_sum<LPR>(acc[j][m]);
            if (lane % LPR == 0) L.rows[((grp * RB + j) * RPP + rp) * NMAT + m] = t;
            acc[j][m] = 0.f;
          }
      }
    };
    for (int s = 0; s < S; s += D) {
#pragma unroll
      for (int d = 0; d < D; d++) {
        if (s + d < S) compute(ring[d], s + d);
        issue(ring[d], s + d + D);
      }
    }
    barrier_lds();
  }
  __device__ __forceinline__ int nrows() const { return r0 < N ? min(rpw, N - r0) : 0; }
};

struct LdsX {  // activation float4s from an LDS copy
  const float4* p;
  __device__ float4 operator()(int i) const { return p[i]; }
};
struct AgentX {  // activation float4s written in this launch by other workgroups
  Rsrc r;
  __device__ float4 operator()(int i) const { return ldb4(r, 16u * (uint32_t)i); }
};

__host__ __device__ inline size_t gemv_lds_bytes(int K, int rows) {
  return (lds_act_bytes(K, ACT_Q8K) + 4 * (size_t)rows + 15) & ~(size_t)15;
}

__device__ __forceinline__ const GLB DecLayer* layer_of(int l) { return cg(s_a.layers) + l; }

// ------------------------------------------------------------------ attention (per item)
// Item = (kv head, chunk of positions); two items per workgroup, one per 256-thread half, both
// halves running the same barrier sequence.  Per item the arithmetic of attn_partial_kernel
// (k_attn.hip), in its order: scores (q.k) * 1/sqrt(hd) for the G query heads of the kv head,
// chunk max, p = exp(s - max) once per (head, position), l = sum p, o = sum p v summed over the
// position groups in order; the record (o, max, l).
// LDS floats of one attention half: scores [G][CL] | wave maxima/sums [4][G] | per position
// group o [R][G][HD] (R = positions per round) | l [G]
__host__ __device__ inline int att_half_floats(int G, int HD, int R, int CL) {
  const int n = G * CL + 4 * G + R * G * HD + G;
  return (n + 3) & ~3;
}

template <typename KT, int HD, int G>
struct Att {
  static constexpr int LPP = attn::KvTraits<KT>::LPP;  // lanes per position (16 B each)
  static constexpr int EPL = HD / LPP;
  static constexpr int HT = 256;
  static constexpr int R = HT / LPP;   // positions per round
  static constexpr int U = 4;          // rounds in flight
  static constexpr int PS = HD + 2;    // record stride

  // this half's LDS (derived here from the LDS array itself: a pointer passed between functions
  // would be generic and its accesses flat instructions)
  __device__ __forceinline__ static float* half_lds(int half) {
    return (float*)smem + (size_t)half * att_half_floats(G, HD, R, s_a.chunk_len);
  }
  // q[0..EPL) of this lane for one head (agent-scope loads, 16 bytes where the slice allows)
  __device__ __forceinline__ static void load_q(Rsrc rq, uint32_t off, float* q) {
    if constexpr (EPL % 4 == 0) {
#pragma unroll
      for (int j = 0; j < EPL / 4; j++) {
        const float4 v = ldb4(rq, off + 16 * j);
        q[4 * j] = v.x; q[4 * j + 1] = v.y; q[4 * j + 2] = v.z; q[4 * j + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < EPL; e++) q[e] = ldb(rq, off + 4 * e);
    }
  }
  __device__ __forceinline__ static uint32_t row_off(int kvh, int p, int li) {
    return (uint32_t)(((kvh * s_a.max_ctx + p) * HD + li * EPL) * sizeof(KT));
  }

  // Scores, softmax statistics and o = sum p v of one item (kv head kvh, positions
  // [p0, p0 + n)), the record to the partial buffer.  k0 holds the K rows of the first round
  // (loaded before the grid barrier); row `fresh` (this step's position) is re-read here, since
  // it was appended during this launch.  The first round's V rows are loaded with q: they are
  // needed only after the scores.  Returns whether the half wrote a record.
  // wait_e > 0: the first round -- the K rows are loaded, then the grid barrier is waited for.
  __device__ __noinline__ static bool partial(int l, int kvh, int chunk, int n, int fresh, int half,
                                              unsigned wait_e) {
    const DecodeArgs& a = s_a;
    const int tid = threadIdx.x, ht = tid & (HT - 1), hw = ht >> 6, lane = tid & 63;
    const int li = ht % LPP, pg = ht / LPP;
    const int CL = a.chunk_len;
    const float scale = a.attn_scale;
    const size_t kv_half = a.layer_kv_bytes / 2;
    const uint8_t* kc = (const uint8_t*)a.kv + (size_t)l * a.layer_kv_bytes;
    const Rsrc rk = rsrc(kc, kv_half), rv = rsrc(kc + kv_half, kv_half);
    const Rsrc rq = rsrc(a.q, 4 * (size_t)a.qd);
    float* s_p = half_lds(half);
    float* s_red = s_p + G * CL;
    float* s_o = s_red + 4 * G;
    float* s_l = s_o + R * G * HD;
    const int p0 = chunk * CL;
    const bool act = n > 0;
    const int plast = min(p0 + CL, a.max_ctx) - 1;
    float k0[U][EPL];
#pragma unroll
    for (int u = 0; u < U; u++) ld_row<KT, EPL>(rk, row_off(kvh, min(p0 + u * R + pg, plast), li), k0[u]);
    if (wait_e) grid_wait(wait_e);

    float q[G][EPL];
#pragma unroll
    for (int h = 0; h < G; h++) load_q(rq, 4u * ((kvh * G + h) * HD + li * EPL), q[h]);
    float v0[U][EPL];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int p = min(p0 + u * R + pg, plast);
      ld_row<KT, EPL>(rv, row_off(kvh, p, li), v0[u]);
      if (p0 + u * R + pg == fresh) ld_row<KT, EPL>(rk, row_off(kvh, fresh, li), k0[u]);
    }

    float mloc[G];
#pragma unroll
    for (int h = 0; h < G; h++) mloc[h] = -INFINITY;
    if (act) {
      for (int base = p0; base < p0 + n; base += R * U) {
        float k[U][EPL];
        if (base == p0) {
#pragma unroll
          for (int u = 0; u < U; u++)
#pragma unroll
            for (int e = 0; e < EPL; e++) k[u][e] = k0[u][e];
        } else {
#pragma unroll
          for (int u = 0; u < U; u++)
            ld_row<KT, EPL>(rk, row_off(kvh, min(base + u * R + pg, plast), li), k[u]);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
          const int p = base + u * R + pg;
#pragma unroll
          for (int h = 0; h < G; h++) {
            float s = 0.f;
#pragma unroll
            for (int e = 0; e < EPL; e++) s = fmaf(q[h][e], k[u][e], s);
            s = lane_group_sum<LPP>(s) * scale;
            if (p < p0 + n) {
              mloc[h] = fmaxf(mloc[h], s);
              if (li == 0) s_p[h * CL + p - p0] = s;
            }
          }
        }
      }
    }
#pragma unroll
    for (int h = 0; h < G; h++) {
      const float m = wave_max_dpp(mloc[h]);
      if (lane == 0) s_red[hw * G + h] = m;
    }
    barrier_lds();
    float M[G];
#pragma unroll
    for (int h = 0; h < G; h++)
      M[h] = fmaxf(fmaxf(s_red[h], s_red[G + h]), fmaxf(s_red[2 * G + h], s_red[3 * G + h]));
    barrier_lds();
#pragma unroll
    for (int h = 0; h < G; h++) {
      float ls = 0.f;
      for (int j = ht; j < n; j += HT) {
        const float w = expf(s_p[h * CL + j] - M[h]);
        s_p[h * CL + j] = w;
        ls += w;
      }
      ls = wave_sum_dpp(ls);
      if (lane == 0) s_red[hw * G + h] = ls;
    }
    barrier_lds();
    if (ht < G) s_l[ht] = ((s_red[ht] + s_red[G + ht]) + s_red[2 * G + ht]) + s_red[3 * G + ht];

    float o[G][EPL];
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
      for (int e = 0; e < EPL; e++) o[h][e] = 0.f;
    if (act) {
      for (int base = p0; base < p0 + n; base += R * U) {
        float vv[U][EPL];
        if (base == p0) {
#pragma unroll
          for (int u = 0; u < U; u++)
#pragma unroll
            for (int e = 0; e < EPL; e++) vv[u][e] = v0[u][e];
        } else {
#pragma unroll
          for (int u = 0; u < U; u++)
            ld_row<KT, EPL>(rv, row_off(kvh, min(base + u * R + pg, plast), li), vv[u]);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
          const int p = base + u * R + pg;
          if (p < p0 + n) {
#pragma unroll
            for (int h = 0; h < G; h++) {
              const float w = s_p[h * CL + p - p0];
#pragma unroll
              for (int e = 0; e < EPL; e++) o[h][e] = fmaf(w, vv[u][e], o[h][e]);
            }
          }
        }
      }
    }
    // the R position groups summed in group order
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
      for (int e = 0; e < EPL; e++) s_o[(pg * G + h) * HD + li * EPL + e] = o[h][e];
    barrier_lds();
    if (act) {
      GLB float* rec = gp(a.part) + ((size_t)kvh * a.n_chunks + chunk) * G * PS;
      for (int i = ht; i < G * HD; i += HT) {
        const int h = i / HD, d = i % HD;
        float s = 0.f;
#pragma unroll
        for (int g = 0; g < R; g++) s += s_o[(g * G + h) * HD + d];
        st_f(rec + h * PS + d, s);
      }
      if (ht < G) {
        st_f(rec + ht * PS + HD, M[ht]);
        st_f(rec + ht * PS + HD + 1, s_l[ht]);
      }
    }
    return act;
  }
};

// ------------------------------------------------------------------ the phases
// candle rope_i on the pair at table index ti; KV pair store (fp16 packed or two f32)
__device__ __forceinline__ void store_kv(GLB uint8_t* cache, int kv_type, size_t ci, float a, float b) {
  if (kv_type == TPT_TYPE_F32) {
    st_f((GLB float*)cache + ci, a);
    st_f((GLB float*)cache + ci + 1, b);
  } else {
    st_u((GLB unsigned*)((GLB uint16_t*)cache + ci), (uint32_t)f2h(a) | ((uint32_t)f2h(b) << 16));
  }
}
// QKV: RMSNorm -> Q|K|V rows -> RoPE -> q buffer; K and V rows of position pos to the cache.
template <int BPP_H, int HD>
__device__ __noinline__ unsigned ph_qkv(int l, int pos, unsigned e) {
  const DecodeArgs& a = s_a;
  const int H = a.H, qd = a.qd, kd = a.kd, max_ctx = a.max_ctx, kv_type = a.kv_type;
  const GLB DecLayer* Ly = layer_of(l);
  Phase<BPP_H, 1, 1, 2> ph;
  ph.init(cg(Ly->qkv), nullptr, a.s_h, H, qd + 2 * kd, a.rpw_qkv);
  const GLB float* norm = cg(Ly->attn_norm);
  GLB uint8_t* kc = gp((uint8_t*)a.kv) + (size_t)l * a.layer_kv_bytes;
  GLB uint8_t* vc = kc + a.layer_kv_bytes / 2;
  const GLB float* rc = cg(a.rope_cos);
  const GLB float* rs = cg(a.rope_sin);
  GLB float* qb = gp(a.q);
  ph.issue_first();
  if (l > 0) grid_wait(e);
  GemvArgs A;
  A.K = H;
  A.prologue = PRO_RMSNORM;
  A.eps = a.eps;
  const Lds Ls = lds_layout(smem, H, ACT_Q8K);
  if (l == 0) ph.template prologue<true>(A, norm, Ls, LdsX{(const float4*)(smem + a.lds - 4 * (size_t)H)});
  else ph.template prologue<true>(A, norm, Ls, AgentX{rsrc(a.x, 4 * (size_t)H)});
  ph.run(Ls);
  const int nr = ph.nrows(), r0 = ph.r0;
  for (int i = 2 * threadIdx.x; i < nr; i += 2 * NT) {
    const float x0 = Ls.rows[i], x1 = Ls.rows[i + 1];
    const int lrow = r0 + i;
    if (lrow < qd + kd) {
      const bool isq = lrow < qd;
      const int rr = isq ? lrow : lrow - qd;
      const size_t ti = (size_t)pos * (HD / 2) + ((rr % HD) >> 1);
      const float cs = rc[ti], sn = rs[ti];
      // candle rope_i: dst[2i] = x0*cos - x1*sin; dst[2i+1] = x0*sin + x1*cos
      const float o0 = x0 * cs - x1 * sn, o1 = x0 * sn + x1 * cs;
      if (isq) {
        st_f(qb + rr, o0);
        st_f(qb + rr + 1, o1);
      } else {
        store_kv(kc, kv_type, ((size_t)(rr / HD) * max_ctx + pos) * HD + rr % HD, o0, o1);
      }
    } else {
      const int rr = lrow - qd - kd;
      store_kv(vc, kv_type, ((size_t)(rr / HD) * max_ctx + pos) * HD + rr % HD, x0, x1);
    }
  }
  return grid_arrive(e);
}

// ATT: the partial records of this workgroup's items (kv head, chunk).  The first round's K rows
// of earlier positions were written by earlier launches, so their loads are issued before the
// grid barrier; q, V and this step's new row are read after it.
template <typename KT, int HD, int G>
__device__ __noinline__ unsigned ph_att(int l, int pos, unsigned e) {
  using AT = Att<KT, HD, G>;
  const DecodeArgs& a = s_a;
  const int L = pos + 1, nch = a.n_chunks, CL = a.chunk_len;
  const int n_items = a.nkv * nch;
  const int half = threadIdx.x >> 8;
  const int rounds = (n_items + 2 * (int)gridDim.x - 1) / (2 * (int)gridDim.x);
  for (int rd = 0; rd < rounds; rd++) {
    const int item = (rd * (int)gridDim.x + (int)blockIdx.x) * 2 + half;
    const bool valid = item < n_items;
    const int kvh = valid ? item / nch : 0, chunk = valid ? item % nch : 0;
    const int n = valid ? min(L, chunk * CL + CL) - chunk * CL : 0;
    AT::partial(l, kvh, chunk, n, pos, half, rd == 0 ? e : 0u);
  }
  if (rounds == 0) grid_wait(e);
  if (l == 0 && blockIdx.x == 0 && threadIdx.x == 0) {  // every workgroup has read the step state
    GLB StepState* st = gp(a.st);
    const int np = st->parity ^ 1;
    st->pos = pos;
    st->next_pos = pos + 1;
    st->parity = np;
    st->amax[np] = 0ull;
    st->use_override = 0;
    if (a.tok_log) gp(a.tok_log)[pos] = s_c.tok;
    *gp(a.epoch) = s_c.base + (unsigned)decode_layers_barriers(a.n_layers);
  }
  return grid_arrive(e);
}

// MRG: att[i] = sum_c w_c o_c[i] / sum_c w_c l_c with w_c = exp(m_c - max m) over the nact live
// chunk records of head i / HD: attn_merge_kernel's arithmetic in its order (k_attn.hip: eight
// interleaved chunk sets, then the sets in order), each workgroup taking a slice of dpw
// consecutive output dims, merged by its first wave (the dims of a slice touch at most two
// heads).  All records of up to MC chunks are loaded in one round.
template <int HD, int G>
__device__ __noinline__ unsigned ph_mrg(int pos, unsigned e) {
  constexpr int PS = HD + 2, MC = 48;
  grid_wait(e);
  const DecodeArgs& a = s_a;
  const int L = pos + 1, nch = a.n_chunks, CL = a.chunk_len;
  const int nact = min(nch, (L + CL - 1) / CL);
  const int nd = a.nq * HD;
  const int dpw = (nd + (int)gridDim.x - 1) / (int)gridDim.x;  // <= 64 (the host checks)
  const int i0 = (int)blockIdx.x * dpw;
  const int lane = threadIdx.x & 63;
  if (threadIdx.x < WAVE && i0 < nd) {
    const Rsrc rp = rsrc(a.part, 4 * (size_t)a.nkv * nch * G * PS);
    float* wbuf = (float*)smem;  // [2][nch]
    const int ilast = min(i0 + dpw, nd) - 1;
    const int i = i0 + lane, ic = min(i, ilast);
    const int h = ic / HD, d = ic % HD;
    const int hlo = i0 / HD, hhi = ilast / HD;
    auto rec = [&](int c, int hh) -> uint32_t {  // record (kv head hh / G, chunk c, head hh % G)
      return (uint32_t)((((hh / G) * nch + c) * G + hh % G) * PS);
    };
    const int cl = min(lane, nact - 1);
    const float m_lo = ldb(rp, 4u * (rec(cl, hlo) + HD)), l_lo = ldb(rp, 4u * (rec(cl, hlo) + HD + 1));
    const float m_hi = ldb(rp, 4u * (rec(cl, hhi) + HD)), l_hi = ldb(rp, 4u * (rec(cl, hhi) + HD + 1));
    float ov[MC];
#pragma unroll
    for (int c = 0; c < MC; c++) ov[c] = ldb(rp, 4u * (rec(min(c, nact - 1), h) + d));
    float lsum[2];
#pragma unroll
    for (int s2 = 0; s2 < 2; s2++) {
      const int hh = s2 ? hhi : hlo;
      const float mv = s2 ? m_hi : m_lo, lv = s2 ? l_hi : l_lo;
      float mm = lane < nact ? mv : -INFINITY;
      for (int c = lane + WAVE; c < nact; c += WAVE) mm = fmaxf(mm, ldb(rp, 4u * (rec(c, hh) + HD)));
      mm = wave_max_dpp(mm);
      float ls = 0.f;
      if (lane < nact) {
        const float w = expf(mv - mm);
        wbuf[s2 * nch + lane] = w;
        ls = fmaf(w, lv, ls);
      }
      for (int c = lane + WAVE; c < nact; c += WAVE) {
        const float w = expf(ldb(rp, 4u * (rec(c, hh) + HD)) - mm);
        wbuf[s2 * nch + c] = w;
        ls = fmaf(w, ldb(rp, 4u * (rec(c, hh) + HD + 1)), ls);
      }
      lsum[s2] = wave_sum_dpp(ls);
    }
    if (i <= ilast) {
      const bool lo = h == hlo;
      const float* w = wbuf + (lo ? 0 : nch);
      float sv[8];  // set j sums the chunks c = j, j + 8, ... in order
#pragma unroll
      for (int j = 0; j < 8; j++) sv[j] = 0.f;
#pragma unroll
      for (int c = 0; c < MC; c++)
        if (c < nact) sv[c % 8] = fmaf(w[c], ov[c], sv[c % 8]);
      for (int cb = MC; cb < nact; cb += MC) {  // further chunks, MC (a multiple of 8) per round
#pragma unroll
        for (int c = 0; c < MC; c++) ov[c] = ldb(rp, 4u * (rec(min(cb + c, nact - 1), h) + d));
#pragma unroll
        for (int c = 0; c < MC; c++)
          if (cb + c < nact) sv[c % 8] = fmaf(w[cb + c], ov[c], sv[c % 8]);
      }
      float t = 0.f;
#pragma unroll
      for (int j = 0; j < 8; j++) t += sv[j];
      st_f(gp(a.att) + i, t / (lo ? lsum[0] : lsum[1]));
    }
  }
  return grid_arrive(e);
}

// WO: x += Wo . att
template <int BPP_H>
__device__ __noinline__ unsigned ph_wo(int l, unsigned e) {
  const DecodeArgs& a = s_a;
  const int H = a.H, qd = a.qd;
  Phase<BPP_H, 1, 1, 2> ph;
  ph.init(cg(layer_of(l)->o), nullptr, a.s_q, qd, H, a.rpw_o);
  const Rsrc rx = rsrc(a.x, 4 * (size_t)H), ratt = rsrc(a.att, 4 * (size_t)qd);
  GLB float* x = gp(a.x);
  ph.issue_first();
  grid_wait(e);
  GemvArgs A;
  A.K = qd;
  A.prologue = PRO_PLAIN;
  const Lds Ls = lds_layout(smem, qd, ACT_Q8K);
  ph.template prologue<false>(A, nullptr, Ls, AgentX{ratt});
  ph.run(Ls);
  const int nr = ph.nrows(), r0 = ph.r0;
  for (int i = threadIdx.x; i < nr; i += NT) st_f(x + r0 + i, Ls.rows[i] + ldb(rx, 4u * (r0 + i)));
  return grid_arrive(e);
}

// GU: h = silu(W1 . n(x)) * (W3 . n(x))
template <int BPP_H>
__device__ __noinline__ unsigned ph_gu(int l, unsigned e) {
  const DecodeArgs& a = s_a;
  const int H = a.H, F = a.F;
  const GLB DecLayer* Ly = layer_of(l);
  Phase<BPP_H, 1, 2, 2> ph;
  ph.init(cg(Ly->gate), cg(Ly->up), a.s_h, H, F, a.rpw_gu);
  const GLB float* norm = cg(Ly->ffn_norm);
  const Rsrc rx = rsrc(a.x, 4 * (size_t)H);
  GLB float* hb = gp(a.h);
  ph.issue_first();
  grid_wait(e);
  GemvArgs A;
  A.K = H;
  A.prologue = PRO_RMSNORM;
  A.eps = a.eps;
  const Lds Ls = lds_layout(smem, H, ACT_Q8K);
  ph.template prologue<true>(A, norm, Ls, AgentX{rx});
  ph.run(Ls);
  const int nr = ph.nrows(), r0 = ph.r0;
  for (int i = threadIdx.x; i < nr; i += NT) st_f(hb + r0 + i, silu_mul(Ls.rows[2 * i], Ls.rows[2 * i + 1]));
  return grid_arrive(e);
}

// DN: x += W2 . h (no arrival after the last layer: the launch ends there)
template <int BPP_F, int RB_F>
__device__ __noinline__ unsigned ph_dn(int l, unsigned e, bool last) {
  const DecodeArgs& a = s_a;
  const int H = a.H, F = a.F;
  Phase<BPP_F, RB_F, 1, 2> ph;
  ph.init(cg(layer_of(l)->down), nullptr, a.s_f, F, H, a.rpw_dn);
  const Rsrc rx = rsrc(a.x, 4 * (size_t)H), rh = rsrc(a.h, 4 * (size_t)F);
  GLB float* x = gp(a.x);
  ph.issue_first();
  grid_wait(e);
  GemvArgs A;
  A.K = F;
  A.prologue = PRO_PLAIN;
  const Lds Ls = lds_layout(smem, F, ACT_Q8K);
  ph.template prologue<false>(A, nullptr, Ls, AgentX{rh});
  ph.run(Ls);
  const int nr = ph.nrows(), r0 = ph.r0;
  for (int i = threadIdx.x; i < nr; i += NT) st_f(x + r0 + i, Ls.rows[i] + ldb(rx, 4u * (r0 + i)));
  return last ? e : grid_arrive(e);
}

// ------------------------------------------------------------------ the kernel
template <typename KT, int HD, int G, int BPP_H, int BPP_F, int RB_F>
__global__ void __launch_bounds__(NT, 1) decode_layers_kernel(const DecodeArgs a) {
  const int tid = threadIdx.x, wg = blockIdx.x;
  // launch arguments to LDS (the phases read them there)
  {
    const int* src = (const int*)&a;
    int* dst = (int*)&s_a;
    for (int i = tid; i < (int)(sizeof(DecodeArgs) / 4); i += NT) dst[i] = src[i];
  }
  // step begin: the token of this position (prompt, override or the last step's argmax)
  if (tid == 0) {
    const StepState* st = a.st;
    const int pos = st->next_pos;
    uint32_t tok;
    if (pos < st->prompt_len) tok = a.prompt[pos];
    else if (st->use_override) tok = st->tok_override;
    else tok = (uint32_t)(st->amax[st->parity] & 0xffffffffull);
    if (tok >= (uint32_t)a.vocab) tok = (uint32_t)(a.vocab - 1);  // never index past the table
    s_c.tok = tok;
    s_c.pos = pos;
    s_c.base = *a.epoch;
    s_c.dead = 0;
  }
  barrier_lds();
  const int pos = s_c.pos;
  // its embedding row, dequantized by every workgroup into LDS (top of the dynamic region); the
  // workgroup's own rows of the residual stream to memory
  {
    const int H = a.H;
    float* ex = (float*)(smem + a.lds - 4 * (size_t)H);
    const uint8_t* row = a.embd + (size_t)s_c.tok * a.embd_row;
    for (int i = tid; i < H; i += NT) ex[i] = dequant_elem(a.embd_type, row, i);
    barrier_lds();
    for (int i = tid; i < a.rpw_o; i += NT) {
      const int r = wg * a.rpw_o + i;
      if (r < H) st_f(gp(a.x) + r, ex[r]);
    }
  }
  unsigned e = 0;
  for (int l = 0; l < a.n_layers; l++) {
    e = ph_qkv<BPP_H, HD>(l, pos, e);
    e = ph_att<KT, HD, G>(l, pos, e);
    e = ph_mrg<HD, G>(pos, e);
    e = ph_wo<BPP_H>(l, e);
    e = ph_gu<BPP_H>(l, e);
    e = ph_dn<BPP_F, RB_F>(l, e, l + 1 == a.n_layers);
  }
}

// ------------------------------------------------------------------ host side
struct Cfg {
  int kv_type, hd, g, bpp_h, bpp_f, rb_f;
};
// the instantiated shapes: Llama-3 8B (hd 128, GQA 4, H 4096, F 14336), Llama-3.2 1B (hd 64,
// GQA 4, H 2048, F 8192) and the tiny test model (hd 64, GQA 2, H 256, F 512); fp16 or f32 cache
#define TPT_DECODE_CFGS(X)                     \
  X(TPT_TYPE_F16, uint16_t, 128, 4, 16, 16, 2) \
  X(TPT_TYPE_F32, float, 128, 4, 16, 16, 2)    \
  X(TPT_TYPE_F16, uint16_t, 64, 4, 8, 16, 1)   \
  X(TPT_TYPE_F32, float, 64, 4, 8, 16, 1)      \
  X(TPT_TYPE_F16, uint16_t, 64, 2, 1, 2, 1)    \
  X(TPT_TYPE_F32, float, 64, 2, 1, 2, 1)

int bpp_of(int K) {
  const int nb = K / QK_K;
  return nb >= 16 ? 16 : nb >= 8 ? 8 : nb >= 4 ? 4 : nb >= 2 ? 2 : 1;
}
int rows_per_wg(int N, int grid, int bpp, int rb) {
  const int rg = rb * (16 / bpp);
  const int unit = rg >= 2 ? rg : 2;
  int rpw = (N + grid - 1) / grid;
  return (rpw + unit - 1) / unit * unit;
}

}  // namespace

// dynamic LDS limit of the kernel: gfx950's 160 KB less the static arguments block
constexpr int kMaxLds = 159 * 1024;

int decode_layers_plan(const tpt_ctx* ctx, DecodeArgs& a) {
  const int grid = ctx && ctx->n_cu > 0 ? ctx->n_cu : 256;
  if (grid > NT) return fail(TPT_ERR_UNSUPPORTED, "decode layers: more compute units than poll threads");
  if (a.qd != a.H) return fail(TPT_ERR_UNSUPPORTED, "decode layers: q width must equal the embedding width");
  if (a.H % 256 || a.F % 256 || a.H > 16384 || a.F > 16384) return fail(TPT_ERR_UNSUPPORTED, "decode layers: unsupported widths");
  if (a.nq % a.nkv) return fail(TPT_ERR_INVALID, "decode layers: bad head counts");
  const int g = a.nq / a.nkv, bh = bpp_of(a.H), bf = bpp_of(a.F), rbf = a.F > 8192 ? 2 : 1;
  bool found = false;
#define TPT_MATCH(KVT, KT, HD, G, BH, BF, RBF) \
  if (a.kv_type == KVT && a.hd == HD && g == G && bh == BH && bf == BF && rbf == RBF) found = true;
  TPT_DECODE_CFGS(TPT_MATCH)
#undef TPT_MATCH
  if (!found) return fail(TPT_ERR_UNSUPPORTED, "decode layers: no persistent kernel for this shape");
  // dynamic LDS beyond 64 KB (the attention's per-position-group sums at long chunks) needs the
  // function attribute, set once per instantiation and device
  int dev = 0;
  TPT_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return fail(TPT_ERR_UNSUPPORTED, "decode layers: device index out of range");
#define TPT_ATTR(KVT, KT, HD, G, BH, BF, RBF)                                                     \
  if (a.kv_type == KVT && a.hd == HD && g == G && bh == BH && bf == BF && rbf == RBF) {            \
    static std::atomic<uint64_t> done{0};                                                         \
    if (!(done.load() >> dev & 1)) {                                                              \
      TPT_HIP(hipFuncSetAttribute((const void*)decode_layers_kernel<KT, HD, G, BH, BF, RBF>,      \
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds));          \
      done.fetch_or(1ull << dev);                                                                 \
    }                                                                                             \
  }
  TPT_DECODE_CFGS(TPT_ATTR)
#undef TPT_ATTR
  if (a.n_chunks <= 0 || a.chunk_len <= 0 || a.chunk_len % 16 || (long)a.n_chunks * a.chunk_len < 1)
    return fail(TPT_ERR_INVALID, "decode layers: bad attention partition");
  a.grid = grid;
  a.rpw_qkv = rows_per_wg(a.qd + 2 * a.kd, grid, bh, 1);
  a.rpw_o = rows_per_wg(a.H, grid, bh, 1);
  a.rpw_gu = rows_per_wg(a.F, grid, bh, 1);
  a.rpw_dn = rows_per_wg(a.H, grid, bf, rbf);
  if ((a.rpw_qkv & 1)) return fail(TPT_ERR_INVALID, "decode layers: odd QKV rows per workgroup");
  size_t gm = gemv_lds_bytes(a.H, a.rpw_qkv);
  gm = std::max(gm, gemv_lds_bytes(a.qd, a.rpw_o));
  gm = std::max(gm, gemv_lds_bytes(a.H, 2 * a.rpw_gu));
  gm = std::max(gm, gemv_lds_bytes(a.F, a.rpw_dn));
  const size_t emb = gm + 4 * (size_t)a.H;
  const int R = 256 / (a.kv_type == TPT_TYPE_F32 ? 32 : 16);  // positions per attention round
  const size_t att = 2 * 4 * (size_t)att_half_floats(g, a.hd, R, a.chunk_len);
  if ((long)a.nq * a.hd > 64L * grid) return fail(TPT_ERR_UNSUPPORTED, "decode layers: merge slices wider than a wave");
  const size_t mrg = 2 * 4 * (size_t)a.n_chunks;
  const size_t lds = (std::max(std::max(emb, att), mrg) + 15) & ~(size_t)15;
  if (lds > (size_t)kMaxLds) return fail(TPT_ERR_UNSUPPORTED, "decode layers: LDS budget exceeded");
  // The grid barriers need every workgroup resident at once: one per compute unit must fit
  // with this LDS size and the instantiation's registers.  (Work of other streams or processes
  // can still hold compute units; the barrier's bounded wait then reports an error.)
  int per_cu = 0;
#define TPT_OCC(KVT, KT, HD, G, BH, BF, RBF)                                                      \
  if (a.kv_type == KVT && a.hd == HD && g == G && bh == BH && bf == BF && rbf == RBF)              \
    TPT_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(                                         \
        &per_cu, (const void*)decode_layers_kernel<KT, HD, G, BH, BF, RBF>, NT, lds));
  TPT_DECODE_CFGS(TPT_OCC)
#undef TPT_OCC
  if ((long)per_cu * grid < grid)
    return fail(TPT_ERR_UNSUPPORTED, "decode layers: a workgroup per compute unit cannot be resident");
  a.lds = (int)lds;
  return TPT_OK;
}

int launch_decode_layers(const DecodeArgs& a, hipStream_t s) {
  if (a.grid <= 0 || a.lds <= 0) return fail(TPT_ERR_INVALID, "decode layers: plan the launch first");
  const int g = a.nq / a.nkv, bh = bpp_of(a.H), bf = bpp_of(a.F), rbf = a.F > 8192 ? 2 : 1;
#define TPT_LAUNCH(KVT, KT, HD, G, BH, BF, RBF)                                                   \
  if (a.kv_type == KVT && a.hd == HD && g == G && bh == BH && bf == BF && rbf == RBF) {            \
    hipLaunchKernelGGL((decode_layers_kernel<KT, HD, G, BH, BF, RBF>), dim3((unsigned)a.grid),     \
                       dim3(NT), (size_t)a.lds, s, a);                                            \
    TPT_HIP(hipGetLastError());                                                                   \
    return TPT_OK;                                                                                \
  }
  TPT_DECODE_CFGS(TPT_LAUNCH)
#undef TPT_LAUNCH
  return fail(TPT_ERR_UNSUPPORTED, "decode layers: no persistent kernel for this shape");
}

}  // namespace tpt
