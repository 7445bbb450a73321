// Small kernels of the decode path: bit-exact dequantization, the decode-step prologue
// (token pick + embedding row), RMSNorm, RoPE and argmax as standalone ops.
#include <cstddef>

#include "kernels.h"

namespace tpt {
namespace {

__global__ void dequant_kernel(int type, const uint8_t* __restrict__ w, float* __restrict__ y,
                               int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    y[i] = dequant_elem(type, w, i);
}

// Decode-step prologue (one workgroup): the token of this position (prompt, host override or
// the previous step's argmax), then its embedding row: the row's bytes are staged in LDS with
// independent 2-byte loads (every GGUF row length here is even) and dequantized from there.
// The whole step state is read in one round trip (three 16-byte loads, both argmax slots), so
// a decode step waits for two dependent loads (state, row) before the row is in LDS.
static_assert(offsetof(StepState, next_pos) == 4 && offsetof(StepState, parity) == 8 &&
                  offsetof(StepState, use_override) == 12 && offsetof(StepState, tok_override) == 16 &&
                  offsetof(StepState, prompt_len) == 20 && offsetof(StepState, amax) == 32 &&
                  sizeof(StepState) == 48,
              "step_begin_kernel reads StepState as three 16-byte words");
__global__ void __launch_bounds__(256) step_begin_kernel(StepState* st, const uint32_t* prompt,
                                                         int embd_type, const uint8_t* embd,
                                                         size_t embd_row_bytes, int H, int vocab,
                                                         float* x, uint32_t* tok_log, float* ssq,
                                                         int n_ssq) {
  extern __shared__ __align__(16) uint16_t s_row[];
  __shared__ uint32_t s_tok;
  __shared__ int s_pos;
  __shared__ float s_ss[256 / WAVE];
  if (threadIdx.x == 0) {
    const uint4* sw = (const uint4*)st;  // 256-byte aligned in the runtime buffer
    const uint4 w0 = sw[0], w1 = sw[1], w2 = sw[2];
    const int pos = (int)w0.y, parity = (int)w0.z, use_override = (int)w0.w;
    const int prompt_len = (int)w1.y;
    uint32_t tok;
    if (pos < prompt_len) tok = prompt[pos];
    else if (use_override) tok = w1.x;
    else tok = parity ? w2.z : w2.x;  // low 32 bits of amax[parity]: the index
    if (tok >= (uint32_t)vocab) tok = (uint32_t)(vocab - 1);  // never index past the table
    s_tok = tok;
    s_pos = pos;
  }
  __syncthreads();
  const uint16_t* row = (const uint16_t*)(embd + (size_t)s_tok * embd_row_bytes);
  const int nh = (int)(embd_row_bytes / 2);
  for (int i = threadIdx.x; i < nh; i += blockDim.x) s_row[i] = row[i];
  __syncthreads();
  float ss = 0.f;
  for (int i = threadIdx.x; i < H; i += blockDim.x) {
    const float v = dequant_elem(embd_type, (const uint8_t*)s_row, i);
    x[i] = v;
    ss = fmaf(v, v, ss);
  }
  if (ssq) {  // sum(x^2) for the first layer's RMSNorm: the total in slot 0, zeros after it
    ss = wave_sum_dpp(ss);
    if ((threadIdx.x & 63) == 0) s_ss[threadIdx.x >> 6] = ss;
    __syncthreads();
    for (int i = threadIdx.x; i < n_ssq; i += blockDim.x) {
      float t = 0.f;
      if (i == 0)
        for (int w = 0; w < 256 / WAVE; w++) t += s_ss[w];
      ssq[i] = t;
    }
  }
  if (threadIdx.x == 0) {
    const int np = st->parity ^ 1;
    st->pos = s_pos;
    st->next_pos = s_pos + 1;
    st->parity = np;
    st->amax[np] = 0ull;
    st->use_override = 0;
    if (tok_log) tok_log[s_pos] = s_tok;
  }
}

// Embedding rows of T token ids (prefill): x[t] = dequant(embd[ids[t]]), one workgroup per row.
__global__ void __launch_bounds__(256) embed_rows_kernel(const uint32_t* ids, int embd_type,
                                                         const uint8_t* embd, size_t embd_row_bytes,
                                                         int H, float* x) {
  const int t = blockIdx.x;
  const uint8_t* row = embd + (size_t)ids[t] * embd_row_bytes;
  for (int i = threadIdx.x; i < H; i += blockDim.x) x[(size_t)t * H + i] = dequant_elem(embd_type, row, i);
}

// Q/K/V post-pass of the prefill: one thread per (even, odd) element pair of a row.  RoPE as
// candle's rope_i (dst[2i] = x0*cos - x1*sin; dst[2i+1] = x0*sin + x1*cos) at the row's position,
// the same arithmetic as the decode GEMV's epilogue.
__global__ void __launch_bounds__(256) qkv_post_kernel(const QkvPostArgs a) {
  const int t = blockIdx.y, pos = a.pos0 + t;
  const int npair = (a.qd + 2 * a.kd) / 2;
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= npair) return;
  const int e = 2 * p;
  const float* row = a.qkv + (size_t)t * (a.qd + 2 * a.kd);
  const float x0 = row[e], x1 = row[e + 1];
  float o0 = x0, o1 = x1;
  if (e < a.qd + a.kd) {
    const int rr = e < a.qd ? e : e - a.qd;
    const size_t ti = (size_t)pos * (a.hd / 2) + ((rr % a.hd) >> 1);
    const float cs = a.rope_cos[ti], sn = a.rope_sin[ti];
    o0 = x0 * cs - x1 * sn;
    o1 = x0 * sn + x1 * cs;
  }
  if (e < a.qd) {
    a.q[(size_t)t * a.qd + e] = o0;
    a.q[(size_t)t * a.qd + e + 1] = o1;
    return;
  }
  const bool isk = e < a.qd + a.kd;
  const int rr = isk ? e - a.qd : e - a.qd - a.kd;
  const size_t ci = ((size_t)(rr / a.hd) * a.max_ctx + pos) * a.hd + rr % a.hd;
  void* cache = isk ? a.kcache : a.vcache;
  if (a.kv_type == TPT_TYPE_F32) {
    ((float*)cache)[ci] = o0;
    ((float*)cache)[ci + 1] = o1;
  } else {
    ((uint16_t*)cache)[ci] = f2h(o0);
    ((uint16_t*)cache)[ci + 1] = f2h(o1);
  }
}

// y[i] = silu(g[i]) * u[i] (the elementwise op the GEMV and GEMM epilogues fuse)
__global__ void __launch_bounds__(256) swiglu_kernel(const float* g, const float* __restrict__ u,
                                                     float* y, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = silu_mul(g[i], u[i]);
}

// candle_nn::ops::rms_norm: m = sqrt(sum(x^2)/n + eps); y = x / m * w (one workgroup)
__global__ void __launch_bounds__(1024) rmsnorm_kernel(const float* __restrict__ x,
                                                       const float* __restrict__ w,
                                                       float* __restrict__ y, int n, float eps) {
  __shared__ float red[16];
  float ss = 0.f;
  for (int i = threadIdx.x; i < n; i += blockDim.x) ss = fmaf(x[i], x[i], ss);
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < (int)(blockDim.x >> 6); i++) t += red[i];
  const float m = sqrtf(t / (float)n + eps);
  for (int i = threadIdx.x; i < n; i += blockDim.x) y[i] = x[i] / m * w[i];
}

// candle rope_i over n_heads heads of hd at one position
__global__ void rope_kernel(float* __restrict__ x, int n_pairs, int hd, int pos,
                            const float* __restrict__ c, const float* __restrict__ s) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_pairs) return;
  const int i = t % (hd / 2);
  const float cs = c[(size_t)pos * (hd / 2) + i], sn = s[(size_t)pos * (hd / 2) + i];
  const float x0 = x[2 * t], x1 = x[2 * t + 1];
  x[2 * t] = x0 * cs - x1 * sn;
  x[2 * t + 1] = x0 * sn + x1 * cs;
}

__global__ void __launch_bounds__(256) argmax_kernel(const float* __restrict__ v, int64_t n,
                                                     unsigned long long* slot) {
  unsigned long long best = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const unsigned long long k = ((unsigned long long)order_key(v[i]) << 32) | (unsigned long long)i;
    best = k > best ? k : best;
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const unsigned long long ob = __shfl_xor(best, o, WAVE);
    best = ob > best ? ob : best;
  }
  if ((threadIdx.x & 63) == 0) atomicMax(slot, best);
}

// plain 16-byte vector copy, grid-stride (HBM calibration reference)
__global__ void __launch_bounds__(256) copy_kernel(uint4* __restrict__ dst,
                                                   const uint4* __restrict__ src, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

}  // namespace

int launch_copy(void* dst, const void* src, size_t bytes, hipStream_t s) {
  const size_t n = bytes / 16;
  size_t blocks = (n + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  if (blocks == 0) return TPT_OK;
  hipLaunchKernelGGL(copy_kernel, dim3((unsigned)blocks), dim3(256), 0, s, (uint4*)dst,
                     (const uint4*)src, n);
  TPT_HIP(hipGetLastError());
  return TPT_OK;
}

int launch_dequant(int type, const void* w, float* y, int64_t n, hipStream_t s) {
  const int bs = type_block(type);
  if (type_bytes(type) == 0) return fail(TPT_ERR_UNSUPPORTED, "dequant: unsupported type");
  if (n < 0 || n % bs) return fail(TPT_ERR_INVALID, "dequant: n must be a multiple of the block size");
  if (n == 0) return TPT_OK;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)blocks), dim3(256), 0, s, type,
                     (const uint8_t*)w, y, n);
  TPT_HIP(hipGetLastError());
  return TPT_OK;
}

int launch_step_begin(StepState* st, const uint32_t* prompt, int embd_type, const uint8_t* embd,
                      size_t embd_row_bytes, int H, int vocab, float* x, uint32_t* tok_log,
                      float* ssq, int n_ssq, hipStream_t s) {
  if (embd_row_bytes % 2 || embd_row_bytes > 65536)
    return fail(TPT_ERR_UNSUPPORTED, "embedding rows must be of even length and at most 64 KB");
  if (ssq && (n_ssq < 1 || n_ssq > kSsqMax)) return fail(TPT_ERR_INVALID, "step begin: 1 .. 256 partial sums");
  hipLaunchKernelGGL(step_begin_kernel, dim3(1), dim3(256), embd_row_bytes, s, st, prompt,
                     embd_type, embd, embd_row_bytes, H, vocab, x, tok_log, ssq, n_ssq);
  TPT_HIP(hipGetLastError());
  return TPT_OK;
}

int launch_embed_rows(const uint32_t* ids, int T, int embd_type, const uint8_t* embd,
                      size_t embd_row_bytes, int H, float* x, hipStream_t s) {
  if (T <= 0 || H <= 0) return fail(TPT_ERR_INVALID, "embed_rows: bad shape");
  hipLaunchKernelGGL(embed_rows_kernel, dim3((unsigned)T), dim3(256), 0, s, ids, embd_type, embd,
                     embd_row_bytes, H, x);
  TPT_HIP(hipGetLastError());
  return TPT_OK;
}

int launch_qkv_post(const QkvPostArgs& a, hipStream_t s) {
  if (a.T <= 0 || a.qd <= 0 || a.kd <= 0 || a.hd <= 0 || (a.hd & 1) || a.qd % a.hd || a.kd % a.hd)
    return fail(TPT_ERR_INVALID, "qkv_post: bad shape");
  if (a.pos0 < 0 || a.pos0 + a.T > a.max_ctx) return fail(TPT_ERR_INVALID, "qkv_post: positions past the cache");
  const int npair = (a.qd + 2 * a.kd) / 2;
  hipLaunchKernelGGL(qkv_post_kernel, dim3((unsigned)((npair + 255) / 256), (unsigned)a.T), dim3(256), 0, s, a);
  TPT_HIP(hipGetLastError());
  return TPT_OK;
}

int launch_swiglu(const float* g, const float* u, float* y, int n, hipStream_t s) {
  if (n <= 0) return fail(TPT_ERR_INVALID, "swiglu: n must be positive");
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, g, u, y, n);
  TPT_HIP(hipGetLastError());
  return TPT_OK;
}

int launch_rmsnorm(const float* x, const float* w, float* y, int n, float eps, hipStream_t s) {
  if (n <= 0) return fail(TPT_ERR_INVALID, "rmsnorm: n must be positive");
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(1024), 0, s, x, w, y, n, eps);
  TPT_HIP(hipGetLastError());
  return TPT_OK;
}

int launch_rope(float* x, int n_heads, int hd, int pos, const float* c, const float* sn,
                hipStream_t s) {
  if (n_heads <= 0 || hd <= 0 || (hd & 1) || pos < 0) return fail(TPT_ERR_INVALID, "rope: bad shape");
  const int pairs = n_heads * hd / 2;
  hipLaunchKernelGGL(rope_kernel, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, s, x, pairs,
                     hd, pos, c, sn);
  TPT_HIP(hipGetLastError());
  return TPT_OK;
}

int launch_argmax(const float* logits, int64_t n, unsigned long long* slot, hipStream_t s) {
  if (n <= 0 || n > 0xffffffffll) return fail(TPT_ERR_INVALID, "argmax: bad length");
  int64_t blocks = (n + 255) / 256;
  if (blocks > 1024) blocks = 1024;
  hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)blocks), dim3(256), 0, s, logits, n, slot);
  TPT_HIP(hipGetLastError());
  return TPT_OK;
}

}  // namespace tpt
