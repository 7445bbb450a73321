// C ABI: error reporting, context, device memory and the op-level entry points.
#include <stdio.h>

#include <cmath>
#include <string>
#include <vector>

#include "kernels.h"

namespace tpt {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what, const char* file, int line) {
  char buf[512];
  snprintf(buf, sizeof buf, "HIP error %d (%s) in %s at %s:%d", (int)e, hipGetErrorString(e), what,
           file, line);
  g_last_error = buf;
  return e == hipErrorOutOfMemory ? TPT_ERR_OOM : TPT_ERR_HIP;
}

int ctx_enter(tpt_ctx* c) {
  if (!c) return fail(TPT_ERR_INVALID, "null context");
  TPT_HIP(hipSetDevice(c->device));
  return TPT_OK;
}

}  // namespace tpt

using namespace tpt;

#define ENTER(c)                        \
  do {                                  \
    int _rc = ::tpt::ctx_enter(c);      \
    if (_rc) return _rc;                \
  } while (0)

extern "C" {

const char* tpt_last_error(void) { return g_last_error.c_str(); }
int tpt_version(void) { return 1; }

int tpt_ctx_create(int device, tpt_ctx** out) {
  if (!out) return fail(TPT_ERR_INVALID, "null out pointer");
  int n = 0;
  TPT_HIP(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) return fail(TPT_ERR_INVALID, "device index out of range");
  TPT_HIP(hipSetDevice(device));
  tpt_ctx* c = new tpt_ctx();
  c->device = device;
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e == hipSuccess) {
    c->n_cu = prop.multiProcessorCount;
    snprintf(c->name, sizeof c->name, "%s (%s)", prop.name, prop.gcnArchName);
  }
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    return hip_fail(e, "tpt_ctx_create", __FILE__, __LINE__);
  }
  *out = c;
  return TPT_OK;
}

int tpt_ctx_destroy(tpt_ctx* c) {
  if (!c) return TPT_OK;
  ENTER(c);
  (void)hipStreamSynchronize(c->stream);
  (void)hipStreamDestroy(c->stream);
  delete c;
  return TPT_OK;
}

int tpt_ctx_synchronize(tpt_ctx* c) {
  ENTER(c);
  TPT_HIP(hipStreamSynchronize(c->stream));
  return TPT_OK;
}

int tpt_ctx_device_info(tpt_ctx* c, int* n_cu, char* name, int name_len) {
  ENTER(c);
  if (n_cu) *n_cu = c->n_cu;
  if (name && name_len > 0) snprintf(name, (size_t)name_len, "%s", c->name);
  return TPT_OK;
}

int tpt_malloc(tpt_ctx* c, size_t bytes, void** dptr) {
  ENTER(c);
  if (!dptr) return fail(TPT_ERR_INVALID, "null out pointer");
  TPT_HIP(hipMalloc(dptr, bytes ? bytes : 1));
  return TPT_OK;
}

int tpt_free(tpt_ctx* c, void* dptr) {
  ENTER(c);
  if (dptr) TPT_HIP(hipFree(dptr));
  return TPT_OK;
}

int tpt_memcpy_h2d(tpt_ctx* c, void* dst, const void* src, size_t bytes) {
  ENTER(c);
  TPT_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
  TPT_HIP(hipStreamSynchronize(c->stream));
  return TPT_OK;
}

int tpt_memcpy_d2h(tpt_ctx* c, void* dst, const void* src, size_t bytes) {
  ENTER(c);
  TPT_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
  TPT_HIP(hipStreamSynchronize(c->stream));
  return TPT_OK;
}

int tpt_memset(tpt_ctx* c, void* dst, int value, size_t bytes) {
  ENTER(c);
  TPT_HIP(hipMemsetAsync(dst, value, bytes, c->stream));
  return TPT_OK;
}

int tpt_dequant(tpt_ctx* c, int type, const void* w, float* y, int64_t n) {
  ENTER(c);
  if (!w || !y) return fail(TPT_ERR_INVALID, "dequant: null pointer");
  return launch_dequant(type, w, y, n, c->stream);
}

int tpt_gemv(tpt_ctx* c, int type, const void* w, const float* x, float* y, int K, int N,
             int act_mode) {
  ENTER(c);
  if (!w || !x || !y) return fail(TPT_ERR_INVALID, "gemv: null pointer");
  if (act_mode == TPT_ACT_F32) return launch_gemv_f32(type, (const uint8_t*)w, x, y, K, N, c->stream);
  if (act_mode != TPT_ACT_Q8) return fail(TPT_ERR_INVALID, "gemv: act_mode must be TPT_ACT_Q8 or TPT_ACT_F32");
  GemvArgs a;
  a.w0 = (const uint8_t*)w;
  a.row_stride = row_bytes(type, K);
  a.K = K;
  a.N = N;
  a.x = x;
  a.y = y;
  return launch_gemv_q8(c, type, a, c->stream);
}

int tpt_gemv_rmsnorm(tpt_ctx* c, int type, const void* w, const float* x, const float* norm_w,
                     float eps, float* y, int K, int N) {
  ENTER(c);
  if (!w || !x || !y || !norm_w) return fail(TPT_ERR_INVALID, "gemv_rmsnorm: null pointer");
  GemvArgs a;
  a.w0 = (const uint8_t*)w;
  a.row_stride = row_bytes(type, K);
  a.K = K;
  a.N = N;
  a.x = x;
  a.norm_w = norm_w;
  a.eps = eps;
  a.prologue = PRO_RMSNORM;
  a.y = y;
  return launch_gemv_q8(c, type, a, c->stream);
}

int tpt_rmsnorm(tpt_ctx* c, const float* x, const float* w, float* y, int n, float eps) {
  ENTER(c);
  if (!x || !w || !y) return fail(TPT_ERR_INVALID, "rmsnorm: null pointer");
  return launch_rmsnorm(x, w, y, n, eps, c->stream);
}

int tpt_swiglu(tpt_ctx* c, const float* g, const float* u, float* y, int n) {
  ENTER(c);
  if (!g || !u || !y) return fail(TPT_ERR_INVALID, "swiglu: null pointer");
  return launch_swiglu(g, u, y, n, c->stream);
}

int tpt_rope(tpt_ctx* c, float* x, int n_heads, int hd, int pos, const float* cos_t,
             const float* sin_t) {
  ENTER(c);
  if (!x || !cos_t || !sin_t) return fail(TPT_ERR_INVALID, "rope: null pointer");
  return launch_rope(x, n_heads, hd, pos, cos_t, sin_t, c->stream);
}

namespace {
// Shared set-up of the op-level attention entry points: argument checks and per-call scratch
// (the chunk records of the split-K partition).
struct AttnCall {
  AttnArgs a;
  void* scratch = nullptr;
};
int attn_prepare(tpt_ctx* c, const float* q, const void* k_cache, const void* v_cache,
                 int kv_type, float* o, int nq, int nkv, int hd, int L, int L_stride,
                 int n_chunks, AttnCall* call) {
  if (!q || !k_cache || !v_cache || !o) return fail(TPT_ERR_INVALID, "attention: null pointer");
  if (nkv <= 0 || nq <= 0 || nq % nkv) return fail(TPT_ERR_INVALID, "attention: bad head counts");
  if (L <= 0 || L > L_stride) return fail(TPT_ERR_INVALID, "attention: L must be in [1, L_stride]");
  if (L > attn_max_len()) return fail(TPT_ERR_UNSUPPORTED, "attention: cache longer than the split-K partition supports");
  AttnArgs& a = call->a;
  a.q = q;
  a.kc = k_cache;
  a.vc = v_cache;
  a.kv_type = kv_type;
  a.o = o;
  a.nq = nq;
  a.nkv = nkv;
  a.hd = hd;
  a.L_stride = L_stride;
  a.L_host = L;
  a.n_chunks = n_chunks > 0 ? n_chunks : attn_default_chunks(L, nkv);
  a.chunk_len = attn_chunk_len(L, a.n_chunks);
  const size_t pf = (size_t)attn_part_floats(nq, nkv, hd, a.n_chunks);
  TPT_HIP(hipMallocAsync(&call->scratch, pf * 4, c->stream));
  a.part = (float*)call->scratch;
  return TPT_OK;
}
}  // namespace

int tpt_attn_decode(tpt_ctx* c, const float* q, const void* k_cache, const void* v_cache,
                    int kv_type, float* o, int nq, int nkv, int hd, int L, int L_stride,
                    int n_chunks) {
  ENTER(c);
  AttnCall call;
  int rc = attn_prepare(c, q, k_cache, v_cache, kv_type, o, nq, nkv, hd, L, L_stride, n_chunks, &call);
  if (rc) return rc;
  rc = launch_attn_decode(call.a, c->stream);
  (void)hipFreeAsync(call.scratch, c->stream);
  return rc;
}

int tpt_attn_prefill(tpt_ctx* c, const float* q, const void* k_cache, const void* v_cache,
                     int kv_type, float* o, int nq, int nkv, int hd, int L0, int T, int L_stride,
                     int form) {
  ENTER(c);
  if (T <= 0 || L0 < 0 || form < 0 || form > 2) return fail(TPT_ERR_INVALID, "attn_prefill: bad T, L0 or form");
  if ((long)L0 + T > L_stride) return fail(TPT_ERR_INVALID, "attn_prefill: queries past the cache");
  // the split-K partition is sized for the last query, which sees L0 + T positions
  AttnCall call;
  int rc = attn_prepare(c, q, k_cache, v_cache, kv_type, o, nq, nkv, hd, L0 + T, L_stride, 0, &call);
  if (rc) return rc;
  (void)hipFreeAsync(call.scratch, c->stream);
  call.scratch = nullptr;
  AttnArgs& a = call.a;
  a.L_host = L0 + 1;
  a.nqb = T;
  a.ldq = a.ldo = nq * hd;
  const bool mfma = form == 2 || (form == 0 && attn_causal_mfma_supported(a));
  if (mfma) return launch_attn_causal_mfma(a, c->stream);
  TPT_HIP(hipMallocAsync(&call.scratch, (size_t)T * attn_part_floats(nq, nkv, hd, a.n_chunks) * 4, c->stream));
  a.part = (float*)call.scratch;
  rc = launch_attn_decode(a, c->stream);
  (void)hipFreeAsync(call.scratch, c->stream);
  return rc;
}

int tpt_bench_attn_prefill(tpt_ctx* c, const float* q, const void* k_cache, const void* v_cache,
                           int kv_type, float* o, int nq, int nkv, int hd, int L0, int T,
                           int L_stride, int iters, float* ms_out) {
  ENTER(c);
  if (iters <= 0 || iters > 4096 || !ms_out) return fail(TPT_ERR_INVALID, "bench_attn_prefill: bad arguments");
  if (!q || !k_cache || !v_cache || !o) return fail(TPT_ERR_INVALID, "bench_attn_prefill: null pointer");
  if (T <= 0 || L0 < 0 || (long)L0 + T > L_stride || nkv <= 0 || nq % nkv)
    return fail(TPT_ERR_INVALID, "bench_attn_prefill: bad shape");
  AttnArgs a;
  a.q = q; a.kc = k_cache; a.vc = v_cache; a.kv_type = kv_type; a.o = o;
  a.nq = nq; a.nkv = nkv; a.hd = hd; a.L_stride = L_stride; a.L_host = L0 + 1;
  a.nqb = T; a.ldq = a.ldo = nq * hd;
  if (!attn_causal_mfma_supported(a))
    return fail(TPT_ERR_UNSUPPORTED, "bench_attn_prefill: shape outside the matrix-core kernel");
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = TPT_OK;
  hipError_t e = hipEventCreate(&e0);
  if (e == hipSuccess) e = hipEventCreate(&e1);
  if (e == hipSuccess) e = hipEventRecord(e0, c->stream);
  for (int i = 0; i < iters && rc == TPT_OK && e == hipSuccess; i++) rc = launch_attn_causal_mfma(a, c->stream);
  if (e == hipSuccess) e = hipEventRecord(e1, c->stream);
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  if (e == hipSuccess && rc == TPT_OK) e = hipEventElapsedTime(ms_out, e0, e1);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (rc) return rc;
  if (e != hipSuccess) return hip_fail(e, "bench_attn_prefill", __FILE__, __LINE__);
  return TPT_OK;
}

int tpt_bench_attn(tpt_ctx* c, const float* q, const void* const* k_caches,
                   const void* const* v_caches, int n_caches, int kv_type, float* o, int nq,
                   int nkv, int hd, int L, int L_stride, int n_chunks, int iters, float* ms_out) {
  ENTER(c);
  if (iters <= 0 || iters > 4096 || !ms_out || !k_caches || !v_caches || n_caches <= 0)
    return fail(TPT_ERR_INVALID, "bench_attn: bad arguments");
  for (int i = 0; i < n_caches; i++)
    if (!k_caches[i] || !v_caches[i]) return fail(TPT_ERR_INVALID, "bench_attn: null cache pointer");
  AttnCall call;
  int rc = attn_prepare(c, q, k_caches[0], v_caches[0], kv_type, o, nq, nkv, hd, L, L_stride, n_chunks, &call);
  if (rc) return rc;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  hipError_t e = hipEventCreate(&e0);
  if (e == hipSuccess) e = hipEventCreate(&e1);
  if (e == hipSuccess) e = hipEventRecord(e0, c->stream);
  for (int i = 0; i < iters && rc == TPT_OK && e == hipSuccess; i++) {
    call.a.kc = k_caches[i % n_caches];
    call.a.vc = v_caches[i % n_caches];
    rc = launch_attn_decode(call.a, c->stream);
  }
  if (e == hipSuccess) e = hipEventRecord(e1, c->stream);
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  if (e == hipSuccess && rc == TPT_OK) e = hipEventElapsedTime(ms_out, e0, e1);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  (void)hipFreeAsync(call.scratch, c->stream);
  if (rc) return rc;
  if (e != hipSuccess) return hip_fail(e, "bench_attn", __FILE__, __LINE__);
  return TPT_OK;
}

int tpt_argmax(tpt_ctx* c, const float* logits, int64_t n, uint32_t* out_host) {
  ENTER(c);
  if (!logits || !out_host) return fail(TPT_ERR_INVALID, "argmax: null pointer");
  unsigned long long* slot = nullptr;
  TPT_HIP(hipMallocAsync((void**)&slot, 8, c->stream));
  hipError_t e = hipMemsetAsync(slot, 0, 8, c->stream);
  int rc = e == hipSuccess ? launch_argmax(logits, n, slot, c->stream) : hip_fail(e, "memset", __FILE__, __LINE__);
  unsigned long long key = 0;
  if (rc == TPT_OK) {
    e = hipMemcpyAsync(&key, slot, 8, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) rc = hip_fail(e, "argmax readback", __FILE__, __LINE__);
  }
  (void)hipFreeAsync(slot, c->stream);
  if (rc == TPT_OK) *out_host = (uint32_t)(key & 0xffffffffull);
  return rc;
}

namespace {
// Device scratch for one tpt_gemm / tpt_bench_gemm call: the prepared activation rows.  F16
// weights in TPT_ACT_Q8 mode (candle's f32 product) run two passes: on the fp16 remainder rows
// (lo), then on the fp16 rows with the first pass's output as the residual.
struct GemmCall {
  GemmArgs g;
  const uint16_t* lo = nullptr;
  void* scratch = nullptr;
};
int gemm_run(const GemmCall& call, hipStream_t s, hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr) {
  if (!call.lo) return launch_gemm_timed(call.g, s, ev0, ev1);
  GemmArgs g = call.g;
  g.af = call.lo;
  int rc = launch_gemm_timed(g, s, ev0, nullptr);
  if (rc) return rc;
  g.af = call.g.af;
  g.resid = g.y;
  g.ldr = g.ldy;
  return launch_gemm_timed(g, s, nullptr, ev1);
}
int gemm_prepare(tpt_ctx* c, int type, const void* w, const float* x, float* y, int M, int K,
                 int N, int act_mode, GemmCall* call) {
  const bool kq = type == TPT_TYPE_Q4_K || type == TPT_TYPE_Q5_K || type == TPT_TYPE_Q6_K;
  const bool q80 = type == TPT_TYPE_Q8_0 || type == TPT_TYPE_Q4_0;
  if (!kq && !q80 && type != TPT_TYPE_F16)
    return fail(TPT_ERR_UNSUPPORTED, "gemm: weight type must be Q4_K, Q5_K, Q6_K, Q8_0, Q4_0 or F16");
  if (act_mode != TPT_ACT_Q8 && act_mode != TPT_ACT_F16) return fail(TPT_ERR_INVALID, "gemm: act_mode must be TPT_ACT_Q8 or TPT_ACT_F16");
  if (q80 && act_mode != TPT_ACT_Q8) return fail(TPT_ERR_UNSUPPORTED, "gemm: Q8_0 and Q4_0 weights take TPT_ACT_Q8");
  if (!w || !x || !y || M <= 0 || N <= 0 || K <= 0 || K % 256) return fail(TPT_ERR_INVALID, "gemm: bad arguments");
  GemmArgs& g = call->g;
  g.M = M; g.N = N; g.K = K;
  g.mode = act_mode == TPT_ACT_F16 || type == TPT_TYPE_F16 ? GEMM_F16 : q80 ? GEMM_Q80 : GEMM_Q8K;
  const bool split = type == TPT_TYPE_F16 && act_mode == TPT_ACT_Q8;
  g.wtype = type;
  g.w = (const uint8_t*)w;
  g.w_stride = row_bytes(type, K);
  g.y = y;
  g.ldy = N;
  ActPrepArgs p;
  p.M = M; p.K = K; p.ldx = K; p.x = x; p.mode = g.mode;
  const size_t mk = (size_t)M * K;
  // fp16 rows [M][K], then GEMM_Q8K block scales [M][K/256] and per-16 sums [M][K/16], GEMM_Q80
  // block scales [M][K/32], or (F16 weights, two passes) the fp16 remainder rows [M][K]
  const size_t o_d = (mk * 2 + 255) & ~(size_t)255;
  const size_t nd = g.mode == GEMM_Q80 ? (size_t)M * (K / 32) : (size_t)M * (K / 256);
  const size_t o_s = o_d + ((nd * 4 + 255) & ~(size_t)255);
  const size_t act_bytes = g.mode == GEMM_Q8K ? o_s + (size_t)M * (K / 16) * 2
                           : g.mode == GEMM_Q80 ? o_s
                           : split ? o_d + mk * 2 : mk * 2;
  // split-K workspace when the output tiles cannot fill the device
  const int ns = gemm_splits(M, N, K);
  const size_t o_p = (act_bytes + 255) & ~(size_t)255;
  const size_t pf = ns > 1 ? (size_t)ns * M * N : 0;
  const size_t bytes = o_p + pf * 4;
  TPT_HIP(hipMallocAsync(&call->scratch, bytes, c->stream));
  g.part = pf ? (float*)((uint8_t*)call->scratch + o_p) : nullptr;
  g.part_floats = pf;
  uint8_t* base = (uint8_t*)call->scratch;
  p.af = (uint16_t*)base;
  g.af = p.af;
  if (g.mode == GEMM_Q8K || g.mode == GEMM_Q80) {
    p.ad = (float*)(base + o_d);
    g.ad = p.ad;
  }
  if (g.mode == GEMM_Q8K) {
    p.as16 = (int16_t*)(base + o_s);
    g.as16 = p.as16;
  }
  if (split) {
    p.af2 = (uint16_t*)(base + o_d);
    call->lo = p.af2;
  }
  int rc = launch_act_prep(p, c->stream);
  if (rc) (void)hipFreeAsync(call->scratch, c->stream);
  return rc;
}
}  // namespace

int tpt_gemm(tpt_ctx* c, int type, const void* w, const float* x, float* y, int M, int K, int N,
             int act_mode) {
  ENTER(c);
  GemmCall call;
  int rc = gemm_prepare(c, type, w, x, y, M, K, N, act_mode, &call);
  if (rc) return rc;
  rc = gemm_run(call, c->stream);
  (void)hipFreeAsync(call.scratch, c->stream);
  return rc;
}

int tpt_bench_gemm(tpt_ctx* c, int type, const void* w, const float* x, float* y, int M, int K,
                   int N, int act_mode, int iters, float* ms_out) {
  ENTER(c);
  if (iters <= 0 || iters > 4096 || !ms_out) return fail(TPT_ERR_INVALID, "bench_gemm: bad arguments");
  GemmCall call;
  int rc = gemm_prepare(c, type, w, x, y, M, K, N, act_mode, &call);
  if (rc) return rc;
  std::vector<hipEvent_t> ev((size_t)2 * iters, nullptr);
  hipError_t e = hipSuccess;
  for (auto& v : ev)
    if (e == hipSuccess) e = hipEventCreate(&v);
  for (int i = 0; i < iters && rc == TPT_OK && e == hipSuccess; i++)
    rc = gemm_run(call, c->stream, ev[2 * i], ev[2 * i + 1]);
  if (e == hipSuccess && rc == TPT_OK) e = hipEventSynchronize(ev.back());
  float total = 0.f;
  for (int i = 0; i < iters && e == hipSuccess && rc == TPT_OK; i++) {
    float ms = 0.f;
    e = hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]);
    total += ms;
  }
  for (auto& v : ev)
    if (v) (void)hipEventDestroy(v);
  (void)hipFreeAsync(call.scratch, c->stream);
  if (rc) return rc;
  if (e != hipSuccess) return hip_fail(e, "bench_gemm", __FILE__, __LINE__);
  *ms_out = total;
  return TPT_OK;
}

int tpt_bench_gemv(tpt_ctx* c, int type, const void* const* weights, int n_weights,
                   const float* x, float* y, int K, int N, int iters, float* ms_out) {
  ENTER(c);
  if (!weights || n_weights <= 0 || iters <= 0 || iters > 4096 || !x || !y || !ms_out)
    return fail(TPT_ERR_INVALID, "bench_gemv: bad arguments");
  GemvArgs a;
  a.row_stride = row_bytes(type, K);
  a.K = K;
  a.N = N;
  a.x = x;
  a.y = y;
  // every launch carries its own start/stop events, timestamped by the dispatch packet itself
  // (hipExtLaunchKernelGGL), so the launches stay back to back and the sum of the intervals is
  // the kernels' own time
  std::vector<hipEvent_t> ev((size_t)2 * iters, nullptr);
  hipError_t e = hipSuccess;
  for (auto& v : ev)
    if (e == hipSuccess) e = hipEventCreate(&v);
  int rc = TPT_OK;
  for (int i = 0; i < iters && rc == TPT_OK && e == hipSuccess; i++) {
    a.w0 = (const uint8_t*)weights[i % n_weights];
    rc = launch_gemv_q8(c, type, a, c->stream, ev[2 * i], ev[2 * i + 1]);
  }
  if (e == hipSuccess && rc == TPT_OK) e = hipEventSynchronize(ev.back());
  float total = 0.f;
  for (int i = 0; i < iters && e == hipSuccess && rc == TPT_OK; i++) {
    float ms = 0.f;
    e = hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]);
    total += ms;
  }
  for (auto& v : ev)
    if (v) (void)hipEventDestroy(v);
  if (rc) return rc;
  if (e != hipSuccess) return hip_fail(e, "bench_gemv", __FILE__, __LINE__);
  *ms_out = total;
  return TPT_OK;
}

int tpt_bench_copy(tpt_ctx* c, void* dst, const void* src, size_t bytes, int iters,
                   float* ms_out) {
  ENTER(c);
  if (!dst || !src || iters <= 0 || !ms_out || bytes % 16) return fail(TPT_ERR_INVALID, "bench_copy: bad arguments");
  hipEvent_t e0, e1;
  TPT_HIP(hipEventCreate(&e0));
  TPT_HIP(hipEventCreate(&e1));
  int rc = TPT_OK;
  hipError_t e = hipEventRecord(e0, c->stream);
  for (int i = 0; i < iters && rc == TPT_OK && e == hipSuccess; i++)
    rc = launch_copy(dst, src, bytes, c->stream);
  if (e == hipSuccess) e = hipEventRecord(e1, c->stream);
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  if (e == hipSuccess && rc == TPT_OK) e = hipEventElapsedTime(ms_out, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (rc) return rc;
  if (e != hipSuccess) return hip_fail(e, "bench_copy", __FILE__, __LINE__);
  return TPT_OK;
}

}  // extern "C"
