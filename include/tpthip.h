/*
 * libtpthip -- MI355X (gfx950) engine for tpt-spark's bs=1 Llama decode path.
 *
 * Plain C ABI: every function returns an int status (TPT_OK = 0, negative = error) and the
 * message of the calling thread's last error is available from tpt_last_error().  No torch
 * or HIP types appear in any signature; device buffers are `void*` device addresses.
 *
 * The reference has no C ABI: its GPU engine is Rust + wgpu (src-tauri/src/engine/).  Each
 * entry point below names the reference interface it replaces.  Threading: the reference
 * serialises every engine call behind EngineHandle's tokio Mutex and may enter from a
 * different OS thread each time (src-tauri/src/commands.rs:55,239,535), so every entry point
 * selects its context's device on entry and no object is internally thread-safe.
 */
#ifndef TPTHIP_H
#define TPTHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TPT_OK 0
#define TPT_ERR_INVALID (-1)     /* bad argument / shape */
#define TPT_ERR_HIP (-2)         /* HIP runtime error */
#define TPT_ERR_IO (-3)          /* file open/mmap/read */
#define TPT_ERR_FORMAT (-4)      /* malformed GGUF, tensor past EOF */
#define TPT_ERR_UNSUPPORTED (-5) /* architecture / dtype not on this path */
#define TPT_ERR_CANCELLED (-6)   /* the token callback asked to stop */
#define TPT_ERR_STATE (-7)       /* no model loaded, context exhausted, ... */
#define TPT_ERR_OOM (-8)

/* ggml tensor types the path reads (values are ggml's GGML_TYPE_* numbers) */
#define TPT_TYPE_F32 0
#define TPT_TYPE_F16 1
#define TPT_TYPE_Q4_0 2
#define TPT_TYPE_Q8_0 8
#define TPT_TYPE_Q4_K 12
#define TPT_TYPE_Q5_K 13
#define TPT_TYPE_Q6_K 14

/* activation handling of a GEMV.  TPT_ACT_Q8: the fp32 input is quantized the way candle's
 * QMatMul does on the CPU (Q8_K per 256 for k-quant weights, Q8_0 per 32 for Q8_0 and Q4_0)
 * and dotted in integer arithmetic -- the parity path.  TPT_ACT_F32: dequantized weights
 * times fp32 activations, fp32 accumulate. */
#define TPT_ACT_Q8 0
#define TPT_ACT_F32 1
#define TPT_ACT_F16 2

const char* tpt_last_error(void);
int tpt_version(void);

/* ------------------------------------------------------------------ context + memory */
/* Replaces GpuContext::try_init (src-tauri/src/engine/wgpu_context.rs:22-97): one device and
 * one HIP stream, default priority. */
typedef struct tpt_ctx tpt_ctx;
int tpt_ctx_create(int device, tpt_ctx** out);
int tpt_ctx_destroy(tpt_ctx* ctx);
int tpt_ctx_synchronize(tpt_ctx* ctx);
/* number of compute units and the device name (for reports) */
int tpt_ctx_device_info(tpt_ctx* ctx, int* n_cu, char* name, int name_len);

/* Device buffers for callers that hold no other GPU allocator (tests, bench). Replaces
 * GpuContext::create_storage_buffer (wgpu_context.rs:100-107) and readback_f32
 * (wgpu_ops.rs:167-179). */
int tpt_malloc(tpt_ctx* ctx, size_t bytes, void** dptr);
int tpt_free(tpt_ctx* ctx, void* dptr);
int tpt_memcpy_h2d(tpt_ctx* ctx, void* dst, const void* src, size_t bytes);
int tpt_memcpy_d2h(tpt_ctx* ctx, void* dst, const void* src, size_t bytes);
int tpt_memset(tpt_ctx* ctx, void* dst, int value, size_t bytes);

/* ------------------------------------------------------------------ op level */
/* Bit-exact dequantization of n elements to fp32 (Q4_K, Q5_K, Q6_K, Q8_0, Q4_0, F16, F32).
 * Replaces the dequant_* WGSL shaders (src-tauri/src/engine/shaders/dequant_q4k.wgsl:74-115,
 * dequant_q5k.wgsl:78-104, dequant_q6k.wgsl:58-92, dequant_q8.wgsl:51-73) as dispatched by
 * append_dequant (wgpu_engine.rs:551-570), with ggml's Q4_K and Q5_K element orders (the
 * WGSL ones are not ggml's). */
int tpt_dequant(tpt_ctx* ctx, int type, const void* w, float* y, int64_t n);

/* y[N] = W[N,K] . x[K] with W in GGUF block layout, rows contiguous.  Replaces
 * dequant_and_gemm (wgpu_engine.rs:581-605) + gemm.wgsl:28-70 at M=1, and candle's
 * QMatMul::forward -> k_quants::matmul on the CPU (the parity target).  type Q4_K, Q5_K, Q6_K,
 * Q8_0, Q4_0 or F16 (dequant_f16.wgsl, wgpu_engine.rs:543).  act_mode TPT_ACT_Q8: candle's
 * arithmetic for the type (x quantized to Q8_K / Q8_0 for the quantized types; for F16, which
 * candle dequantizes and multiplies in f32, x stays f32, K <= 15360); TPT_ACT_F32: the
 * dequantized weights times f32 x, for every type. */
int tpt_gemv(tpt_ctx* ctx, int type, const void* w, const float* x, float* y, int K, int N,
             int act_mode);

/* Prefill GEMM on MFMA: Y[M,N] = X[M,K] . W[N,K]^T with W in Q4_K, Q5_K, Q6_K, Q8_0, Q4_0 or
 * F16 rows (type), X fp32 rows (a real Q4_K_M file holds Q6_K attn_v / ffn_down matrices in
 * some layers).  act_mode TPT_ACT_Q8 is candle's prefill arithmetic for the type: every X row
 * quantized to Q8_K (k-quants) or Q8_0 (Q8_0, Q4_0 weights) as candle's QMatMul does, with
 * integer-exact products; for F16 weights, which candle multiplies in f32, X split into fp16
 * rounding plus remainder (two passes, X carried to 2^-22 relative; |X| < 65504).
 * TPT_ACT_F16 (k-quants and F16): X and the dequantized W in fp16 on the matrix cores, fp32
 * accumulate.  Replaces the per-position prefill of gpu_infer (wgpu_engine.rs:254-261) and
 * candle's batched QMatMul (candle_engine.rs:272-273). */
int tpt_gemm(tpt_ctx* ctx, int type, const void* w, const float* x, float* y, int M, int K, int N,
             int act_mode);

/* y = rmsnorm(x) . W (fused norm prologue; the residual stream is normalised in-kernel).
 * Replaces rms_norm.wgsl:22-65 followed by dequant_and_gemm (wgpu_engine.rs:377-416). */
int tpt_gemv_rmsnorm(tpt_ctx* ctx, int type, const void* w, const float* x,
                     const float* norm_w, float eps, float* y, int K, int N);

/* y = rmsnorm(x) with weight w.  Replaces rms_norm.wgsl:22-65 (n_rows = 1). */
int tpt_rmsnorm(tpt_ctx* ctx, const float* x, const float* w, float* y, int n, float eps);

/* y[i] = silu(g[i]) * up[i] with silu(t) = t / (1 + exp(-t)) in f32 (candle's silu; the decode
 * and prefill paths fuse the same device function into their GEMV / activation kernels).
 * Replaces silu.wgsl:20-29 (in place there; y may alias g here). */
int tpt_swiglu(tpt_ctx* ctx, const float* g, const float* up, float* y, int n);

/* In-place interleaved RoPE of n_heads heads of hd at position pos, using host-built f32
 * tables cos_t/sin_t [>= pos+1][hd/2] in device memory.  Replaces rope.wgsl:23-51
 * (dispatch_rope, wgpu_engine.rs:625-640) with candle's rope_i pairing. */
int tpt_rope(tpt_ctx* ctx, float* x, int n_heads, int hd, int pos, const float* cos_t,
             const float* sin_t);

/* Decode attention for one query position: o[Nq,hd] = softmax(q K^T / sqrt(hd)) V over the
 * first L positions of a cache laid out [Nkv][L_stride][hd] with elements of kv_type
 * (TPT_TYPE_F16 or TPT_TYPE_F32; GQA: head h reads kv head h / (Nq/Nkv)).  Replaces
 * attention.wgsl:31-170 (dispatch_attention, wgpu_engine.rs:666-726).  n_chunks = 0 picks the
 * split-K partition count (at most 256 chunks of at most 1024 positions). */
int tpt_attn_decode(tpt_ctx* ctx, const float* q, const void* k_cache, const void* v_cache,
                    int kv_type, float* o, int nq, int nkv, int hd, int L, int L_stride,
                    int n_chunks);

/* tpt_attn_decode without any device allocation.  No counterpart in the reference: it is for
 * callers that cannot allocate (code under HIP graph capture, serving loops and harnesses that
 * must not call hipMalloc).  Same arguments, kernels and results as tpt_attn_decode; the split-K
 * chunk records live in a fixed 4 MiB device array that each GPU holds until the process ends
 * (TPT_ERR_UNSUPPORTED when nq * n_chunks * (hd + 2) * 4 bytes exceed it).  Calls that overlap on
 * one GPU share that array and race. */
int tpt_attn_decode_noalloc(tpt_ctx* ctx, const float* q, const void* k_cache,
                            const void* v_cache, int kv_type, float* o, int nq, int nkv, int hd,
                            int L, int L_stride, int n_chunks);

/* Causal attention of a prompt batch: T query rows q [T][Nq*hd], row t at position L0 + t seeing
 * cache positions [0, L0 + t] (the cache must hold positions < L0 + T); o [T][Nq*hd].  The
 * attention of candle's batched prompt forward (candle_engine.rs:272-273: the whole prompt in one
 * quantized_llama forward under its causal mask); the reference's wgpu engine runs
 * attention.wgsl:31-170 once per position instead.  form 0: the model's choice (matrix cores
 * where supported: fp16 cache, hd 64 or 128, Nq/Nkv 1, 2, 4 or 8; else per-query split-K),
 * 1: per-query split-K, 2: matrix cores (TPT_ERR_UNSUPPORTED outside their shapes). */
int tpt_attn_prefill(tpt_ctx* ctx, const float* q, const void* k_cache, const void* v_cache,
                     int kv_type, float* o, int nq, int nkv, int hd, int L0, int T, int L_stride,
                     int form);

/* Greedy token of a logits vector: the last index among equal maxima under f32 total order
 * (candle LogitsProcessor::sample_argmax, used by sample_token wgpu_engine.rs:868-878). */
int tpt_argmax(tpt_ctx* ctx, const float* logits, int64_t n, uint32_t* out_host);

/* ------------------------------------------------------------------ measurement */
/* No reference counterpart (the reference publishes no kernel timings): these time kernels
 * with HIP events recorded on the context's own stream. */
/* iters (<= 4096) back-to-back launches of tpt_gemv, launch i reading weights[i % n_weights]
 * (distinct copies defeat the 256 MB Infinity Cache); *ms_out = the sum over launches of the
 * interval between the start and stop events each dispatch timestamps itself. */
int tpt_bench_gemv(tpt_ctx* ctx, int type, const void* const* weights, int n_weights,
                   const float* x, float* y, int K, int N, int iters, float* ms_out);
/* iters launches of the GEMM kernel of tpt_gemm (activation rows prepared once, before the
 * timed launches); *ms_out = the sum of the dispatch-stamped event intervals. */
int tpt_bench_gemm(tpt_ctx* ctx, int type, const void* w, const float* x, float* y, int M, int K,
                   int N, int act_mode, int iters, float* ms_out);
/* iters back-to-back launches of tpt_attn_decode, launch i reading the caches
 * k_caches[i % n_caches] / v_caches[i % n_caches] (distinct copies defeat the Infinity Cache);
 * *ms_out = the event time over all launches (events recorded on the context's stream). */
int tpt_bench_attn(tpt_ctx* ctx, const float* q, const void* const* k_caches,
                   const void* const* v_caches, int n_caches, int kv_type, float* o, int nq,
                   int nkv, int hd, int L, int L_stride, int n_chunks, int iters, float* ms_out);
/* iters back-to-back launches of tpt_attn_prefill's matrix-core form over the same caches
 * (T queries after L0 cached positions); *ms_out = the event time over all launches. */
int tpt_bench_attn_prefill(tpt_ctx* ctx, const float* q, const void* k_cache, const void* v_cache,
                           int kv_type, float* o, int nq, int nkv, int hd, int L0, int T,
                           int L_stride, int iters, float* ms_out);
/* iters launches of a plain vector copy of `bytes` (HBM calibration for PMC counters) */
int tpt_bench_copy(tpt_ctx* ctx, void* dst, const void* src, size_t bytes, int iters,
                   float* ms_out);

/* ------------------------------------------------------------------ model level */
/* Replaces load_gguf_to_vram + extract_meta (src-tauri/src/engine/wgpu_loader.rs:87-201,
 * 305-406), KvCache (wgpu_kvcache.rs:15-79) and run_forward_pass (wgpu_engine.rs:339-490). */
typedef struct tpt_model tpt_model;

typedef struct {
  char architecture[32];
  int n_layers, n_heads, n_kv_heads, head_dim, embed, ffn, vocab;
  int context_length; /* from GGUF metadata */
  int max_ctx;        /* KV capacity actually allocated */
  int kv_type;        /* KV cache element type: TPT_TYPE_F16 or TPT_TYPE_F32 */
  float rms_eps, rope_base, rope_scale;
  uint64_t weight_bytes; /* quantized bytes resident in HBM */
  uint64_t decode_bytes_per_token; /* weight bytes one decode step streams */
  int type_q, type_k, type_v, type_o, type_gate, type_up, type_down, type_embd, type_out;
} tpt_model_desc;

/* progress(user, done, total) after each uploaded tensor (LlmEngine::load's on_progress,
 * src-tauri/src/engine/mod.rs:63-70) */
typedef void (*tpt_progress_fn)(void* user, uint32_t done, uint32_t total);

/* mmap + validate + upload the k-quant blocks unchanged.  max_ctx <= 0 uses the GGUF
 * context_length.  kv_type TPT_TYPE_F16 (half the KV bytes) or TPT_TYPE_F32 (the cache candle
 * keeps: the CandleEngine-exact mode). */
int tpt_model_load(tpt_ctx* ctx, const char* gguf_path, int max_ctx, int kv_type,
                   tpt_progress_fn progress, void* user, tpt_model** out);
/* Host only (no device, no context): parse and validate a GGUF as tpt_model_load would --
 * metadata keys and defaults, architecture, every tensor the forward pass reads present with the
 * shape, type and byte size the kernels assume, no tensor past the end of the file -- and fill
 * *out (max_ctx and kv_type left 0).  Replaces extract_meta (wgpu_loader.rs:305-406) and the
 * validation half of load_gguf_to_vram (wgpu_loader.rs:105-135). */
int tpt_model_inspect(const char* gguf_path, tpt_model_desc* out);
int tpt_model_describe(const tpt_model* m, tpt_model_desc* out);
int tpt_model_destroy(tpt_model* m);

/* Run positions pos0..pos0+n-1 for ids[0..n) (the KV cache gains those positions).  Writes
 * the greedy token after the last position to *next_out and, if logits_out is non-NULL, the
 * last position's logits [vocab] (host memory). */
int tpt_model_prefill(tpt_model* m, const uint32_t* ids, int n, int pos0, uint32_t* next_out,
                      float* logits_out);
/* One decode step (token tok at position pos); same outputs as prefill. */
int tpt_model_decode_step(tpt_model* m, uint32_t tok, int pos, uint32_t* next_out,
                          float* logits_out);
/* Greedy decode of n_steps tokens starting with token first at position pos0, replaying one
 * captured HIP graph per step with the argmax kept on the device.  tokens_out[i] is the
 * greedy token produced by step i.  stop_token >= 0 ends the run after that token is produced
 * (steps already in flight are discarded).  Returns the number of tokens written. */
int tpt_model_decode_greedy(tpt_model* m, uint32_t first, int pos0, int n_steps,
                            int64_t stop_token, uint32_t* tokens_out);
/* Copy the current residual stream (fp32 [embed]) to host memory (parity tests). */
int tpt_model_hidden(tpt_model* m, float* out_host);
/* How a decode step runs on the device.  Replaces the per-token loop of
 * WgpuEngine::run_forward_pass (src-tauri/src/engine/wgpu_engine.rs:339-490), which submits
 * each op of each layer separately.  TPT_DECODE_KERNELS (the only form): one launch per fused
 * op, captured into a HIP graph per step.  TPT_DECODE_PERSISTENT (one launch for every layer,
 * grid barriers between the phases) was measured slower and removed: setting it returns
 * TPT_ERR_UNSUPPORTED; the value stays reserved. */
#define TPT_DECODE_KERNELS 0
#define TPT_DECODE_PERSISTENT 1
int tpt_model_set_decode_path(tpt_model* m, int path);
int tpt_model_get_decode_path(const tpt_model* m, int* path);
/* Layer-range forward for parity checks (no counterpart in the reference): runs decoder layers
 * [l0, l1) on n caller-given residual rows x_in (host fp32 [n][embed]) at positions
 * pos0 .. pos0+n-1 and writes the resulting rows to x_out (host, same shape).  The layers' K/V
 * rows at those positions are written as a forward pass writes them.  path 0: the batched
 * prefill kernels (MFMA GEMMs; needs every layer matrix Q4_K, else TPT_ERR_UNSUPPORTED);
 * path 1: the decode-step kernels, one position after another. */
int tpt_model_run_layers(tpt_model* m, const float* x_in, int n, int pos0, int l0, int l1, int path,
                         float* x_out);
/* Copy one layer's K and V cache (each [n_kv_heads][max_ctx][head_dim] of the model's kv_type)
 * to host memory, for cache-layout parity checks (no counterpart in the reference). */
int tpt_model_kv_read(tpt_model* m, int layer, void* k_host, void* v_host);

/* ------------------------------------------------------------------ engine (LlmEngine) */
/* Mirrors `trait LlmEngine` (src-tauri/src/engine/mod.rs:62-82) for an engine-hip backend.
 * Tokenization stays on the caller's side (the tokenizers crate): prompts and tokens are
 * ids.  The callback returns 0 to continue; non-zero cancels (the Rust side maps its
 * on_token Err to non-zero), after which one done=1 event is still delivered and
 * tpt_engine_infer returns TPT_ERR_CANCELLED (wgpu_engine.rs:297-300). */
typedef struct tpt_engine tpt_engine;

typedef struct {
  char name[256];
  char path[1024];
  uint64_t size_bytes;
  char backend[64];
} tpt_model_info; /* ModelInfo, mod.rs:85-92 */

typedef struct {
  uint32_t max_tokens; /* InferenceParams, mod.rs:35-59 */
  float temperature;
  float top_p;
  float repeat_penalty;
  int64_t eos_token_id; /* find_eos_token (candle_engine.rs:76-83) result; <0 = none */
  uint64_t seed;        /* sampling seed (LogitsProcessor::new(42, ..) in the reference) */
} tpt_infer_params;

typedef struct {
  uint32_t prompt_tokens, cached_prefix, generated;
  double prefill_ms, decode_ms, ttft_ms;
} tpt_infer_stats;

typedef int (*tpt_token_fn)(void* user, uint32_t token_id, int done);

int tpt_engine_create(int device, tpt_engine** out);
/* KV cache element type used by the next tpt_engine_load (default TPT_TYPE_F16). */
int tpt_engine_set_kv_type(tpt_engine* e, int kv_type);
int tpt_engine_destroy(tpt_engine* e);
int tpt_engine_load(tpt_engine* e, const char* model_path, tpt_progress_fn progress, void* user,
                    tpt_model_info* info_out);
int tpt_engine_unload(tpt_engine* e);
int tpt_engine_is_loaded(const tpt_engine* e);
int tpt_engine_model_info(const tpt_engine* e, tpt_model_info* info_out);
int tpt_engine_infer(tpt_engine* e, const tpt_infer_params* params, const uint32_t* prompt,
                     size_t n_prompt, tpt_token_fn on_token, void* user, tpt_infer_stats* stats);
/* KvCache::common_prefix_len (wgpu_kvcache.rs:63-69) as a free function: the number of
 * leading ids a and b share.  Pure host code (no device needed). */
size_t tpt_common_prefix_len(const uint32_t* a, size_t na, const uint32_t* b, size_t nb);
/* KvCache::common_prefix_len (wgpu_kvcache.rs:63-69) against the engine's cached tokens */
int tpt_engine_cached_prefix(const tpt_engine* e, const uint32_t* tokens, size_t n,
                             size_t* out);
/* KvCache::reset (wgpu_kvcache.rs:55-58) */
int tpt_engine_reset_cache(tpt_engine* e);

#ifdef __cplusplus
}
#endif
#endif /* TPTHIP_H */
