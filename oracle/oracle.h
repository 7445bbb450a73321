/*
 * CPU oracle for the bs=1 Q4_K_M Llama decode path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker (or, for cpu_baseline, as the timed CPU restatement).
 * The product library never links or calls it.
 *
 * This is a plain-C restatement of the arithmetic the reference's CandleEngine runs
 * (src-tauri/src/engine/candle_engine.rs:205-334).  That arithmetic lives in the crates
 * candle-core / candle-nn / candle-transformers 0.8.4 (pinned at src-tauri/Cargo.lock:316-370),
 * which are NOT vendored under the reference.  Each function names the candle routine it
 * restates; where candle has several code paths the generic one is followed, because the
 * reference builds without `target-feature=avx` (no RUSTFLAGS in src-tauri/).
 *
 * Pinning status (what checks each function; see tests/test_oracle_golden.py):
 *   dequant q4k/q6k/q8_0      hand-built known-answer blocks + closed forms         PINNED
 *   dequant q5k/q4_0          hand-built known-answer blocks (every 5th-bit lane,
 *                             both nibbles, the -8 offset)                          PINNED
 *   quantize_q8k / q8_0       hand-computed known answers (tie rule, half-away)     PINNED
 *   vec_dot q4k/q5k/q6k/q8_0/q4_0  fp64 identity over dequantized operands          PINNED
 *   matmul F16 (dequantize, f32 matmul)  exact widening (every f16 class) + fp64 dot    PINNED
 *   rmsnorm / silu / rope     closed forms (constant vector, 0, pos=0, pair norm)   PINNED
 *   attention                 single position (o=v), uniform scores (o=mean V)      PINNED
 *   argmax                    crafted ties (last index wins), NaN order             PINNED
 *   llama forward             closed forms with zeroed branches (residual rows =
 *                             embedding; x + Wo.repeat_kv(Wv.n(x)); x + W2.(silu(W1.n').W3.n');
 *                             logits from the last position), prefix reuse == full
 *                             recompute, batched == stepwise (tests/test_oracle_model.py)  PINNED
 *   candle's exact f32 summation order (gemm crate, rayon chunks)                   parity unpinned
 */
#ifndef TPT_ORACLE_H
#define TPT_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14, ORC_Q8_K = 15 };

#define ORC_QK_K 256
#define ORC_QK8_0 32

#pragma pack(push, 1)
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; } orc_blk_q4k;      /* 144 B */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } orc_blk_q6k; /* 210 B */
typedef struct { uint16_t d; int8_t qs[32]; } orc_blk_q8_0;                                  /*  34 B */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; } orc_blk_q5k; /* 176 B */
typedef struct { uint16_t d; uint8_t qs[16]; } orc_blk_q4_0;                                  /*  18 B */
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } orc_blk_q8k;                 /* 292 B */
#pragma pack(pop)

float orc_fp16_to_f32(uint16_t h);
uint16_t orc_f32_to_fp16(float f); /* round-to-nearest-even, as half::f16::from_f32 */
size_t orc_type_size(int type);     /* bytes per block */
int orc_block_size(int type);       /* elements per block */

/* dequantize n elements (n % block == 0) */
int orc_dequant(int type, const void* src, float* dst, int64_t n);

/* activation quantization (candle BlockQ8K::from_float / BlockQ8_0::from_float) */
int orc_quantize_q8k(const float* x, int64_t k, orc_blk_q8k* out);
int orc_quantize_q8_0(const float* x, int64_t k, orc_blk_q8_0* out);

/* one output element: candle GgmlType::vec_dot_unopt for the weight type */
float orc_vec_dot(int type, int64_t k, const void* w_row, const void* act_q);

/* candle k_quants::matmul: dst[M,N] = lhs[M,K] . W[N,K]^T with per-row activation quant;
 * F16 / F32 weights: candle's dequantize-then-f32-matmul (no activation quant).
 * nthreads <= 0 uses all cores. */
int orc_matmul(int type, int64_t m, int64_t k, int64_t n, const float* lhs, const void* w,
               float* dst, int nthreads);

/* fp64 reference GEMV over dequantized weights: y[n] = sum_k W[n,k]*x[k] */
int orc_gemv_f64(int type, int64_t k, int64_t n, const void* w, const double* x, double* y);

/* candle_nn::ops::rms_norm (f32): y = x / sqrt(sum(x^2)/n + eps) * w */
void orc_rmsnorm(const float* x, const float* w, int64_t n, float eps, float* y);
/* candle_nn::ops::silu: v / (1 + exp(-v)) */
float orc_silu(float v);
/* quantized_llama::precomput_freqs_cis: cos/sin tables [n_pos][rope_dim/2] */
void orc_rope_tables(int rope_dim, float freq_base, int n_pos, float* cos_t, float* sin_t);
/* candle_nn::rotary_emb::rope_i for one position over n_heads heads of hd (in place) */
void orc_rope_i(float* x, int n_heads, int hd, const float* cos_row, const float* sin_row);
/* decode attention for one query position over L cached positions (f32 cache, layout
 * [Nkv][L_stride][hd]); q [Nq][hd] -> o [Nq][hd].  candle: repeat_kv + matmul + softmax + matmul,
 * the products as fused multiply-adds (the gemm crate on an FMA host) */
void orc_attention(const float* q, const float* kc, const float* vc, int nq, int nkv, int hd,
                   int L, int L_stride, float* o);
/* candle LogitsProcessor::sample_argmax: max_by(total_cmp), last index wins on ties */
uint32_t orc_argmax(const float* logits, int64_t n);
/* candle_engine.rs:87-101 apply_repeat_penalty (applied once per occurrence in seen) */
void orc_repeat_penalty(float* logits, int64_t n, const uint32_t* seen, int64_t n_seen, float penalty);

/* ---- GGUF + Llama model (quantized_llama::ModelWeights restated) ---- */
typedef struct orc_model orc_model;
typedef struct {
  int n_layers, n_heads, n_kv_heads, head_dim, embed, ffn, vocab, rope_dim, ctx_len;
  float eps, rope_base;
} orc_model_cfg;

orc_model* orc_model_open(const char* gguf_path, char* err, int errlen);
void orc_model_close(orc_model* m);
void orc_model_get_cfg(const orc_model* m, orc_model_cfg* cfg);
/* kv_f16: 1 rounds cached K/V to fp16 (mirrors the GPU cache), 0 keeps f32 like candle */
/* The attention dot products as fused multiply-adds (on, the default: candle's gemm crate on
 * an FMA host, which is what every x86-64-v3 CPU is) or separate multiply and add (off: the
 * gemm crate on a host without FMA).  Both are candle's results on some CPU; the spread between
 * them bounds how closely any other summation order can be expected to track candle on an
 * ill-conditioned model. */
int orc_model_set_attn_fma(orc_model* m, int on);
int orc_model_reset(orc_model* m, int max_pos, int kv_f16);
/* Batched forward of n tokens at positions pos0..pos0+n-1 (causal); writes last-position
 * logits [vocab].  Mirrors ModelWeights::forward(&[1,n], pos0). nthreads as orc_matmul. */
int orc_model_forward(orc_model* m, const uint32_t* tokens, int n, int pos0, float* logits,
                      int nthreads);
/* read back hidden state after the last forward (final residual stream, pre-norm) */
/* forward that also records the residual rows entering each layer and leaving the last into
 * trace ([n_layers + 1][n][embed] floats) */
int orc_model_forward_trace(orc_model* m, const uint32_t* tokens, int n, int pos0, float* logits,
                            int nthreads, float* trace);
/* Decoder layers [l0, l1) on caller-given residual rows x_in ([n][embed]) at positions
 * pos0..pos0+n-1 (writing those layers' K/V rows); result rows to x_out. */
int orc_model_run_layers(orc_model* m, const float* x_in, int n, int pos0, int l0, int l1, float* x_out,
                         int nthreads);
/* Summation-order variant of the k-quant dot products (off: candle's generic vec_dot order;
 * on: integer lanes reduced inside each super-block, one f32 term per block).  A test
 * instrument: the same integers with another f32 rounding, to measure how far a model's
 * outputs move under a change of summation order alone. */
void orc_set_dot_block_order(int on);
/* test instrument: RMSNorm's sum of squares in a 16-run + pairwise-tree order (off: candle's) */
void orc_set_rms_order(int on);
/* copy of one layer's K and V cache, each [n_kv_heads][max_pos][head_dim] f32 */
int orc_model_kv(const orc_model* m, int layer, float* k_out, float* v_out);
int orc_model_last_hidden(const orc_model* m, float* out);
/* benchmark aid: K/V of positions [0, n_pos) filled with seeded synthetic values (not a model's),
 * so decode from n_pos reads as many cached positions as after a prompt of that length */
int orc_model_prime_cache(orc_model* m, int n_pos, uint64_t seed);

/* raw tensor lookup for tests: returns pointer into the mmapped file or NULL */
const void* orc_model_tensor(const orc_model* m, const char* name, int* type, int64_t* ne0,
                             int64_t* ne1);

#ifdef __cplusplus
}
#endif
#endif
