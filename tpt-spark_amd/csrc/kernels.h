// Kernel launch interfaces shared by the C ABI, the model and the tests' entry points.
#pragma once
#include "tpt_common.h"

namespace tpt {

enum GemvPrologue { PRO_PLAIN = 0, PRO_RMSNORM = 1 };
enum GemvEpilogue {
  EPI_STORE = 0,     // y[r] = acc
  EPI_RESID = 1,     // y[r] = acc + resid[r]   (resid may alias y)
  EPI_ROPE_QKV = 2,  // rows [0,qd) -> q (RoPE), [qd,qd+kd) -> k cache (RoPE, fp16), rest -> v cache
  EPI_SWIGLU = 3,    // two matrices: y[r] = silu(acc0) * acc1
  EPI_ARGMAX = 4,    // y[r] = acc (if y) + device argmax into amax slot
};

// Decode-step state kept in device memory so one captured graph serves every step.
struct StepState {
  int pos;             // position processed by the current step
  int next_pos;        // position of the next step
  int parity;          // amax slot written by the current step's LM head
  int use_override;    // 1: the next step's token is tok_override
  uint32_t tok_override;
  int prompt_len;      // positions < prompt_len take their token from the prompt buffer
  int pad[2];
  unsigned long long amax[2];  // (order_key(logit) << 32) | index, max-reduced
};

struct GemvArgs {
  const uint8_t* w0 = nullptr;
  const uint8_t* w1 = nullptr;  // second matrix (EPI_SWIGLU)
  size_t row_stride = 0;        // bytes per weight row
  int K = 0, N = 0;             // N = rows of this launch
  int row0 = 0;                 // logical row index of this launch's row 0 (EPI_ROPE_QKV)
  const float* x = nullptr;
  const float* norm_w = nullptr;
  float eps = 0.f;
  int prologue = PRO_PLAIN, epilogue = EPI_STORE;
  float* y = nullptr;
  const float* resid = nullptr;
  // EPI_ROPE_QKV
  int qd = 0, kd = 0, hd = 0, max_ctx = 0;
  const float* rope_cos = nullptr;
  const float* rope_sin = nullptr;
  void* kcache = nullptr;        // [nkv][max_ctx][hd] of kv_type
  void* vcache = nullptr;
  int kv_type = TPT_TYPE_F16;    // TPT_TYPE_F16 or TPT_TYPE_F32
  const StepState* state = nullptr;  // position/parity source (nullptr: pos_host / slot 0)
  int pos_host = 0;
  // EPI_ARGMAX
  unsigned long long* amax = nullptr;  // slot array; slot = state ? amax[state->parity] : amax[0]
  // EPI_RESID: ssq_out[blockIdx.x] = the sum of squares of the rows the workgroup stores, so the
  // next RMSNorm prologue can take sum(x^2) from these partials
  float* ssq_out = nullptr;
  // PRO_RMSNORM: sum(x^2) given as n_ssq (<= kSsqMax) partial sums; every wave adds them itself,
  // so the prologue needs no workgroup reduction.  nullptr: the workgroup reduces x.
  const float* ssq_in = nullptr;
  int n_ssq = 0;
};
constexpr int kSsqMax = 256;

// Chooses the lane layout for K and launches.  wtype in {Q4_K, Q5_K, Q6_K, Q8_0, Q4_0, F16}.  ev0/ev1, when
// given, are timestamped by the dispatch itself (hipExtLaunchKernelGGL) around the kernel.
int launch_gemv_q8(const tpt_ctx* ctx, int wtype, const GemvArgs& a, hipStream_t s,
                   hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr);
// The workgroup count launch_gemv_q8 would use for this type and shape (0 if it would fail).
int gemv_grid(const tpt_ctx* ctx, int wtype, const GemvArgs& a);
int launch_gemv_f32(int wtype, const uint8_t* w, const float* x, float* y, int K, int N,
                    hipStream_t s);

// ---- prefill GEMM (k_gemm.hip): Y[M,N] = X[M,K] . W[N,K]^T, W in Q4_K, Q5_K, Q6_K, Q8_0, Q4_0
// or F16 rows.  Modes: GEMM_Q8K (k-quant weights, Q8_K activation rows), GEMM_Q80 (Q8_0 / Q4_0
// weights, Q8_0 activation rows), GEMM_F16 (fp16 activation rows; k-quants dequantized to fp16,
// F16 weights as stored).
enum GemmMode { GEMM_Q8K = 0, GEMM_F16 = 1, GEMM_Q80 = 2 };
struct GemmArgs {
  int M = 0, N = 0, K = 0, mode = GEMM_Q8K;
  int wtype = TPT_TYPE_Q4_K;         // weight rows: Q4_K, Q5_K, Q6_K (GEMM_Q8K / GEMM_F16), Q8_0,
                                     // Q4_0 (GEMM_Q80), F16 (GEMM_F16)
  const uint8_t* w = nullptr;
  size_t w_stride = 0;               // bytes per weight row
  const uint16_t* af = nullptr;      // [M][K] fp16 bits (GEMM_Q8K / GEMM_Q80: the int8 values, exact)
  const float* ad = nullptr;         // GEMM_Q8K: [M][K/256] block scales; GEMM_Q80: [M][K/32]
  const int16_t* as16 = nullptr;     // GEMM_Q8K: [M][K/16] per-16 sums
  float* y = nullptr;
  int ldy = 0;
  const float* resid = nullptr;      // optional: y = X.W^T + resid
  int ldr = 0;
  // optional split-K workspace (f32): with at least gemm_splits(M, N, K) * M * N floats a
  // launch whose output tiles cannot fill the device splits K and sums the splits in order
  float* part = nullptr;
  size_t part_floats = 0;
};
int gemm_splits(int M, int N, int K);
int launch_gemm(const GemmArgs& g, hipStream_t s);
// the same launch with dispatch-stamped start/stop events (hipExtLaunchKernelGGL)
int launch_gemm_timed(const GemmArgs& g, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1);

// Activation rows for the prefill GEMM: optional RMSNorm (w, eps) or SwiGLU (silu(x) * x2),
// then Q8_K quantization (GEMM_Q8K: the int8 values as fp16 in af, with ad / as16), Q8_0
// quantization (GEMM_Q80: af, ad per 32) or fp16 conversion (GEMM_F16: af; with af2 also the
// remainder x - af rounded to fp16, so that af + af2 carries x to 2^-22 relative).
// x rows of K floats, stride ldx.
struct ActPrepArgs {
  int M = 0, K = 0, ldx = 0;
  const float* x = nullptr;
  const float* x2 = nullptr;         // SwiGLU: up values (same layout as x = gate)
  const float* norm_w = nullptr;     // RMSNorm weights (nullptr: no norm)
  float eps = 0.f;
  int mode = GEMM_Q8K;
  float* ad = nullptr;
  int16_t* as16 = nullptr;
  uint16_t* af = nullptr;
  uint16_t* af2 = nullptr;           // GEMM_F16: optional fp16 remainder rows
};
int launch_act_prep(const ActPrepArgs& a, hipStream_t s);

int launch_dequant(int type, const void* w, float* y, int64_t n, hipStream_t s);
int launch_rmsnorm(const float* x, const float* w, float* y, int n, float eps, hipStream_t s);
int launch_swiglu(const float* g, const float* u, float* y, int n, hipStream_t s);
int launch_rope(float* x, int n_heads, int hd, int pos, const float* c, const float* sn,
                hipStream_t s);
int launch_copy(void* dst, const void* src, size_t bytes, hipStream_t s);
int launch_argmax(const float* logits, int64_t n, unsigned long long* slot, hipStream_t s);

struct AttnArgs {
  const float* q = nullptr;
  const void* kc = nullptr;      // [nkv][L_stride][hd] of kv_type
  const void* vc = nullptr;
  int kv_type = TPT_TYPE_F16;    // TPT_TYPE_F16 or TPT_TYPE_F32
  float* o = nullptr;
  int nq = 0, nkv = 0, hd = 0, L_stride = 0;
  int L_host = 0;                    // used when state == nullptr
  const StepState* state = nullptr;  // L = state->pos + 1
  int n_chunks = 0;
  int chunk_len = 0;                 // positions per chunk (multiple of 16, <= 1024); chunk c
                                     // covers [c*chunk_len, (c+1)*chunk_len) clipped to L
  float* part = nullptr;             // [nqb][nkv][n_chunks][G][hd + 2] chunk records
  // prefill: nqb query positions at once; query t reads q + t*ldq, writes o + t*ldo and sees
  // L + t cached positions (causal)
  int nqb = 1, ldq = 0, ldo = 0;
};
int attn_part_floats(int nq, int nkv, int hd, int n_chunks);
int attn_default_chunks(int L, int nkv);
int attn_chunk_len(int L, int n_chunks);  // smallest multiple of 16 covering L in n_chunks
int attn_max_len();  // longest cache the split-K partition supports
int launch_attn_decode(const AttnArgs& a, hipStream_t s);
// Causal multi-query attention of a prompt batch on the matrix cores (k_attn_causal.hip): query t
// of nqb sits at position L_host - 1 + t and sees positions [0, L_host + t); fp16 cache, head_dim
// 64 or 128, Nq/Nkv 1, 2, 4 or 8, 16-byte aligned rows; the chunk fields and part are unused.
bool attn_causal_mfma_supported(const AttnArgs& a);
int launch_attn_causal_mfma(const AttnArgs& a, hipStream_t s);

// Start of a decode step: pick the token, embed it (x = dequant(token_embd[tok])), advance the
// step state and clear the amax slot the LM head will write.
// Prefill helpers: embedding rows of T token ids, and the Q/K/V post-pass (interleaved RoPE of
// q and k at positions pos0 + t, q to q_out [T][qd], k and v appended to the cache).
int launch_embed_rows(const uint32_t* ids, int T, int embd_type, const uint8_t* embd,
                      size_t embd_row_bytes, int H, float* x, hipStream_t s);
struct QkvPostArgs {
  const float* qkv = nullptr;  // [T][qd + 2kd]
  int T = 0, qd = 0, kd = 0, hd = 0;
  float* q = nullptr;          // [T][qd]
  void* kcache = nullptr;
  void* vcache = nullptr;
  int kv_type = TPT_TYPE_F16, max_ctx = 0, pos0 = 0;
  const float* rope_cos = nullptr;
  const float* rope_sin = nullptr;
};
int launch_qkv_post(const QkvPostArgs& a, hipStream_t s);

// ssq (optional): n_ssq slots receive sum(x^2) in slot 0 and zeros after it, the partial-sum
// form the first layer's RMSNorm prologue reads (GemvArgs::ssq_in).
int launch_step_begin(StepState* st, const uint32_t* prompt, int embd_type,
                      const uint8_t* embd, size_t embd_row_bytes, int H, int vocab, float* x,
                      uint32_t* tok_log, float* ssq, int n_ssq, hipStream_t s);

}  // namespace tpt
