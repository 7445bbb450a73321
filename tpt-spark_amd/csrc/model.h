// Device-resident Llama model for bs=1 decode (host side).
#pragma once
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "gguf.h"
#include "kernels.h"

struct tpt_model {
  struct Layer {
    const uint8_t *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr;
    const uint8_t *gate = nullptr, *up = nullptr, *down = nullptr;
    const float *attn_norm = nullptr, *ffn_norm = nullptr;
    int tq = 0, tk = 0, tv = 0, to = 0, tg = 0, tu = 0, td = 0;
    bool qkv_adjacent = false;  // q, k, v rows contiguous in HBM and of one type
    bool gu_adjacent = false;   // gate and up rows contiguous in HBM and of one type
  };

  tpt_ctx* ctx = nullptr;  // not owned
  hipStream_t stream = nullptr;
  tpt_model_desc desc{};
  std::string path;

  uint8_t* arena = nullptr;  // all weights, blocks unchanged
  size_t arena_bytes = 0;
  std::vector<Layer> layers;
  const uint8_t* embd = nullptr;
  int embd_type = 0;
  size_t embd_row = 0;
  const uint8_t* out = nullptr;
  int out_type = 0;
  const float* out_norm = nullptr;

  // runtime buffers
  void* kv = nullptr;  // [layer][K|V][nkv][max_ctx][hd] of desc.kv_type (fp16 or f32)
  size_t kv_elem = 2;
  float *x = nullptr, *qbuf = nullptr, *attn = nullptr, *hbuf = nullptr, *logits = nullptr;
  float *rope_cos = nullptr, *rope_sin = nullptr;  // [max_ctx][hd/2]
  tpt::StepState* st = nullptr;
  uint32_t* prompt_dev = nullptr;  // [max_ctx] token ids by position
  uint32_t* tok_log = nullptr;     // [max_ctx] token consumed at each position
  float* attn_part = nullptr;
  int attn_max_chunks = 0;
  // RMSNorm partial sums (GemvArgs::ssq_in): ssq_a = sum(x^2) pieces after the attention block's
  // residual add (written by the Wo GEMV), ssq_b after the FFN block's (down GEMV, or step_begin
  // for the first layer); ssq_b_n = how many slots of ssq_b the last writer filled (0: none,
  // the next RMSNorm reduces x itself)
  float *ssq_a = nullptr, *ssq_b = nullptr;
  int ssq_b_n = 0;
  void* runtime = nullptr;  // one allocation holding the buffers above

  tpt::StepState* st_host = nullptr;  // pinned
  uint32_t* ids_host = nullptr;       // pinned staging for prompt ids [max_ctx]
  bool use_graphs = true;
  std::map<int, hipGraphExec_t> graphs;  // by length bucket

  int set_decode_path(int path);  // TPT_DECODE_KERNELS only

  // batched prefill (MFMA GEMMs over up to kPrefillT positions at once)
  static constexpr int kPrefillT = 2048;
  bool batched_prefill = false;       // every layer matrix is Q4_K
  bool causal_mfma = true;            // prompt attention on the matrix cores where supported
  float* pf_gsplit = nullptr;         // split-K workspace of the prefill GEMMs (short prompts)
  size_t pf_gsplit_floats = 0;
  void* pf_mem = nullptr;             // scratch of the batched prefill, grown on demand
  size_t pf_bytes = 0;
  float *pf_x = nullptr, *pf_qkv = nullptr, *pf_q = nullptr, *pf_att = nullptr, *pf_g = nullptr,
        *pf_u = nullptr, *pf_part = nullptr, *pf_ad = nullptr;
  uint16_t* pf_af = nullptr;  // activation rows for the GEMMs (fp16)
  uint16_t* pf_af2 = nullptr; // F16 layer matrices: the fp16 remainder rows
  bool has_f16_matrix = false;
  int16_t* pf_as16 = nullptr;
  uint32_t* pf_ids = nullptr;

  ~tpt_model();
  int load(tpt_ctx* c, const char* gguf_path, int max_ctx, int kv_type, tpt_progress_fn progress,
           void* user);
  int enqueue_step(int bucket, bool lm_head);
  int enqueue_layer(int l, int n_chunks, int chunk_len);
  int launch_step(int L, bool lm_head);  // graph replay (or direct launches)
  int bucket_of(int L) const;
  int set_state(int next_pos, int prompt_len, int use_override, uint32_t tok);
  int read_state(tpt::StepState* out);
  int prefill(const uint32_t* ids, int n, int pos0, uint32_t* next_out, float* logits_out);
  int prefill_steps(int n, int pos0);       // one decode step per position
  int prefill_batched(int n, int pos0);     // GEMM path; ids already in ids_host
  int prefill_scratch(int T, int n_chunks);
  int batched_layers(int T, int p0, int l0, int l1);  // layers [l0, l1) over the rows in pf_x
  int run_layers(const float* x_in, int n, int pos0, int l0, int l1, int path, float* x_out);
  // fn(user, s, tok) receives the token step s produced, in order; non-zero stops the run.
  typedef int (*StepFn)(void* user, int s, uint32_t tok);
  int decode_stream(uint32_t first, int pos0, int n_steps, StepFn fn, void* user, int* n_delivered);
  int decode_greedy(uint32_t first, int pos0, int n_steps, int64_t stop, uint32_t* out);
};
