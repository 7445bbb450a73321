// Device-resident Llama model: GGUF upload, decode step, prefill, greedy decode loop.
//
// Replaces load_gguf_to_vram (src-tauri/src/engine/wgpu_loader.rs:87-201), KvCache
// (wgpu_kvcache.rs:15-79) and the per-token run_forward_pass (wgpu_engine.rs:339-490).  The
// forward pass restates candle's quantized_llama (the reference CandleEngine's model):
//   x = embed(tok); per layer: x += Wo . attn(rope(Wq.n(x)), rope(Wk.n(x)), Wv.n(x));
//   x += W2 . (silu(W1.n'(x)) * W3.n'(x)); logits = Wout . n_out(x)
// with the residual adds the wgpu engine omits (wgpu_engine.rs:443,474).  One decode step is
// 2 + 5 * n_layers kernels (step begin, per layer QKV+RoPE+KV append / attention / Wo+residual /
// gate|up+SiLU / down+residual, LM head + argmax), captured once into a HIP graph and replayed
// for every token: position, token source and argmax slot live in a device StepState.
#include "model.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <cstddef>

using namespace tpt;

namespace {

bool matrix_type_ok(int t) {
  return t == TPT_TYPE_Q4_K || t == TPT_TYPE_Q5_K || t == TPT_TYPE_Q6_K || t == TPT_TYPE_Q8_0 || t == TPT_TYPE_Q4_0 ||
         t == TPT_TYPE_F16;
}

const char* type_name(int t) {
  switch (t) {
    case TPT_TYPE_F32: return "F32";
    case TPT_TYPE_F16: return "F16";
    case TPT_TYPE_Q8_0: return "Q8_0";
    case TPT_TYPE_Q4_0: return "Q4_0";
    case TPT_TYPE_Q5_K: return "Q5_K";
    case TPT_TYPE_Q4_K: return "Q4_K";
    case TPT_TYPE_Q6_K: return "Q6_K";
  }
  return "unsupported";
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace

tpt_model::~tpt_model() {
  if (ctx) (void)hipSetDevice(ctx->device);
  if (stream) (void)hipStreamSynchronize(stream);
  for (auto& kv : graphs) (void)hipGraphExecDestroy(kv.second);
  graphs.clear();
  if (arena) (void)hipFree(arena);
  if (runtime) (void)hipFree(runtime);
  if (pf_mem) (void)hipFree(pf_mem);
  if (st_host) (void)hipHostFree(st_host);
  if (ids_host) (void)hipHostFree(ids_host);
}

// Metadata and tensor table of a Llama GGUF, validated for this engine: extract_meta's keys and
// defaults (wgpu_loader.rs:305-406), the architecture check of CandleEngine::load
// (candle_engine.rs:146-156), and every tensor the forward pass reads present with the shape,
// type and byte size its kernels assume.  Host only: nothing touches a device.
struct ModelTensors {
  struct LT { const GgufTensor *q, *k, *v, *o, *g, *u, *d, *an, *fn; };
  std::vector<LT> lt;
  const GgufTensor *te = nullptr, *to = nullptr, *ton = nullptr;
};

static int read_model_meta(const GgufFile& f, tpt_model_desc& desc, ModelTensors& mt) {
  int rc;
  // ---- metadata (extract_meta, wgpu_loader.rs:305-406; arch check as CandleEngine::load,
  //      candle_engine.rs:146-156: the Llama-dense families this engine implements)
  std::string arch = "llama";
  f.get_str("general.architecture", &arch);
  if (arch != "llama" && arch != "mistral")
    return fail(TPT_ERR_UNSUPPORTED, "Architecture '" + arch + "' is not supported by engine-hip. Supported: llama, mistral.");
  const std::string a = arch;
  uint64_t u;
  float fv;
  desc = tpt_model_desc{};
  snprintf(desc.architecture, sizeof desc.architecture, "%s", arch.c_str());
  desc.context_length = f.get_u64(a + ".context_length", &u) ? (int)u : 4096;
  desc.n_layers = f.get_u64(a + ".block_count", &u) ? (int)u : 32;
  desc.n_heads = f.get_u64(a + ".attention.head_count", &u) ? (int)u : 32;
  desc.n_kv_heads = f.get_u64(a + ".attention.head_count_kv", &u) ? (int)u : desc.n_heads;
  desc.embed = f.get_u64(a + ".embedding_length", &u) ? (int)u : 4096;
  desc.rope_base = f.get_f32(a + ".rope.freq_base", &fv) ? fv : 10000.f;
  desc.rms_eps = f.get_f32(a + ".attention.layer_norm_rms_epsilon", &fv) ? fv : 1e-5f;
  desc.rope_scale = 1.f;  // candle's quantized_llama applies no RoPE scaling
  if (desc.n_layers < 1 || desc.n_layers > 4096 || desc.embed < 1)
    return fail(TPT_ERR_FORMAT, "block_count / embedding_length out of range in GGUF metadata");
  if (desc.n_heads <= 0 || desc.n_kv_heads <= 0 || desc.embed % desc.n_heads || desc.n_heads % desc.n_kv_heads)
    return fail(TPT_ERR_FORMAT, "inconsistent head counts in GGUF metadata");
  desc.head_dim = desc.embed / desc.n_heads;
  const int rope_dim = f.get_u64(a + ".rope.dimension_count", &u) ? (int)u : desc.head_dim;
  if (rope_dim != desc.head_dim)
    return fail(TPT_ERR_UNSUPPORTED, "partial rotary embeddings (rope.dimension_count != head_dim) are not supported");
  const int H = desc.embed, hd = desc.head_dim, nq = desc.n_heads, nkv = desc.n_kv_heads;
  const int qd = nq * hd, kd = nkv * hd;

  // ---- tensors
  auto need = [&](const std::string& name, int64_t ne0, int64_t ne1, const GgufTensor** out) -> int {
    const GgufTensor* t = f.find(name);
    if (!t) return fail(TPT_ERR_FORMAT, "missing tensor " + name);
    if (type_bytes(t->type) == 0 || !t->data)
      return fail(TPT_ERR_UNSUPPORTED, "tensor " + name + " has ggml type " + std::to_string(t->type) + ", which engine-hip does not read");
    // a matrix [ne1][ne0] or a vector [ne0]: higher extents 1, at least one row, and exactly the
    // bytes the kernels read (ne1 rows of ne0 elements), so no kernel reads past the tensor
    if (t->n_dims > 2 || t->ne[2] != 1 || t->ne[3] != 1 || t->ne[0] != ne0 || t->ne[1] < 1 ||
        (ne1 >= 0 && t->ne[1] != ne1))
      return fail(TPT_ERR_FORMAT, "tensor " + name + " has an unexpected shape");
    if (t->bytes != (size_t)t->ne[1] * row_bytes(t->type, (int)ne0))
      return fail(TPT_ERR_FORMAT, "tensor " + name + " has an unexpected byte size");
    *out = t;
    return TPT_OK;
  };
  const GgufTensor *&te = mt.te, *&to = mt.to, *&ton = mt.ton;
  if ((rc = need("token_embd.weight", H, -1, &te))) return rc;
  desc.vocab = (int)te->ne[1];
  if (f.find("output.weight")) {
    if ((rc = need("output.weight", H, desc.vocab, &to))) return rc;
  } else {
    to = te;  // quantized_llama falls back to tok_embeddings
  }
  if ((rc = need("output_norm.weight", H, -1, &ton))) return rc;
  if (ton->type != TPT_TYPE_F32) return fail(TPT_ERR_UNSUPPORTED, "output_norm must be F32");
  if (!matrix_type_ok(to->type)) return fail(TPT_ERR_UNSUPPORTED, std::string("output.weight type ") + type_name(to->type) + " is not supported");
  const GgufTensor* g0 = f.find("blk.0.ffn_gate.weight");
  if (!g0) return fail(TPT_ERR_FORMAT, "missing tensor blk.0.ffn_gate.weight");
  uint64_t ffn_meta;
  desc.ffn = f.get_u64(a + ".feed_forward_length", &ffn_meta) ? (int)ffn_meta : (int)g0->ne[1];

  mt.lt.resize(desc.n_layers);
  std::vector<ModelTensors::LT>& lt = mt.lt;
  for (int l = 0; l < desc.n_layers; l++) {
    const std::string p = "blk." + std::to_string(l) + ".";
    ModelTensors::LT& t = lt[l];
    if ((rc = need(p + "attn_q.weight", H, qd, &t.q)) || (rc = need(p + "attn_k.weight", H, kd, &t.k)) ||
        (rc = need(p + "attn_v.weight", H, kd, &t.v)) || (rc = need(p + "attn_output.weight", qd, H, &t.o)) ||
        (rc = need(p + "ffn_gate.weight", H, desc.ffn, &t.g)) || (rc = need(p + "ffn_up.weight", H, desc.ffn, &t.u)) ||
        (rc = need(p + "ffn_down.weight", desc.ffn, H, &t.d)) || (rc = need(p + "attn_norm.weight", H, -1, &t.an)) ||
        (rc = need(p + "ffn_norm.weight", H, -1, &t.fn)))
      return rc;
    for (const GgufTensor* m : {t.q, t.k, t.v, t.o, t.g, t.u, t.d})
      if (!matrix_type_ok(m->type))
        return fail(TPT_ERR_UNSUPPORTED, "tensor " + m->name + " has type " + type_name(m->type) + "; engine-hip reads Q4_K, Q5_K, Q6_K, Q8_0, Q4_0 and F16 matrices");
    if (t.an->type != TPT_TYPE_F32 || t.fn->type != TPT_TYPE_F32) return fail(TPT_ERR_UNSUPPORTED, "norm weights must be F32");
    if (t.g->type != t.u->type)
      return fail(TPT_ERR_UNSUPPORTED, "ffn_gate and ffn_up of different types are not supported yet");
    if (H % 256 || desc.ffn % 256 || qd % 256) return fail(TPT_ERR_UNSUPPORTED, "dimensions must be multiples of 256");
  }

  uint64_t step_bytes = 0, total = 0;
  for (const ModelTensors::LT& t : lt)
    for (const GgufTensor* m : {t.q, t.k, t.v, t.o, t.g, t.u, t.d, t.an, t.fn}) step_bytes += m->bytes;
  total = step_bytes + te->bytes + (to != te ? to->bytes : 0) + ton->bytes;
  desc.weight_bytes = total;
  desc.decode_bytes_per_token = step_bytes + to->bytes + ton->bytes + row_bytes(te->type, desc.embed);
  desc.type_q = lt[0].q->type; desc.type_k = lt[0].k->type; desc.type_v = lt[0].v->type;
  desc.type_o = lt[0].o->type; desc.type_gate = lt[0].g->type; desc.type_up = lt[0].u->type;
  desc.type_down = lt[0].d->type; desc.type_embd = te->type; desc.type_out = to->type;
  return TPT_OK;
}

int tpt_model::load(tpt_ctx* c, const char* gguf_path, int max_ctx_req, int kv_type,
                    tpt_progress_fn progress, void* user) {
  if (kv_type != TPT_TYPE_F16 && kv_type != TPT_TYPE_F32)
    return fail(TPT_ERR_UNSUPPORTED, "KV cache type must be F16 or F32");
  ctx = c;
  stream = c->stream;
  path = gguf_path;
  GgufFile f;
  int rc = f.open(gguf_path);
  if (rc) return rc;
  ModelTensors mt;
  if ((rc = read_model_meta(f, desc, mt))) return rc;
  const int H = desc.embed, hd = desc.head_dim, nq = desc.n_heads, nkv = desc.n_kv_heads;
  const int qd = nq * hd;
  const std::vector<ModelTensors::LT>& lt = mt.lt;
  const GgufTensor *te = mt.te, *to = mt.to, *ton = mt.ton;

  // ---- HBM layout: per layer q|k|v adjacent (one GEMV over qd + 2 kd rows), then the rest
  std::vector<std::pair<const GgufTensor*, size_t>> plan;  // tensor, arena offset
  size_t off = 0;
  auto place = [&](const GgufTensor* t, size_t align) {
    off = align_up(off, align);
    plan.push_back({t, off});
    off += t->bytes;
  };
  for (auto& t : lt) {
    place(t.q, 256);
    place(t.k, 1);
    place(t.v, 1);
    place(t.o, 256);
    place(t.g, 256);
    place(t.u, 256);
    place(t.d, 256);
    place(t.an, 256);
    place(t.fn, 256);
  }
  place(te, 256);
  if (to != te) place(to, 256);
  place(ton, 256);
  arena_bytes = align_up(off, 256);
  TPT_HIP(hipSetDevice(c->device));
  TPT_HIP(hipMalloc((void**)&arena, arena_bytes));

  // ---- upload, blocks unchanged, through two pinned staging buffers
  const size_t SB = 64u << 20;
  uint8_t* stage[2] = {nullptr, nullptr};
  hipEvent_t ev[2] = {nullptr, nullptr};
  TPT_HIP(hipHostMalloc((void**)&stage[0], SB));
  TPT_HIP(hipHostMalloc((void**)&stage[1], SB));
  TPT_HIP(hipEventCreate(&ev[0]));
  TPT_HIP(hipEventCreate(&ev[1]));
  int which = 0;
  bool used[2] = {false, false};
  uint32_t done = 0;
  const uint32_t total = (uint32_t)plan.size();
  hipError_t he = hipSuccess;
  for (auto& pt : plan) {
    const uint8_t* src = pt.first->data;
    size_t left = pt.first->bytes, doff = pt.second;
    while (left && he == hipSuccess) {
      const size_t n = std::min(left, SB);
      if (used[which]) he = hipEventSynchronize(ev[which]);
      if (he != hipSuccess) break;
      memcpy(stage[which], src, n);
      he = hipMemcpyAsync(arena + doff, stage[which], n, hipMemcpyHostToDevice, stream);
      if (he == hipSuccess) he = hipEventRecord(ev[which], stream);
      used[which] = true;
      which ^= 1;
      src += n;
      doff += n;
      left -= n;
    }
    if (he != hipSuccess) break;
    done++;
    if (progress) progress(user, done, total);  // on_progress(done, total), wgpu_loader.rs:184-187
  }
  if (he == hipSuccess) he = hipStreamSynchronize(stream);
  (void)hipEventDestroy(ev[0]);
  (void)hipEventDestroy(ev[1]);
  (void)hipHostFree(stage[0]);
  (void)hipHostFree(stage[1]);
  if (he != hipSuccess) return hip_fail(he, "weight upload", __FILE__, __LINE__);

  auto dev = [&](const GgufTensor* t) -> const uint8_t* {
    for (auto& pt : plan)
      if (pt.first == t) return arena + pt.second;
    return nullptr;
  };
  layers.resize(desc.n_layers);
  for (int l = 0; l < desc.n_layers; l++) {
    Layer& L = layers[l];
    const ModelTensors::LT& t = lt[l];
    L.q = dev(t.q); L.k = dev(t.k); L.v = dev(t.v); L.o = dev(t.o);
    L.gate = dev(t.g); L.up = dev(t.u); L.down = dev(t.d);
    L.attn_norm = (const float*)dev(t.an);
    L.ffn_norm = (const float*)dev(t.fn);
    L.tq = t.q->type; L.tk = t.k->type; L.tv = t.v->type; L.to = t.o->type;
    L.tg = t.g->type; L.tu = t.u->type; L.td = t.d->type;
    L.qkv_adjacent = L.tq == L.tk && L.tk == L.tv && L.k == L.q + t.q->bytes && L.v == L.k + t.k->bytes;
    L.gu_adjacent = L.tg == L.tu && L.up == L.gate + t.g->bytes;
  }
  embd = dev(te);
  embd_type = te->type;
  embd_row = row_bytes(te->type, H);
  out = dev(to);
  out_type = to->type;
  out_norm = (const float*)dev(ton);
  desc.weight_bytes = arena_bytes;

  // ---- runtime state
  const int max_ctx = max_ctx_req > 0 ? max_ctx_req : desc.context_length;
  if (max_ctx <= 0) return fail(TPT_ERR_INVALID, "max_ctx must be positive");
  if (max_ctx > attn_max_len()) return fail(TPT_ERR_UNSUPPORTED, "max_ctx exceeds the attention partition limit");
  desc.max_ctx = max_ctx;
  desc.kv_type = kv_type;
  kv_elem = kv_type == TPT_TYPE_F32 ? 4 : 2;
  attn_max_chunks = attn_default_chunks(max_ctx, nkv);
  for (int L = 1; L <= max_ctx; L = bucket_of(L) + 1)
    attn_max_chunks = std::max(attn_max_chunks, attn_default_chunks(bucket_of(L), nkv));
  const size_t kv_elems = (size_t)desc.n_layers * 2 * nkv * (size_t)max_ctx * hd;
  size_t ro = 0;
  auto carve = [&](size_t bytes) { size_t o = ro; ro = align_up(ro + bytes, 256); return o; };
  const size_t o_kv = carve(kv_elems * kv_elem), o_x = carve((size_t)H * 4), o_q = carve((size_t)qd * 4),
               o_at = carve((size_t)qd * 4), o_h = carve((size_t)desc.ffn * 4),
               o_lg = carve((size_t)desc.vocab * 4), o_rc = carve((size_t)max_ctx * hd / 2 * 4),
               o_rs = carve((size_t)max_ctx * hd / 2 * 4), o_st = carve(sizeof(StepState)),
               o_pr = carve((size_t)max_ctx * 4), o_tl = carve((size_t)max_ctx * 4),
               o_ap = carve((size_t)attn_part_floats(nq, nkv, hd, attn_max_chunks) * 4),
               o_ss = carve((size_t)2 * kSsqMax * 4);
  TPT_HIP(hipMalloc(&runtime, ro));
  uint8_t* R = (uint8_t*)runtime;
  kv = R + o_kv;
  x = (float*)(R + o_x);
  qbuf = (float*)(R + o_q);
  attn = (float*)(R + o_at);
  hbuf = (float*)(R + o_h);
  logits = (float*)(R + o_lg);
  rope_cos = (float*)(R + o_rc);
  rope_sin = (float*)(R + o_rs);
  st = (StepState*)(R + o_st);
  prompt_dev = (uint32_t*)(R + o_pr);
  tok_log = (uint32_t*)(R + o_tl);
  attn_part = (float*)(R + o_ap);
  ssq_a = (float*)(R + o_ss);
  ssq_b = ssq_a + kSsqMax;
  TPT_HIP(hipMemsetAsync(runtime, 0, ro, stream));  // load time, outside any graph

  // RoPE tables exactly as quantized_llama::precomput_freqs_cis: f32 theta = 1/base^(2i/d)
  // (powf), angle = (f32)pos * theta, cosf/sinf of the host libm.
  {
    const int half = hd / 2;
    std::vector<float> theta(half), tc((size_t)max_ctx * half), ts((size_t)max_ctx * half);
    for (int i = 0; i < half; i++) theta[i] = 1.f / powf(desc.rope_base, (float)(2 * i) / (float)hd);
    for (int p = 0; p < max_ctx; p++)
      for (int i = 0; i < half; i++) {
        const float ang = (float)p * theta[i];
        tc[(size_t)p * half + i] = cosf(ang);
        ts[(size_t)p * half + i] = sinf(ang);
      }
    // on the model stream, behind the clearing of the runtime region (a plain hipMemcpy runs
    // on the null stream, which does not wait for this non-blocking stream), and complete
    // before the host tables go out of scope
    TPT_HIP(hipMemcpyAsync(rope_cos, tc.data(), tc.size() * 4, hipMemcpyHostToDevice, stream));
    TPT_HIP(hipMemcpyAsync(rope_sin, ts.data(), ts.size() * 4, hipMemcpyHostToDevice, stream));
    TPT_HIP(hipStreamSynchronize(stream));
  }
  TPT_HIP(hipHostMalloc((void**)&st_host, sizeof(StepState)));
  TPT_HIP(hipHostMalloc((void**)&ids_host, (size_t)max_ctx * 4));
  // every layer matrix type has a GEMM form: the batched prefill is the default
  batched_prefill = true;
  has_f16_matrix = false;
  for (const Layer& L : layers)
    for (int t : {L.tq, L.tk, L.tv, L.to, L.tg, L.tu, L.td}) has_f16_matrix |= t == TPT_TYPE_F16;
  const char* ev_pf = getenv("TPT_HIP_PREFILL");
  if (ev_pf && strcmp(ev_pf, "steps") == 0) batched_prefill = false;
  const char* ev_att = getenv("TPT_HIP_CAUSAL_ATTN");
  causal_mfma = !(ev_att && strcmp(ev_att, "splitk") == 0);
  const char* ev_graph = getenv("TPT_HIP_GRAPHS");
  use_graphs = !(ev_graph && ev_graph[0] == '0');
  TPT_HIP(hipStreamSynchronize(stream));
  return TPT_OK;
}

// One launch per fused op is the only decode form: a persistent kernel (embedding and every layer
// in one launch, grid barriers between the phases) decoded the 8B shape at 476-488 tok/s
// against 586-592 and was removed; TPT_DECODE_PERSISTENT is refused.
int tpt_model::set_decode_path(int path) {
  if (path == TPT_DECODE_KERNELS) return TPT_OK;
  if (path == TPT_DECODE_PERSISTENT)
    return fail(TPT_ERR_UNSUPPORTED, "no persistent decode kernel: decode steps run one launch per fused op");
  return fail(TPT_ERR_INVALID, "decode path must be TPT_DECODE_KERNELS or TPT_DECODE_PERSISTENT");
}

// Attention partition of the length bucket holding L (64, 128, 256, 512, then multiples of
// 512): the chunk count and chunk length are fixed per bucket, so one captured graph serves every
// length in it, and chunks past the live length cost an early exit only.
int tpt_model::bucket_of(int L) const {
  if (L > 512) return (L + 511) / 512 * 512;
  int b = 64;
  while (b < L) b *= 2;
  return b;
}

int tpt_model::enqueue_step(int bucket, bool lm_head) {
  const int n_chunks = std::min(attn_default_chunks(bucket, desc.n_kv_heads), attn_max_chunks);
  const int chunk_len = attn_chunk_len(bucket, n_chunks);
  int rc;
  if ((rc = launch_step_begin(st, prompt_dev, embd_type, embd, embd_row, desc.embed, desc.vocab,
                              x, tok_log, ssq_b, kSsqMax, stream)))
    return rc;
  ssq_b_n = kSsqMax;
  for (int l = 0; l < desc.n_layers; l++)
    if ((rc = enqueue_layer(l, n_chunks, chunk_len))) return rc;
  if (lm_head) {
    GemvArgs lh;
    lh.w0 = out;
    lh.row_stride = row_bytes(out_type, desc.embed);
    lh.K = desc.embed;
    lh.N = desc.vocab;
    lh.x = x;
    lh.norm_w = out_norm;
    lh.eps = desc.rms_eps;
    lh.prologue = PRO_RMSNORM;
    lh.epilogue = EPI_ARGMAX;
    lh.y = logits;
    lh.amax = (unsigned long long*)((char*)st + offsetof(StepState, amax));  // device address
    lh.state = st;
    lh.ssq_in = ssq_b_n ? ssq_b : nullptr;
    lh.n_ssq = ssq_b_n;
    if ((rc = launch_gemv_q8(ctx, out_type, lh, stream))) return rc;
  }
  return TPT_OK;
}

// One decoder layer of a decode step on the residual stream x at position state->pos.
int tpt_model::enqueue_layer(int l, int n_chunks, int chunk_len) {
  const int H = desc.embed, hd = desc.head_dim, nq = desc.n_heads, nkv = desc.n_kv_heads;
  const int qd = nq * hd, kd = nkv * hd, F = desc.ffn, mc = desc.max_ctx;
  const size_t layer_kv = (size_t)2 * nkv * mc * hd;
  int rc;
  {
    const Layer& L = layers[l];
    uint8_t* kc = (uint8_t*)kv + (size_t)l * layer_kv * kv_elem;
    uint8_t* vc = kc + (size_t)nkv * mc * hd * kv_elem;
    // norm -> Q|K|V GEMV -> RoPE -> q buffer / fp16 KV append at state->pos
    GemvArgs g;
    g.K = H;
    g.x = x;
    g.norm_w = L.attn_norm;
    g.eps = desc.rms_eps;
    g.prologue = PRO_RMSNORM;
    g.epilogue = EPI_ROPE_QKV;
    g.y = qbuf;
    g.qd = qd;
    g.kd = kd;
    g.hd = hd;
    g.max_ctx = mc;
    g.rope_cos = rope_cos;
    g.rope_sin = rope_sin;
    g.kcache = kc;
    g.vcache = vc;
    g.kv_type = desc.kv_type;
    g.state = st;
    g.ssq_in = ssq_b_n ? ssq_b : nullptr;
    g.n_ssq = ssq_b_n;
    if (L.qkv_adjacent) {
      g.w0 = L.q;
      g.row_stride = row_bytes(L.tq, H);
      g.N = qd + 2 * kd;
      if ((rc = launch_gemv_q8(ctx, L.tq, g, stream))) return rc;
    } else {
      const uint8_t* ws[3] = {L.q, L.k, L.v};
      const int ts[3] = {L.tq, L.tk, L.tv}, ns[3] = {qd, kd, kd}, r0[3] = {0, qd, qd + kd};
      for (int i = 0; i < 3; i++) {
        g.w0 = ws[i];
        g.row_stride = row_bytes(ts[i], H);
        g.N = ns[i];
        g.row0 = r0[i];
        if ((rc = launch_gemv_q8(ctx, ts[i], g, stream))) return rc;
      }
    }
    // attention over positions 0..state->pos
    AttnArgs at;
    at.q = qbuf;
    at.kc = kc;
    at.vc = vc;
    at.kv_type = desc.kv_type;
    at.o = attn;
    at.nq = nq;
    at.nkv = nkv;
    at.hd = hd;
    at.L_stride = mc;
    at.state = st;
    at.n_chunks = n_chunks;
    at.chunk_len = chunk_len;
    at.part = attn_part;
    if ((rc = launch_attn_decode(at, stream))) return rc;
    // x += Wo . attn
    GemvArgs wo;
    wo.w0 = L.o;
    wo.row_stride = row_bytes(L.to, qd);
    wo.K = qd;
    wo.N = H;
    wo.x = attn;
    wo.epilogue = EPI_RESID;
    wo.y = x;
    wo.resid = x;
    const int n_wo = gemv_grid(ctx, L.to, wo);
    if (n_wo >= 1 && n_wo <= kSsqMax) wo.ssq_out = ssq_a;
    if ((rc = launch_gemv_q8(ctx, L.to, wo, stream))) return rc;
    // h = silu(W1 . n(x)) * (W3 . n(x))
    GemvArgs gu;
    gu.w0 = L.gate;
    gu.w1 = L.up;
    gu.row_stride = row_bytes(L.tg, H);
    gu.K = H;
    gu.N = F;
    gu.x = x;
    gu.norm_w = L.ffn_norm;
    gu.eps = desc.rms_eps;
    gu.prologue = PRO_RMSNORM;
    gu.epilogue = EPI_SWIGLU;
    gu.y = hbuf;
    if (wo.ssq_out) {
      gu.ssq_in = ssq_a;
      gu.n_ssq = n_wo;
    }
    if ((rc = launch_gemv_q8(ctx, L.tg, gu, stream))) return rc;
    // x += W2 . h
    GemvArgs dn;
    dn.w0 = L.down;
    dn.row_stride = row_bytes(L.td, F);
    dn.K = F;
    dn.N = H;
    dn.x = hbuf;
    dn.epilogue = EPI_RESID;
    dn.y = x;
    dn.resid = x;
    const int n_dn = gemv_grid(ctx, L.td, dn);
    ssq_b_n = n_dn >= 1 && n_dn <= kSsqMax ? n_dn : 0;
    if (ssq_b_n) dn.ssq_out = ssq_b;
    if ((rc = launch_gemv_q8(ctx, L.td, dn, stream))) return rc;
  }
  return TPT_OK;
}

int tpt_model::launch_step(int L, bool lm_head) {
  if (L > desc.max_ctx) return fail(TPT_ERR_STATE, "context length exhausted");
  const int nch = bucket_of(L);
  if (!use_graphs || !lm_head) return enqueue_step(nch, lm_head);
  auto it = graphs.find(nch);
  if (it == graphs.end()) {
    hipGraph_t g = nullptr;
    TPT_HIP(hipStreamBeginCapture(stream, hipStreamCaptureModeRelaxed));
    int rc = enqueue_step(nch, true);
    hipError_t e = hipStreamEndCapture(stream, &g);
    if (rc) {
      if (g) (void)hipGraphDestroy(g);
      return rc;
    }
    if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture", __FILE__, __LINE__);
    hipGraphExec_t ex = nullptr;
    e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate", __FILE__, __LINE__);
    it = graphs.emplace(nch, ex).first;
  }
  TPT_HIP(hipGraphLaunch(it->second, stream));
  return TPT_OK;
}

int tpt_model::set_state(int next_pos, int prompt_len, int use_override, uint32_t tok) {
  memset(st_host, 0, sizeof(StepState));
  st_host->next_pos = next_pos;
  st_host->prompt_len = prompt_len;
  st_host->use_override = use_override;
  st_host->tok_override = tok;
  TPT_HIP(hipMemcpyAsync(st, st_host, sizeof(StepState), hipMemcpyHostToDevice, stream));
  // the pinned source must not change before the copy runs
  TPT_HIP(hipStreamSynchronize(stream));
  return TPT_OK;
}

int tpt_model::read_state(StepState* out_state) {
  TPT_HIP(hipMemcpyAsync(st_host, st, sizeof(StepState), hipMemcpyDeviceToHost, stream));
  TPT_HIP(hipStreamSynchronize(stream));
  *out_state = *st_host;
  return TPT_OK;
}

int tpt_model::prefill_steps(int n, int pos0) {
  int rc = set_state(pos0, pos0 + n, 0, 0);
  if (rc) return rc;
  for (int i = 0; i < n; i++)
    if ((rc = launch_step(pos0 + i + 1, true))) return rc;
  return TPT_OK;
}

int tpt_model::prefill_scratch(int T, int n_chunks) {
  const int H = desc.embed, qd = desc.n_heads * desc.head_dim, kd = desc.n_kv_heads * desc.head_dim;
  const int F = desc.ffn, Kmax = std::max(std::max(H, qd), F);
  size_t off = 0;
  auto carve = [&](size_t bytes) { size_t o = off; off = align_up(off + bytes, 256); return o; };
  const size_t o_x = carve((size_t)T * H * 4), o_af = carve((size_t)T * Kmax * 2),
               o_af2 = carve(has_f16_matrix ? (size_t)T * Kmax * 2 : 0),
               o_ad = carve((size_t)T * (Kmax / 32) * 4), o_as = carve((size_t)T * (Kmax / 16) * 2),
               o_qkv = carve((size_t)T * (qd + 2 * kd) * 4), o_q = carve((size_t)T * qd * 4),
               o_att = carve((size_t)T * qd * 4), o_g = carve((size_t)T * 2 * F * 4),
               o_part = carve((size_t)T * attn_part_floats(desc.n_heads, desc.n_kv_heads, desc.head_dim, n_chunks) * 4),
               o_ids = carve((size_t)T * 4);
  // split-K workspace of the GEMMs (short prompts): the largest splits x T x N over the shapes
  size_t gsplit = 0;
  const int shapes[5][2] = {{H, qd + 2 * kd}, {qd, H}, {H, F}, {H, 2 * F}, {F, H}};  // (K, N)
  for (const auto& kn : shapes) {
    const int ns = gemm_splits(T, kn[1], kn[0]);
    if (ns > 1) gsplit = std::max(gsplit, (size_t)ns * T * kn[1]);
  }
  const size_t o_gsplit = carve(gsplit * 4);
  if (off > pf_bytes) {
    if (pf_mem) {
      TPT_HIP(hipStreamSynchronize(stream));
      TPT_HIP(hipFree(pf_mem));
      pf_mem = nullptr;
      pf_bytes = 0;
    }
    TPT_HIP(hipMalloc(&pf_mem, off));
    pf_bytes = off;
  }
  uint8_t* b = (uint8_t*)pf_mem;
  pf_x = (float*)(b + o_x);
  pf_af = (uint16_t*)(b + o_af);
  pf_af2 = has_f16_matrix ? (uint16_t*)(b + o_af2) : nullptr;
  pf_ad = (float*)(b + o_ad);
  pf_as16 = (int16_t*)(b + o_as);
  pf_qkv = (float*)(b + o_qkv);
  pf_q = (float*)(b + o_q);
  pf_att = (float*)(b + o_att);
  pf_g = (float*)(b + o_g);  // rows of 2F: gate outputs, then up outputs
  pf_u = pf_g + F;
  pf_part = (float*)(b + o_part);
  pf_ids = (uint32_t*)(b + o_ids);
  pf_gsplit = gsplit ? (float*)(b + o_gsplit) : nullptr;
  pf_gsplit_floats = gsplit;
  return TPT_OK;
}

// Attention partition of a batched slice whose last position is Lmax - 1.
static int slice_chunks(int Lmax) { return (Lmax + 511) / 512; }

// Batched prefill of positions pos0 .. pos0+n-1 (ids in ids_host[pos0 ..]): slices of up to
// kPrefillT positions run the whole layer stack as GEMMs (candle's batched forward,
// candle_engine.rs:272-273), leaving the last position's residual stream in x for the LM head.
int tpt_model::prefill_batched(int n, int pos0) {
  int rc;
  for (int c0 = 0; c0 < n; c0 += kPrefillT) {
    const int T = std::min(kPrefillT, n - c0), p0 = pos0 + c0;
    if ((rc = prefill_scratch(T, slice_chunks(p0 + T)))) return rc;
    TPT_HIP(hipMemcpyAsync(pf_ids, ids_host + p0, (size_t)T * 4, hipMemcpyHostToDevice, stream));
    if ((rc = launch_embed_rows(pf_ids, T, embd_type, embd, embd_row, desc.embed, pf_x, stream))) return rc;
    if ((rc = batched_layers(T, p0, 0, desc.n_layers))) return rc;
    // the last position's residual stream feeds the LM head
    TPT_HIP(hipMemcpyAsync(x, pf_x + (size_t)(T - 1) * desc.embed, (size_t)desc.embed * 4,
                           hipMemcpyDeviceToDevice, stream));
  }
  return TPT_OK;
}

// Layers [l0, l1) over the T residual rows in pf_x (positions p0 .. p0+T-1), per layer as
// candle's forward orders it: rms_norm, Q/K/V, rope_i, KV append, causal attention, Wo +
// residual, rms_norm, SwiGLU, down + residual.  The scratch must be sized for (T, p0 + T).
int tpt_model::batched_layers(int T, int p0, int l0, int l1) {
  const int H = desc.embed, hd = desc.head_dim, nq = desc.n_heads, nkv = desc.n_kv_heads;
  const int qd = nq * hd, kd = nkv * hd, F = desc.ffn, mc = desc.max_ctx;
  const size_t layer_kv = (size_t)2 * nkv * mc * hd;
  const int Lmax = p0 + T, nch = slice_chunks(Lmax), cl = attn_chunk_len(Lmax, nch);
  int rc;
  // candle's arithmetic per weight type: Q8_K activation rows for the k-quants, Q8_0 rows for
  // Q8_0 / Q4_0, f32 for F16 (fp16 rounding plus remainder, two GEMM passes)
  auto mode_of = [](int type) {
    return type == TPT_TYPE_F16 ? GEMM_F16 : type == TPT_TYPE_Q8_0 || type == TPT_TYPE_Q4_0 ? GEMM_Q80 : GEMM_Q8K;
  };
  // activation rows of (x, x2, norm) in the mode the next GEMM needs; rows already prepared
  // for the same input and mode are reused
  struct Prepared { const float* x; const float* x2; const float* nw; int K, mode; } last{nullptr, nullptr, nullptr, 0, -1};
  auto prep = [&](const float* xx, const float* x2, int K, const float* nw, int type, int ldx = 0) {
    const int mode = mode_of(type);
    if (last.x == xx && last.x2 == x2 && last.nw == nw && last.K == K && last.mode == mode) return (int)TPT_OK;
    ActPrepArgs a;
    a.M = T; a.K = K; a.ldx = ldx ? ldx : K; a.x = xx; a.x2 = x2; a.norm_w = nw; a.eps = desc.rms_eps;
    a.mode = mode; a.af = pf_af; a.ad = pf_ad; a.as16 = pf_as16;
    a.af2 = mode == GEMM_F16 ? pf_af2 : nullptr;
    last = {xx, x2, nw, K, mode};
    return launch_act_prep(a, stream);
  };
  auto gemm = [&](int type, const uint8_t* w, int K, int N, float* y, int ldy, const float* resid) {
    GemmArgs g;
    g.M = T; g.N = N; g.K = K; g.mode = mode_of(type); g.wtype = type;
    g.w = w; g.w_stride = row_bytes(type, K);
    g.af = pf_af; g.ad = pf_ad; g.as16 = pf_as16;
    g.y = y; g.ldy = ldy; g.resid = resid; g.ldr = ldy;
    g.part = pf_gsplit; g.part_floats = pf_gsplit_floats;
    if (type != TPT_TYPE_F16) return launch_gemm(g, stream);
    // y = W . lo (+ resid), then y = W . hi + y
    g.af = pf_af2;
    int r = launch_gemm(g, stream);
    if (r) return r;
    g.af = pf_af;
    g.resid = y;
    return launch_gemm(g, stream);
  };
  for (int l = l0; l < l1; l++) {
    const Layer& L = layers[l];
    uint8_t* kc = (uint8_t*)kv + (size_t)l * layer_kv * kv_elem;
    uint8_t* vc = kc + (size_t)nkv * mc * hd * kv_elem;
    const int ldq = qd + 2 * kd;
    if (L.qkv_adjacent) {
      if ((rc = prep(pf_x, nullptr, H, L.attn_norm, L.tq)) || (rc = gemm(L.tq, L.q, H, ldq, pf_qkv, ldq, nullptr))) return rc;
    } else {
      if ((rc = prep(pf_x, nullptr, H, L.attn_norm, L.tq)) || (rc = gemm(L.tq, L.q, H, qd, pf_qkv, ldq, nullptr)) ||
          (rc = prep(pf_x, nullptr, H, L.attn_norm, L.tk)) || (rc = gemm(L.tk, L.k, H, kd, pf_qkv + qd, ldq, nullptr)) ||
          (rc = prep(pf_x, nullptr, H, L.attn_norm, L.tv)) || (rc = gemm(L.tv, L.v, H, kd, pf_qkv + qd + kd, ldq, nullptr)))
        return rc;
    }
    QkvPostArgs qp;
    qp.qkv = pf_qkv; qp.T = T; qp.qd = qd; qp.kd = kd; qp.hd = hd; qp.q = pf_q;
    qp.kcache = kc; qp.vcache = vc; qp.kv_type = desc.kv_type; qp.max_ctx = mc; qp.pos0 = p0;
    qp.rope_cos = rope_cos; qp.rope_sin = rope_sin;
    if ((rc = launch_qkv_post(qp, stream))) return rc;
    AttnArgs at;
    at.q = pf_q; at.ldq = qd; at.kc = kc; at.vc = vc; at.kv_type = desc.kv_type;
    at.o = pf_att; at.ldo = qd; at.nq = nq; at.nkv = nkv; at.hd = hd; at.L_stride = mc;
    at.L_host = p0 + 1; at.nqb = T; at.n_chunks = nch; at.chunk_len = cl; at.part = pf_part;
    rc = causal_mfma && attn_causal_mfma_supported(at) ? launch_attn_causal_mfma(at, stream)
                                                       : launch_attn_decode(at, stream);
    if (rc) return rc;
    if ((rc = prep(pf_att, nullptr, qd, nullptr, L.to)) || (rc = gemm(L.to, L.o, qd, H, pf_x, H, pf_x))) return rc;
    // pf_x changed in place: the rows prepared from it before are stale
    last.mode = -1;
    // gate and up outputs side by side in rows of 2F; adjacent matrices of one type are one GEMM
    // over 2F weight rows (twice the output tiles: whole rounds over the CUs at 2048 positions)
    if (L.gu_adjacent) {
      if ((rc = prep(pf_x, nullptr, H, L.ffn_norm, L.tg)) || (rc = gemm(L.tg, L.gate, H, 2 * F, pf_g, 2 * F, nullptr)))
        return rc;
    } else {
      if ((rc = prep(pf_x, nullptr, H, L.ffn_norm, L.tg)) || (rc = gemm(L.tg, L.gate, H, F, pf_g, 2 * F, nullptr)) ||
          (rc = prep(pf_x, nullptr, H, L.ffn_norm, L.tu)) || (rc = gemm(L.tu, L.up, H, F, pf_u, 2 * F, nullptr)))
        return rc;
    }
    if ((rc = prep(pf_g, pf_u, F, nullptr, L.td, 2 * F)) || (rc = gemm(L.td, L.down, F, H, pf_x, H, pf_x))) return rc;
    last.mode = -1;
  }
  return TPT_OK;
}

// Layers [l0, l1) on caller-given residual rows (x_in, host [n][embed]) at positions pos0 ..,
// through the batched kernels (path 0) or one decode-step layer stack per position (path 1);
// the layers' K/V rows at those positions are written as a forward pass writes them.
int tpt_model::run_layers(const float* x_in, int n, int pos0, int l0, int l1, int path, float* x_out) {
  const int H = desc.embed;
  if (n <= 0 || pos0 < 0 || pos0 + n > desc.max_ctx || l0 < 0 || l1 > desc.n_layers || l0 > l1 ||
      (path != 0 && path != 1))
    return fail(TPT_ERR_INVALID, "run_layers: bad range or path");
  if (path == 0 && !batched_prefill) return fail(TPT_ERR_UNSUPPORTED, "run_layers: batched path needs Q4_K, Q5_K or Q6_K layer matrices");
  int rc;
  if (path == 0) {
    for (int c0 = 0; c0 < n; c0 += kPrefillT) {
      const int T = std::min(kPrefillT, n - c0), p0 = pos0 + c0;
      if ((rc = prefill_scratch(T, slice_chunks(p0 + T)))) return rc;
      TPT_HIP(hipMemcpyAsync(pf_x, x_in + (size_t)c0 * H, (size_t)T * H * 4, hipMemcpyHostToDevice, stream));
      if ((rc = batched_layers(T, p0, l0, l1))) return rc;
      TPT_HIP(hipMemcpyAsync(x_out + (size_t)c0 * H, pf_x, (size_t)T * H * 4, hipMemcpyDeviceToHost, stream));
      TPT_HIP(hipStreamSynchronize(stream));
    }
    return TPT_OK;
  }
  for (int t = 0; t < n; t++) {
    const int p = pos0 + t, bucket = bucket_of(p + 1);
    const int nch = std::min(attn_default_chunks(bucket, desc.n_kv_heads), attn_max_chunks);
    memset(st_host, 0, sizeof(StepState));
    st_host->pos = p;
    st_host->next_pos = p + 1;
    TPT_HIP(hipMemcpyAsync(st, st_host, sizeof(StepState), hipMemcpyHostToDevice, stream));
    TPT_HIP(hipMemcpyAsync(x, x_in + (size_t)t * H, (size_t)H * 4, hipMemcpyHostToDevice, stream));
    ssq_b_n = 0;  // x came from the host: the first RMSNorm reduces it itself
    for (int l = l0; l < l1; l++)
      if ((rc = enqueue_layer(l, nch, attn_chunk_len(bucket, nch)))) return rc;
    TPT_HIP(hipMemcpyAsync(x_out + (size_t)t * H, x, (size_t)H * 4, hipMemcpyDeviceToHost, stream));
    TPT_HIP(hipStreamSynchronize(stream));
  }
  return TPT_OK;
}

int tpt_model::prefill(const uint32_t* ids, int n, int pos0, uint32_t* next_out, float* logits_out) {
  if (n <= 0 || pos0 < 0 || pos0 + n > desc.max_ctx) return fail(TPT_ERR_INVALID, "prefill: positions out of range");
  for (int i = 0; i < n; i++)
    if (ids[i] >= (uint32_t)desc.vocab) return fail(TPT_ERR_INVALID, "prefill: token id out of vocabulary");
  memcpy(ids_host + pos0, ids, (size_t)n * 4);
  TPT_HIP(hipMemcpyAsync(prompt_dev + pos0, ids_host + pos0, (size_t)n * 4, hipMemcpyHostToDevice, stream));
  int rc;
  if (batched_prefill && n >= 2) {
    if ((rc = prefill_batched(n, pos0))) return rc;
    // LM head + greedy token of the last position, with the step state pointing at it
    memset(st_host, 0, sizeof(StepState));
    st_host->pos = pos0 + n - 1;
    st_host->next_pos = pos0 + n;
    st_host->prompt_len = pos0 + n;
    TPT_HIP(hipMemcpyAsync(st, st_host, sizeof(StepState), hipMemcpyHostToDevice, stream));
    TPT_HIP(hipStreamSynchronize(stream));  // the pinned source must not change before the copy
    GemvArgs lh;
    lh.w0 = out;
    lh.row_stride = row_bytes(out_type, desc.embed);
    lh.K = desc.embed;
    lh.N = desc.vocab;
    lh.x = x;
    lh.norm_w = out_norm;
    lh.eps = desc.rms_eps;
    lh.prologue = PRO_RMSNORM;
    lh.epilogue = EPI_ARGMAX;
    lh.y = logits;
    lh.amax = (unsigned long long*)((char*)st + offsetof(StepState, amax));
    lh.state = st;
    if ((rc = launch_gemv_q8(ctx, out_type, lh, stream))) return rc;
  } else if ((rc = prefill_steps(n, pos0))) {
    return rc;
  }
  StepState s;
  if ((rc = read_state(&s))) return rc;
  if (next_out) *next_out = (uint32_t)(s.amax[s.parity] & 0xffffffffull);
  if (logits_out) {
    TPT_HIP(hipMemcpyAsync(logits_out, logits, (size_t)desc.vocab * 4, hipMemcpyDeviceToHost, stream));
    TPT_HIP(hipStreamSynchronize(stream));
  }
  return TPT_OK;
}

int tpt_model::decode_stream(uint32_t first, int pos0, int n_steps, StepFn fn, void* user,
                             int* n_delivered) {
  *n_delivered = 0;
  if (n_steps <= 0) return TPT_OK;
  if (pos0 < 0 || pos0 + n_steps > desc.max_ctx) return fail(TPT_ERR_INVALID, "decode: positions out of range");
  if (first >= (uint32_t)desc.vocab) return fail(TPT_ERR_INVALID, "decode: token id out of vocabulary");
  int rc = set_state(pos0, 0, 1, first);
  if (rc) return rc;
  // Steps go out in batches; while batch b runs, the host reads the tokens batch b-1 produced
  // (step s's token is logged by step s+1's begin kernel) and hands them to fn in order.
  const int BATCH = 16;
  std::vector<uint32_t> log((size_t)n_steps + 1);
  std::vector<hipEvent_t> evs;
  int launched = 0, delivered = 0;
  bool stop = false;
  auto deliver = [&](int upto) -> int {  // tokens produced by steps [delivered, upto)
    if (upto > delivered) {
      TPT_HIP(hipMemcpy(log.data() + delivered, tok_log + pos0 + 1 + delivered,
                        (size_t)(upto - delivered) * 4, hipMemcpyDeviceToHost));
      for (int s = delivered; s < upto && !stop; s++) {
        delivered = s + 1;
        if (fn(user, s, log[s])) stop = true;
      }
    }
    return TPT_OK;
  };
  while (launched < n_steps && !stop) {
    const int nb = std::min(BATCH, n_steps - launched);
    for (int i = 0; i < nb && rc == TPT_OK; i++) rc = launch_step(pos0 + launched + i + 1, true);
    if (rc) break;
    launched += nb;
    hipEvent_t e;
    TPT_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    TPT_HIP(hipEventRecord(e, stream));
    evs.push_back(e);
    if (evs.size() >= 2) {
      TPT_HIP(hipEventSynchronize(evs[evs.size() - 2]));
      if ((rc = deliver(launched - nb - 1))) break;
    }
  }
  hipError_t e = hipStreamSynchronize(stream);
  for (hipEvent_t ev : evs) (void)hipEventDestroy(ev);
  if (rc) return rc;
  if (e != hipSuccess) return hip_fail(e, "decode", __FILE__, __LINE__);
  if (!stop && (rc = deliver(launched - 1))) return rc;
  if (!stop && delivered == launched - 1) {
    StepState s;
    if ((rc = read_state(&s))) return rc;
    const uint32_t last = (uint32_t)(s.amax[s.parity] & 0xffffffffull);
    delivered = launched;
    fn(user, launched - 1, last);
  }
  *n_delivered = delivered;
  return TPT_OK;
}

namespace {
struct GreedyCollect {
  uint32_t* out;
  int64_t stop;
  int n;
};
int greedy_collect(void* u, int s, uint32_t tok) {
  GreedyCollect* g = (GreedyCollect*)u;
  g->out[s] = tok;
  g->n = s + 1;
  return g->stop >= 0 && tok == (uint32_t)g->stop;
}
}  // namespace

int tpt_model::decode_greedy(uint32_t first, int pos0, int n_steps, int64_t stop_tok, uint32_t* out_tok) {
  GreedyCollect g{out_tok, stop_tok, 0};
  int delivered = 0;
  const int rc = decode_stream(first, pos0, n_steps, greedy_collect, &g, &delivered);
  return rc ? rc : g.n;
}

// ------------------------------------------------------------------ C ABI

extern "C" {

int tpt_model_load(tpt_ctx* c, const char* gguf_path, int max_ctx, int kv_type,
                   tpt_progress_fn progress, void* user, tpt_model** out) {
  int rc = ctx_enter(c);
  if (rc) return rc;
  if (!gguf_path || !out) return fail(TPT_ERR_INVALID, "null argument");
  tpt_model* m = new tpt_model();
  rc = m->load(c, gguf_path, max_ctx, kv_type, progress, user);
  if (rc) {
    delete m;
    return rc;
  }
  *out = m;
  return TPT_OK;
}

int tpt_model_inspect(const char* gguf_path, tpt_model_desc* out) {
  if (!gguf_path || !out) return fail(TPT_ERR_INVALID, "null argument");
  GgufFile f;
  int rc = f.open(gguf_path);
  if (rc) return rc;
  tpt_model_desc d{};
  ModelTensors mt;
  if ((rc = read_model_meta(f, d, mt))) return rc;
  *out = d;
  return TPT_OK;
}

int tpt_model_describe(const tpt_model* m, tpt_model_desc* out) {
  if (!m || !out) return fail(TPT_ERR_INVALID, "null argument");
  *out = m->desc;
  return TPT_OK;
}

int tpt_model_destroy(tpt_model* m) {
  delete m;
  return TPT_OK;
}

int tpt_model_prefill(tpt_model* m, const uint32_t* ids, int n, int pos0, uint32_t* next_out,
                      float* logits_out) {
  if (!m || !ids) return fail(TPT_ERR_INVALID, "null argument");
  int rc = ctx_enter(m->ctx);
  if (rc) return rc;
  return m->prefill(ids, n, pos0, next_out, logits_out);
}

int tpt_model_decode_step(tpt_model* m, uint32_t tok, int pos, uint32_t* next_out,
                          float* logits_out) {
  if (!m) return fail(TPT_ERR_INVALID, "null argument");
  int rc = ctx_enter(m->ctx);
  if (rc) return rc;
  return m->prefill(&tok, 1, pos, next_out, logits_out);
}

int tpt_model_decode_greedy(tpt_model* m, uint32_t first, int pos0, int n_steps,
                            int64_t stop_token, uint32_t* tokens_out) {
  if (!m || (!tokens_out && n_steps > 0)) return fail(TPT_ERR_INVALID, "null argument");
  int rc = ctx_enter(m->ctx);
  if (rc) return rc;
  return m->decode_greedy(first, pos0, n_steps, stop_token, tokens_out);
}

int tpt_model_run_layers(tpt_model* m, const float* x_in, int n, int pos0, int l0, int l1, int path,
                         float* x_out) {
  if (!m || !x_in || !x_out) return fail(TPT_ERR_INVALID, "null argument");
  int rc = ctx_enter(m->ctx);
  if (rc) return rc;
  return m->run_layers(x_in, n, pos0, l0, l1, path, x_out);
}

int tpt_model_kv_read(tpt_model* m, int layer, void* k_host, void* v_host) {
  if (!m || !k_host || !v_host) return fail(TPT_ERR_INVALID, "null argument");
  if (layer < 0 || layer >= m->desc.n_layers) return fail(TPT_ERR_INVALID, "kv_read: layer out of range");
  int rc = ctx_enter(m->ctx);
  if (rc) return rc;
  const size_t half = (size_t)m->desc.n_kv_heads * m->desc.max_ctx * m->desc.head_dim * m->kv_elem;
  const uint8_t* kc = (const uint8_t*)m->kv + (size_t)layer * 2 * half;
  TPT_HIP(hipMemcpyAsync(k_host, kc, half, hipMemcpyDeviceToHost, m->stream));
  TPT_HIP(hipMemcpyAsync(v_host, kc + half, half, hipMemcpyDeviceToHost, m->stream));
  TPT_HIP(hipStreamSynchronize(m->stream));
  return TPT_OK;
}

int tpt_model_set_decode_path(tpt_model* m, int path) {
  if (!m) return fail(TPT_ERR_INVALID, "null argument");
  int rc = ctx_enter(m->ctx);
  if (rc) return rc;
  return m->set_decode_path(path);
}

int tpt_model_get_decode_path(const tpt_model* m, int* path) {
  if (!m || !path) return fail(TPT_ERR_INVALID, "null argument");
  *path = TPT_DECODE_KERNELS;
  return TPT_OK;
}

int tpt_model_hidden(tpt_model* m, float* out_host) {
  if (!m || !out_host) return fail(TPT_ERR_INVALID, "null argument");
  int rc = ctx_enter(m->ctx);
  if (rc) return rc;
  TPT_HIP(hipMemcpyAsync(out_host, m->x, (size_t)m->desc.embed * 4, hipMemcpyDeviceToHost, m->stream));
  TPT_HIP(hipStreamSynchronize(m->stream));
  return TPT_OK;
}

}  // extern "C"
