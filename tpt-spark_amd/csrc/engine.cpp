// engine-hip: the LlmEngine mirror over the model (src-tauri/src/engine/mod.rs:62-82).
//
// infer() follows the reference engines' loop (candle_engine.rs:231-334 for the sampling and
// stop rules, wgpu_engine.rs:186-334 for prompt truncation and multi-turn KV prefix reuse):
//   1. front-truncate the prompt to context_length - max_tokens (truncation resets the cache);
//   2. reuse the longest common prefix with the tokens whose K/V are resident
//      (KvCache::common_prefix_len, wgpu_kvcache.rs:63-69), always recomputing at least the
//      last prompt position so its logits exist;
//   3. prefill the rest, sample the first token;
//   4. loop: stop on EOS / max_tokens / context limit, emit the token, feed it, sample.
// Greedy decoding (temperature <= 0, repeat_penalty == 1: run_benchmark's parameters,
// commands.rs:518-525) keeps the argmax on the GPU and pipelines steps through captured HIP
// graphs.  Other settings copy the logits to the host each step for the repeat penalty
// (candle_engine.rs:87-101, one application per occurrence) and temperature / top-p sampling.
#include <math.h>
#include <stdio.h>
#include <string.h>
#include <sys/stat.h>

#include <algorithm>
#include <chrono>
#include <numeric>
#include <string>
#include <vector>

#include "model.h"

using namespace tpt;

struct tpt_engine {
  tpt_ctx* ctx = nullptr;
  tpt_model* model = nullptr;
  tpt_model_info info{};
  std::vector<uint32_t> cached_tokens;  // tokens whose K/V occupy positions [0, n)
  int kv_type = TPT_TYPE_F16;
};

namespace {

using Clock = std::chrono::steady_clock;
double ms_since(Clock::time_point t) {
  return std::chrono::duration<double, std::milli>(Clock::now() - t).count();
}

size_t common_prefix(const std::vector<uint32_t>& a, const std::vector<uint32_t>& b) {
  size_t n = 0;
  while (n < a.size() && n < b.size() && a[n] == b[n]) n++;
  return n;
}

// apply_repeat_penalty (candle_engine.rs:87-101)
void repeat_penalty(std::vector<float>& logits, const std::vector<uint32_t>& seen, float p) {
  if (fabsf(p - 1.f) < 1.1920929e-07f) return;
  for (uint32_t id : seen)
    if (id < logits.size()) logits[id] = logits[id] >= 0.f ? logits[id] / p : logits[id] * p;
}

// f32::total_cmp argmax, last index wins (LogitsProcessor::sample_argmax)
uint32_t host_argmax(const std::vector<float>& v) {
  auto key = [](float f) {
    int32_t b;
    memcpy(&b, &f, 4);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
  };
  size_t best = 0;
  int32_t bk = key(v[0]);
  for (size_t i = 1; i < v.size(); i++) {
    const int32_t k = key(v[i]);
    if (k >= bk) {
      bk = k;
      best = i;
    }
  }
  return (uint32_t)best;
}

struct Rng {  // splitmix64; temperature sampling only (not candle's StdRng stream)
  uint64_t s;
  double uniform() {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (double)(z >> 11) * (1.0 / 9007199254740992.0);
  }
};

// LogitsProcessor::sample with Some(temperature) [and Some(top_p)]: softmax(logits / T),
// optional nucleus truncation (probabilities past cumulative top_p zeroed), multinomial draw.
uint32_t sample(std::vector<float>& logits, float temperature, float top_p, Rng& rng) {
  if (temperature <= 0.f) return host_argmax(logits);
  const size_t n = logits.size();
  float mx = -INFINITY;
  for (float& l : logits) {
    l /= temperature;
    mx = std::max(mx, l);
  }
  std::vector<float> pr(n);
  double sum = 0;
  for (size_t i = 0; i < n; i++) sum += (pr[i] = expf(logits[i] - mx));
  for (float& p : pr) p = (float)(p / sum);
  if (top_p < 1.f) {
    std::vector<uint32_t> idx(n);
    std::iota(idx.begin(), idx.end(), 0u);
    std::sort(idx.begin(), idx.end(), [&](uint32_t a, uint32_t b) { return pr[a] > pr[b]; });
    float cum = 0.f;
    for (uint32_t i : idx) {
      if (cum >= top_p) pr[i] = 0.f;
      else cum += pr[i];
    }
  }
  double tot = 0;
  for (float p : pr) tot += p;
  double u = rng.uniform() * tot, c = 0;
  for (size_t i = 0; i < n; i++) {
    c += pr[i];
    if (u < c) return (uint32_t)i;
  }
  return (uint32_t)(n - 1);
}

struct GreedyLoop {
  tpt_engine* e;
  const tpt_infer_params* p;
  tpt_token_fn cb;
  void* user;
  std::vector<uint32_t>* tokens;
  uint32_t generated = 0;
  size_t pos = 0;
  int ctx_len = 0;
  bool cancelled = false;
  Clock::time_point t_first;
  bool first_seen = false;
  // the candle_engine loop body for one sampled token; returns 1 to stop
  int take(uint32_t tok) {
    if (p->eos_token_id >= 0 && tok == (uint32_t)p->eos_token_id) return 1;
    if (generated >= p->max_tokens) return 1;
    if (pos >= (size_t)ctx_len) return 1;
    if (!first_seen) {
      first_seen = true;
      t_first = Clock::now();
    }
    if (cb(user, tok, 0)) {
      cancelled = true;
      return 1;
    }
    tokens->push_back(tok);
    e->cached_tokens.push_back(tok);
    generated++;
    pos++;
    return 0;
  }
  static int step_fn(void* u, int, uint32_t tok) { return ((GreedyLoop*)u)->take(tok); }
};

}  // namespace

extern "C" {

int tpt_engine_create(int device, tpt_engine** out) {
  if (!out) return fail(TPT_ERR_INVALID, "null out pointer");
  tpt_engine* e = new tpt_engine();
  int rc = tpt_ctx_create(device, &e->ctx);
  if (rc) {
    delete e;
    return rc;
  }
  *out = e;
  return TPT_OK;
}

int tpt_engine_set_kv_type(tpt_engine* e, int kv_type) {
  if (!e) return fail(TPT_ERR_INVALID, "null engine");
  if (kv_type != TPT_TYPE_F16 && kv_type != TPT_TYPE_F32)
    return fail(TPT_ERR_UNSUPPORTED, "KV cache type must be F16 or F32");
  e->kv_type = kv_type;
  return TPT_OK;
}

int tpt_engine_destroy(tpt_engine* e) {
  if (!e) return TPT_OK;
  tpt_engine_unload(e);
  tpt_ctx_destroy(e->ctx);
  delete e;
  return TPT_OK;
}

int tpt_engine_load(tpt_engine* e, const char* model_path, tpt_progress_fn progress, void* user,
                    tpt_model_info* info_out) {
  if (!e || !model_path) return fail(TPT_ERR_INVALID, "null argument");
  tpt_engine_unload(e);  // free the previous model's HBM before allocating the next
  tpt_model* m = nullptr;
  int rc = tpt_model_load(e->ctx, model_path, 0, e->kv_type, progress, user, &m);
  if (rc) return rc;
  e->model = m;
  e->cached_tokens.clear();
  tpt_model_info& inf = e->info;
  memset(&inf, 0, sizeof inf);
  std::string p = model_path, stem = p.substr(p.find_last_of('/') == std::string::npos ? 0 : p.find_last_of('/') + 1);
  const size_t dot = stem.find_last_of('.');
  if (dot != std::string::npos && dot > 0) stem = stem.substr(0, dot);
  snprintf(inf.name, sizeof inf.name, "%s", stem.c_str());
  snprintf(inf.path, sizeof inf.path, "%s", model_path);
  struct stat st;
  inf.size_bytes = stat(model_path, &st) == 0 ? (uint64_t)st.st_size : 0;
  // backend string like "wgpu-vulkan" / "candle-cpu" (wgpu_engine.rs:102, candle_engine.rs:177)
  std::string arch = e->ctx->name;
  const size_t lp = arch.find('('), rp = arch.find(')');
  arch = lp != std::string::npos && rp != std::string::npos ? arch.substr(lp + 1, rp - lp - 1) : "gfx";
  const size_t colon = arch.find(':');
  if (colon != std::string::npos) arch = arch.substr(0, colon);
  snprintf(inf.backend, sizeof inf.backend, "hip-%s", arch.c_str());
  if (info_out) *info_out = inf;
  return TPT_OK;
}

int tpt_engine_unload(tpt_engine* e) {
  if (!e) return fail(TPT_ERR_INVALID, "null engine");
  if (e->model) {
    ctx_enter(e->ctx);
    tpt_model_destroy(e->model);  // frees HBM immediately (wgpu_engine.rs:126-136)
    e->model = nullptr;
  }
  e->cached_tokens.clear();
  memset(&e->info, 0, sizeof e->info);
  return TPT_OK;
}

int tpt_engine_is_loaded(const tpt_engine* e) { return e && e->model ? 1 : 0; }

int tpt_engine_model_info(const tpt_engine* e, tpt_model_info* info_out) {
  if (!e || !info_out) return fail(TPT_ERR_INVALID, "null argument");
  if (!e->model) return fail(TPT_ERR_STATE, "no model loaded");
  *info_out = e->info;
  return TPT_OK;
}

size_t tpt_common_prefix_len(const uint32_t* a, size_t na, const uint32_t* b, size_t nb) {
  if (!a || !b) return 0;
  size_t n = 0;
  while (n < na && n < nb && a[n] == b[n]) n++;
  return n;
}

int tpt_engine_cached_prefix(const tpt_engine* e, const uint32_t* tokens, size_t n, size_t* out) {
  if (!e || !out || (!tokens && n)) return fail(TPT_ERR_INVALID, "null argument");
  std::vector<uint32_t> t(tokens, tokens + n);
  *out = common_prefix(e->cached_tokens, t);
  return TPT_OK;
}

int tpt_engine_reset_cache(tpt_engine* e) {
  if (!e) return fail(TPT_ERR_INVALID, "null engine");
  e->cached_tokens.clear();
  return TPT_OK;
}

int tpt_engine_infer(tpt_engine* e, const tpt_infer_params* p, const uint32_t* prompt,
                     size_t n_prompt, tpt_token_fn on_token, void* user, tpt_infer_stats* stats) {
  if (!e || !p || !on_token || (!prompt && n_prompt)) return fail(TPT_ERR_INVALID, "null argument");
  if (!e->model) return fail(TPT_ERR_STATE, "no model loaded");
  int rc = ctx_enter(e->ctx);
  if (rc) return rc;
  tpt_model* m = e->model;
  const int ctx_len = m->desc.max_ctx;
  const Clock::time_point t0 = Clock::now();
  tpt_infer_stats S{};

  std::vector<uint32_t> tokens(prompt, prompt + n_prompt);
  for (uint32_t t : tokens)
    if (t >= (uint32_t)m->desc.vocab) return fail(TPT_ERR_INVALID, "prompt token id out of vocabulary");
  const size_t max_prompt = (size_t)std::max<int64_t>(0, (int64_t)ctx_len - (int64_t)p->max_tokens);
  if (tokens.size() > max_prompt) {
    tokens.erase(tokens.begin(), tokens.end() - (ptrdiff_t)max_prompt);
    e->cached_tokens.clear();  // truncation breaks position alignment
  }
  if (tokens.empty()) return fail(TPT_ERR_INVALID, "Prompt is empty after tokenization");

  size_t prefix = common_prefix(e->cached_tokens, tokens);
  if (prefix == 0) e->cached_tokens.clear();
  if (prefix >= tokens.size()) prefix = tokens.size() - 1;  // recompute the last position's logits
  S.prompt_tokens = (uint32_t)tokens.size();
  S.cached_prefix = (uint32_t)prefix;

  const bool greedy = p->temperature <= 0.f && fabsf(p->repeat_penalty - 1.f) < 1.1920929e-07f;
  Rng rng{p->seed};
  std::vector<float> logits;
  uint32_t next = 0;
  e->cached_tokens.assign(tokens.begin(), tokens.begin() + (ptrdiff_t)prefix);
  if (greedy) {
    rc = tpt_model_prefill(m, tokens.data() + prefix, (int)(tokens.size() - prefix), (int)prefix, &next, nullptr);
  } else {
    logits.resize((size_t)m->desc.vocab);
    rc = tpt_model_prefill(m, tokens.data() + prefix, (int)(tokens.size() - prefix), (int)prefix, &next, logits.data());
    if (rc == TPT_OK) {
      repeat_penalty(logits, tokens, p->repeat_penalty);
      next = sample(logits, p->temperature, p->top_p, rng);
    }
  }
  if (rc) {
    e->cached_tokens.clear();
    return rc;
  }
  e->cached_tokens = tokens;
  S.prefill_ms = ms_since(t0);

  GreedyLoop lp;
  lp.e = e;
  lp.p = p;
  lp.cb = on_token;
  lp.user = user;
  lp.tokens = &tokens;
  lp.pos = tokens.size();
  lp.ctx_len = ctx_len;
  if (lp.take(next) == 0) {
    if (greedy) {
      const int n_steps = (int)std::min<int64_t>((int64_t)p->max_tokens, (int64_t)ctx_len - (int64_t)(lp.pos - 1));
      int delivered = 0;
      // step s feeds the token emitted s-th (at position pos0 + s) and hands back the next
      rc = m->decode_stream(next, (int)(lp.pos - 1), n_steps, GreedyLoop::step_fn, &lp, &delivered);
    } else {
      uint32_t cur = next;
      while (true) {
        rc = tpt_model_decode_step(m, cur, (int)(lp.pos - 1), nullptr, logits.data());
        if (rc) break;
        repeat_penalty(logits, tokens, p->repeat_penalty);
        cur = sample(logits, p->temperature, p->top_p, rng);
        if (lp.take(cur)) break;
      }
    }
  }
  S.generated = lp.generated;
  S.ttft_ms = lp.first_seen ? std::chrono::duration<double, std::milli>(lp.t_first - t0).count() : S.prefill_ms;
  S.decode_ms = lp.first_seen ? ms_since(lp.t_first) : 0.0;
  if (stats) *stats = S;
  if (rc) {
    e->cached_tokens.clear();
    return rc;
  }
  if (lp.cancelled) {
    on_token(user, 0, 1);  // done:true before propagating the cancel (wgpu_engine.rs:297-300)
    return fail(TPT_ERR_CANCELLED, "inference cancelled");
  }
  on_token(user, 0, 1);
  return TPT_OK;
}

}  // extern "C"
