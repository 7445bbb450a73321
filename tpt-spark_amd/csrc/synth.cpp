// Synthetic workload generator (host only; libtptsynth.so): seeded random-init Llama GGUF
// files and k-quant quantizers for the GEMV workloads.
//
// The reference ships no model files or fixtures, so the workloads are generated: weights
// ~ N(0, std) (std 0.02), norm weights 1.0, matrices quantized to Q4_K / Q6_K / Q8_0 in ggml's
// block layouts.  Draws are counter-based (tensor-name hash, element index), so a file is a
// pure function of (config, seed): any thread count on any host that runs this build writes
// the same bytes.  The quantizers are this project's own min/max fits (not ggml's iterative
// make_qkx2_quants search); any valid blocks serve, because every consumer -- the oracle and
// the GPU engine -- reads the stored blocks, not the pre-quantization floats.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <unistd.h>

#include <algorithm>
#include <string>
#include <thread>
#include <vector>

namespace {

enum { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14 };

int blk_elems(int t) { return t == T_Q4_K || t == T_Q5_K || t == T_Q6_K ? 256 : t == T_Q8_0 || t == T_Q4_0 ? 32 : 1; }
int blk_bytes(int t) {
  return t == T_Q4_K ? 144 : t == T_Q5_K ? 176 : t == T_Q6_K ? 210 : t == T_Q8_0 ? 34 : t == T_Q4_0 ? 18 : t == T_F16 ? 2 : 4;
}

uint16_t f32_to_f16(float v) {  // round to nearest even
  uint32_t x;
  memcpy(&x, &v, 4);
  const uint32_t sign = (x >> 16) & 0x8000, exp = (x >> 23) & 0xff, man = x & 0x7fffff;
  if (exp == 0xff) return (uint16_t)(sign | 0x7c00 | (man ? 0x200 : 0));
  const int32_t e = (int32_t)exp - 112;
  if (e >= 0x1f) return (uint16_t)(sign | 0x7c00);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    const uint32_t m = man | 0x800000, sh = (uint32_t)(14 - e);
    uint32_t h = m >> sh;
    const uint32_t rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
    if (rem > half || (rem == half && (h & 1))) h++;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1fff;
  if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) h++;
  return (uint16_t)(sign | h);
}

float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31, exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ff, f;
  if (exp == 0) {
    if (!man) f = sign;
    else {
      int k = 0;
      while (!(man & 0x400)) { man <<= 1; k++; }
      f = sign | ((uint32_t)(113 - k) << 23) | ((man & 0x3ff) << 13);
    }
  } else if (exp == 31) f = sign | 0x7f800000u | (man << 13);
  else f = sign | ((exp + 112) << 23) | (man << 13);
  float r;
  memcpy(&r, &f, 4);
  return r;
}

inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t name_hash(const char* s) {  // FNV-1a
  uint64_t h = 0xcbf29ce484222325ull;
  for (; *s; s++) h = (h ^ (uint8_t)*s) * 0x100000001b3ull;
  return h;
}

// N(0,1) draws for elements [i0, i0+n) of stream `key` (Box-Muller on 24-bit uniforms; element
// 2k and 2k+1 share pair k).
void normals(uint64_t key, int64_t i0, int64_t n, float std, float* out) {
  for (int64_t i = i0; i < i0 + n; i++) {
    const uint64_t h = mix64(key + 0x9E3779B97F4A7C15ull * (uint64_t)(i >> 1));
    const float u1 = ((float)(h >> 40) + 0.5f) * (1.f / 16777216.f);
    const float u2 = ((float)((h >> 16) & 0xFFFFFF) + 0.5f) * (1.f / 16777216.f);
    const float r = sqrtf(-2.f * logf(u1));
    const float a = 6.2831853071795864f * u2;
    out[i - i0] = std * r * ((i & 1) ? sinf(a) : cosf(a));
  }
}

int nearest(float v) { return (int)lrintf(v); }

// ---- Q4_K: 8 sub-blocks of 32, per-sub-block scale and min (6-bit) under f16 d / dmin
void quant_q4k(const float* x, uint8_t* out) {
  float scale[8], mn[8];
  for (int j = 0; j < 8; j++) {
    float lo = x[32 * j], hi = x[32 * j];
    for (int l = 1; l < 32; l++) {
      lo = std::min(lo, x[32 * j + l]);
      hi = std::max(hi, x[32 * j + l]);
    }
    lo = std::min(lo, 0.f);
    scale[j] = (hi - lo) / 15.f;
    mn[j] = -lo;
  }
  float ms = 0, mm = 0;
  for (int j = 0; j < 8; j++) {
    ms = std::max(ms, scale[j]);
    mm = std::max(mm, mn[j]);
  }
  const uint16_t dh = f32_to_f16(ms / 63.f), mh = f32_to_f16(mm / 63.f);
  const float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
  int sc[8], m[8];
  for (int j = 0; j < 8; j++) {
    sc[j] = d > 0 ? std::min(63, std::max(0, nearest(scale[j] / d))) : 0;
    m[j] = dmin > 0 ? std::min(63, std::max(0, nearest(mn[j] / dmin))) : 0;
  }
  uint8_t* s = out + 4;
  memcpy(out, &dh, 2);
  memcpy(out + 2, &mh, 2);
  for (int j = 0; j < 4; j++) {
    s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
    s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
    s[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
  }
  uint8_t q[256];
  for (int j = 0; j < 8; j++) {
    const float ds = d * (float)sc[j], dm = dmin * (float)m[j];
    for (int l = 0; l < 32; l++) {
      const int v = ds > 0 ? nearest((x[32 * j + l] + dm) / ds) : 0;
      q[32 * j + l] = (uint8_t)std::min(15, std::max(0, v));
    }
  }
  uint8_t* qs = out + 16;
  for (int g = 0; g < 4; g++)
    for (int l = 0; l < 32; l++) qs[32 * g + l] = (uint8_t)(q[64 * g + l] | (q[64 * g + 32 + l] << 4));
}

// ---- Q5_K: Q4_K's scales with 5-bit values (31 levels); the fifth bits go to qh (bit 2g of
// qh[l] for element 64g + l, bit 2g + 1 for element 64g + 32 + l)
void quant_q5k(const float* x, uint8_t* out) {
  float scale[8], mn[8];
  for (int j = 0; j < 8; j++) {
    float lo = x[32 * j], hi = x[32 * j];
    for (int l = 1; l < 32; l++) {
      lo = std::min(lo, x[32 * j + l]);
      hi = std::max(hi, x[32 * j + l]);
    }
    lo = std::min(lo, 0.f);
    scale[j] = (hi - lo) / 31.f;
    mn[j] = -lo;
  }
  float ms = 0, mm = 0;
  for (int j = 0; j < 8; j++) {
    ms = std::max(ms, scale[j]);
    mm = std::max(mm, mn[j]);
  }
  const uint16_t dh = f32_to_f16(ms / 63.f), mh = f32_to_f16(mm / 63.f);
  const float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
  int sc[8], m[8];
  for (int j = 0; j < 8; j++) {
    sc[j] = d > 0 ? std::min(63, std::max(0, nearest(scale[j] / d))) : 0;
    m[j] = dmin > 0 ? std::min(63, std::max(0, nearest(mn[j] / dmin))) : 0;
  }
  uint8_t* s = out + 4;
  memcpy(out, &dh, 2);
  memcpy(out + 2, &mh, 2);
  for (int j = 0; j < 4; j++) {
    s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
    s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
    s[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
  }
  uint8_t q[256];
  for (int j = 0; j < 8; j++) {
    const float ds = d * (float)sc[j], dm = dmin * (float)m[j];
    for (int l = 0; l < 32; l++) {
      const int v = ds > 0 ? nearest((x[32 * j + l] + dm) / ds) : 0;
      q[32 * j + l] = (uint8_t)std::min(31, std::max(0, v));
    }
  }
  uint8_t* qh = out + 16;
  uint8_t* qs = out + 48;
  memset(qh, 0, 32);
  for (int g = 0; g < 4; g++)
    for (int l = 0; l < 32; l++) {
      const int lo = q[64 * g + l], hi = q[64 * g + 32 + l];
      qs[32 * g + l] = (uint8_t)((lo & 15) | ((hi & 15) << 4));
      qh[l] |= (uint8_t)(((lo >> 4) << (2 * g)) | ((hi >> 4) << (2 * g + 1)));
    }
}

// ---- Q4_0: per 32, d = (signed value of the largest magnitude) / -8, q = x / d + 8 in [0, 15];
// element j < 16 in the low nibble of qs[j], element j + 16 in its high nibble
void quant_q4_0(const float* x, uint8_t* out) {
  float amax = 0, mx = 0;
  for (int l = 0; l < 32; l++)
    if (fabsf(x[l]) > amax) {
      amax = fabsf(x[l]);
      mx = x[l];
    }
  const uint16_t dh = f32_to_f16(mx / -8.f);
  const float d = f16_to_f32(dh), id = d != 0.f ? 1.f / d : 0.f;
  memcpy(out, &dh, 2);
  for (int j = 0; j < 16; j++) {
    const int a = std::min(15, std::max(0, (int)(x[j] * id + 8.5f)));
    const int b = std::min(15, std::max(0, (int)(x[j + 16] * id + 8.5f)));
    out[2 + j] = (uint8_t)(a | (b << 4));
  }
}

// ---- Q6_K: 16 sub-blocks of 16, int8 scales under an f16 d, 6-bit q - 32
void quant_q6k(const float* x, uint8_t* out) {
  float s[16];
  float smax = 0;
  for (int j = 0; j < 16; j++) {
    float a = 0;
    for (int l = 0; l < 16; l++) a = std::max(a, fabsf(x[16 * j + l]));
    s[j] = a / 31.f;
    smax = std::max(smax, s[j]);
  }
  const uint16_t dh = f32_to_f16(smax / 127.f);
  const float d = f16_to_f32(dh);
  int8_t sc[16];
  for (int j = 0; j < 16; j++) sc[j] = (int8_t)(d > 0 ? std::min(127, std::max(-128, nearest(s[j] / d))) : 0);
  uint8_t q[256];
  for (int i = 0; i < 256; i++) {
    const float ds = d * (float)sc[i / 16];
    const int v = ds != 0 ? nearest(x[i] / ds) : 0;
    q[i] = (uint8_t)(std::min(31, std::max(-32, v)) + 32);
  }
  uint8_t* ql = out;
  uint8_t* qh = out + 128;
  for (int p = 0; p < 2; p++)
    for (int l = 0; l < 32; l++) {
      const uint8_t q1 = q[128 * p + l], q2 = q[128 * p + l + 32], q3 = q[128 * p + l + 64],
                    q4 = q[128 * p + l + 96];
      ql[64 * p + l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
      ql[64 * p + l + 32] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
      qh[32 * p + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
    }
  memcpy(out + 192, sc, 16);
  memcpy(out + 208, &dh, 2);
}

// ---- Q8_0: d = amax/127 (stored f16), q = round(x / d)
void quant_q8_0(const float* x, uint8_t* out) {
  float a = 0;
  for (int l = 0; l < 32; l++) a = std::max(a, fabsf(x[l]));
  const float d = a / 127.f, id = d > 0 ? 1.f / d : 0.f;
  const uint16_t dh = f32_to_f16(d);
  memcpy(out, &dh, 2);
  for (int l = 0; l < 32; l++) out[2 + l] = (uint8_t)(int8_t)std::min(127, std::max(-127, nearest(x[l] * id)));
}

int quantize(int type, const float* x, int64_t n, uint8_t* out) {
  const int be = blk_elems(type), bb = blk_bytes(type);
  if (n % be) return -1;
  for (int64_t b = 0; b < n / be; b++) {
    const float* xs = x + b * be;
    uint8_t* o = out + b * bb;
    switch (type) {
      case T_Q4_K: quant_q4k(xs, o); break;
      case T_Q5_K: quant_q5k(xs, o); break;
      case T_Q4_0: quant_q4_0(xs, o); break;
      case T_Q6_K: quant_q6k(xs, o); break;
      case T_Q8_0: quant_q8_0(xs, o); break;
      case T_F32: memcpy(o, xs, 4); break;
      case T_F16: { uint16_t h = f32_to_f16(xs[0]); memcpy(o, &h, 2); } break;
      default: return -2;
    }
  }
  return 0;
}

// ---- GGUF writer
struct Buf {
  std::vector<uint8_t> b;
  void raw(const void* p, size_t n) { b.insert(b.end(), (const uint8_t*)p, (const uint8_t*)p + n); }
  void u32(uint32_t v) { raw(&v, 4); }
  void u64(uint64_t v) { raw(&v, 8); }
  void f32(float v) { raw(&v, 4); }
  void str(const std::string& s) { u64(s.size()); raw(s.data(), s.size()); }
  void kv_u32(const std::string& k, uint32_t v) { str(k); u32(4); u32(v); }
  void kv_f32(const std::string& k, float v) { str(k); u32(6); f32(v); }
  void kv_str(const std::string& k, const std::string& v) { str(k); u32(8); str(v); }
};

struct TensorSpec {
  std::string name;
  int type;
  int64_t ne0, ne1;  // ne1 = 1 for vectors
  int init;          // 0 = normal(std), 1 = ones
  uint64_t offset;
  size_t bytes;
};

}  // namespace

extern "C" {

typedef struct {
  int n_layers, embed, n_heads, n_kv_heads, ffn, vocab, context_length;
  float rope_base, rms_eps, init_std;
  int type_matrix, type_embd, type_out;
  uint32_t eos_token_id;
  // nonzero: attn_v and ffn_down of the layers llama.cpp's Q4_K_M recipe gives more bits
  // (the first and last eighth of the layers and every third layer between) get this type
  int type_more_bits;
} tpt_synth_cfg;

// Quantize n floats (a whole number of blocks) into GGUF blocks of `type`.
int tpt_synth_quantize(int type, const float* x, int64_t n, void* out) {
  return quantize(type, x, n, (uint8_t*)out);
}

// The generator's N(0, std) draws for elements [i0, i0+n) of the stream named `name`.
void tpt_synth_normal(uint64_t seed, const char* name, int64_t i0, int64_t n, float std, float* out) {
  normals(mix64(seed ^ name_hash(name)), i0, n, std, out);
}

// Write a random-init Llama GGUF (v3).  Returns 0 or a negative error.
int tpt_synth_write_llama(const char* path, const tpt_synth_cfg* c, uint64_t seed, int nthreads) {
  if (!path || !c || c->embed % 256 || c->ffn % 256 || c->n_heads <= 0 || c->embed % c->n_heads ||
      c->n_kv_heads <= 0 || c->n_heads % c->n_kv_heads)
    return -1;
  const int64_t H = c->embed, hd = H / c->n_heads, qd = H, kd = c->n_kv_heads * hd, F = c->ffn,
                V = c->vocab;
  std::vector<TensorSpec> ts;
  auto add = [&](const std::string& n, int t, int64_t ne0, int64_t ne1, int init) {
    ts.push_back({n, t, ne0, ne1, init, 0, 0});
  };
  add("token_embd.weight", c->type_embd, H, V, 0);
  add("output_norm.weight", T_F32, H, 1, 1);
  add("output.weight", c->type_out, H, V, 0);
  const int nl = c->n_layers;
  for (int l = 0; l < nl; l++) {
    const std::string p = "blk." + std::to_string(l) + ".";
    const bool more = c->type_more_bits && (l < nl / 8 || l >= 7 * nl / 8 || (l - nl / 8) % 3 == 2);
    const int tvd = more ? c->type_more_bits : c->type_matrix;
    add(p + "attn_norm.weight", T_F32, H, 1, 1);
    add(p + "attn_q.weight", c->type_matrix, H, qd, 0);
    add(p + "attn_k.weight", c->type_matrix, H, kd, 0);
    add(p + "attn_v.weight", tvd, H, kd, 0);
    add(p + "attn_output.weight", c->type_matrix, qd, H, 0);
    add(p + "ffn_norm.weight", T_F32, H, 1, 1);
    add(p + "ffn_gate.weight", c->type_matrix, H, F, 0);
    add(p + "ffn_up.weight", c->type_matrix, H, F, 0);
    add(p + "ffn_down.weight", tvd, F, H, 0);
  }
  const uint64_t ALIGN = 32;
  uint64_t off = 0;
  for (auto& t : ts) {
    if (t.ne0 % blk_elems(t.type)) return -2;
    t.bytes = (size_t)(t.ne0 / blk_elems(t.type)) * blk_bytes(t.type) * (size_t)t.ne1;
    off = (off + ALIGN - 1) / ALIGN * ALIGN;
    t.offset = off;
    off += t.bytes;
  }
  Buf h;
  h.u32(0x46554747u);
  h.u32(3);
  h.u64(ts.size());
  h.u64(13);
  h.kv_str("general.architecture", "llama");
  h.kv_str("general.name", "tpt-synthetic-llama");
  h.kv_u32("general.alignment", (uint32_t)ALIGN);
  h.kv_u32("llama.context_length", (uint32_t)c->context_length);
  h.kv_u32("llama.embedding_length", (uint32_t)H);
  h.kv_u32("llama.block_count", (uint32_t)c->n_layers);
  h.kv_u32("llama.feed_forward_length", (uint32_t)F);
  h.kv_u32("llama.attention.head_count", (uint32_t)c->n_heads);
  h.kv_u32("llama.attention.head_count_kv", (uint32_t)c->n_kv_heads);
  h.kv_u32("llama.rope.dimension_count", (uint32_t)hd);
  h.kv_f32("llama.rope.freq_base", c->rope_base);
  h.kv_f32("llama.attention.layer_norm_rms_epsilon", c->rms_eps);
  h.kv_u32("llama.vocab_size", (uint32_t)V);
  for (auto& t : ts) {
    h.str(t.name);
    const bool vec = t.ne1 == 1 && t.type == T_F32;
    h.u32(vec ? 1 : 2);
    h.u64((uint64_t)t.ne0);
    if (!vec) h.u64((uint64_t)t.ne1);
    h.u32((uint32_t)t.type);
    h.u64(t.offset);
  }
  const uint64_t data0 = (h.b.size() + ALIGN - 1) / ALIGN * ALIGN;
  const uint64_t total = data0 + off;
  const int fd = open(path, O_RDWR | O_CREAT | O_TRUNC, 0644);
  if (fd < 0) return -3;
  if (ftruncate(fd, (off_t)total) != 0) {
    close(fd);
    return -3;
  }
  uint8_t* map = (uint8_t*)mmap(nullptr, total, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
  close(fd);
  if (map == MAP_FAILED) return -3;
  memcpy(map, h.b.data(), h.b.size());
  memset(map + h.b.size(), 0, data0 - h.b.size());
  if (nthreads <= 0) nthreads = (int)std::max(1u, std::thread::hardware_concurrency());
  for (const auto& t : ts) {
    uint8_t* dst = map + data0 + t.offset;
    if (t.init == 1) {
      std::vector<float> ones((size_t)(t.ne0 * t.ne1), 1.f);
      quantize(t.type, ones.data(), t.ne0 * t.ne1, dst);
      continue;
    }
    const uint64_t key = mix64(seed ^ name_hash(t.name.c_str()));
    const int be = blk_elems(t.type), bb = blk_bytes(t.type);
    const int64_t nblk = t.ne0 * t.ne1 / be;
    // 256 elements per work unit for every type (Q8_0: 8 blocks)
    const int per = 256 / be;
    const int64_t units = nblk / per;
    auto work = [&](int tid) {
      float buf[256];
      for (int64_t u = (int64_t)tid * units / nthreads; u < (int64_t)(tid + 1) * units / nthreads; u++) {
        normals(key, u * 256, 256, c->init_std, buf);
        quantize(t.type, buf, 256, dst + (size_t)u * per * bb);
      }
    };
    std::vector<std::thread> th;
    for (int i = 0; i < nthreads; i++) th.emplace_back(work, i);
    for (auto& x : th) x.join();
  }
  munmap(map, total);  // the page cache holds the bytes for any reader that opens the file
  return 0;
}

}  // extern "C"
