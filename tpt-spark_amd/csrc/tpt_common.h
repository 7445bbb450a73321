// Shared definitions of libtpthip: GGUF block layouts, device helpers, error plumbing.
// All device code is compiled for gfx950 with -ffp-contract=off; fused multiply-adds are
// written out explicitly (fmaf) where they are wanted, so every non-FMA expression keeps
// the rounding of the CPU arithmetic it restates.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <string>

#include "../../include/tpthip.h"

namespace tpt {

constexpr int QK_K = 256;
constexpr int QK8_0 = 32;
constexpr int WAVE = 64;

// ggml block layouts (bytes are uploaded unchanged; these describe them).
struct __attribute__((packed)) BlockQ4K { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; };
struct __attribute__((packed)) BlockQ6K { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; };
struct __attribute__((packed)) BlockQ8_0 { uint16_t d; int8_t qs[32]; };
static_assert(sizeof(BlockQ4K) == 144, "q4k");
static_assert(sizeof(BlockQ6K) == 210, "q6k");
static_assert(sizeof(BlockQ8_0) == 34, "q8_0");

__host__ __device__ inline int type_block(int t) {
  return t == TPT_TYPE_Q4_K || t == TPT_TYPE_Q5_K || t == TPT_TYPE_Q6_K ? QK_K
         : t == TPT_TYPE_Q8_0 || t == TPT_TYPE_Q4_0 ? QK8_0 : 1;
}
__host__ __device__ inline int type_bytes(int t) {
  return t == TPT_TYPE_Q4_K ? 144 : t == TPT_TYPE_Q5_K ? 176 : t == TPT_TYPE_Q6_K ? 210
         : t == TPT_TYPE_Q8_0 ? 34 : t == TPT_TYPE_Q4_0 ? 18
         : t == TPT_TYPE_F16 ? 2 : t == TPT_TYPE_F32 ? 4 : 0;
}
inline size_t row_bytes(int t, int64_t k) { return (size_t)(k / type_block(t)) * type_bytes(t); }

// ---------------------------------------------------------------- device helpers

__device__ __forceinline__ float h2f(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);  // v_cvt_f32_f16: exact
}
__device__ __forceinline__ uint16_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);  // round to nearest even
}

// candle's silu(g) * u: g / (1 + exp(-g)) in f32 (correctly rounded divide), times u.  exp(-g)
// is the f64 exponential rounded once to f32, i.e. the correctly rounded f32 value, which the
// host libm's expf returns for all but a vanishing fraction of arguments (its error bound is a
// hair above half an ulp); the device's single-precision expf differs from it in the last place
// for about 3% of arguments.
__device__ __forceinline__ float silu_mul(float g, float u) {
  const float e = (float)exp(-(double)g);
  return g / (1.f + e) * u;
}

template <typename T>
__device__ __forceinline__ T ldg_u(const uint8_t* p) {  // unaligned-tolerant load
  T v;
  __builtin_memcpy(&v, p, sizeof(T));
  return v;
}

__device__ __forceinline__ int sdot4(int a, int b, int c) {
  return __builtin_amdgcn_sdot4(a, b, c, false);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, WAVE);
  return v;
}
template <int W>
__device__ __forceinline__ float group_sum(float v) {  // sum over aligned groups of W lanes
#pragma unroll
  for (int o = W / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, WAVE);
  return v;
}
// Sum over aligned groups of 16 lanes with DPP (no LDS traffic): quad_perm [1,0,3,2],
// quad_perm [2,3,0,1], row_half_mirror, row_mirror.  Every lane of a group ends with the same
// bits (each step adds a value to its partner's, and f32 addition is commutative).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               0xF, 0xF, false));
}
__device__ __forceinline__ float sum16(float v) {
  v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);  // row_half_mirror: lane i <- lane 7-i within 8
  v += dpp_mov<0x140>(v);  // row_mirror: lane i <- lane 15-i within 16
  return v;
}
template <int W>
__device__ __forceinline__ float lane_group_sum(float v) {  // aligned groups of W lanes
  static_assert(W == 4 || W == 8 || W == 16 || W == 32 || W == 64, "group of 4 .. 64 lanes");
  v += dpp_mov<0xB1>(v);                        // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);                        // quad_perm [2,3,0,1]
  if constexpr (W >= 8) v += dpp_mov<0x141>(v);   // row_half_mirror
  if constexpr (W >= 16) v += dpp_mov<0x140>(v);  // row_mirror
  if constexpr (W >= 32) v += __shfl_xor(v, 16, WAVE);
  if constexpr (W >= 64) v += __shfl_xor(v, 32, WAVE);
  return v;
}
// Wave-wide max / sum without LDS: DPP within each 16-lane row, then the four row values
// through readlane (the result is identical on every lane).
__device__ __forceinline__ float readlane_f(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));
  v = fmaxf(v, dpp_mov<0x4E>(v));
  v = fmaxf(v, dpp_mov<0x141>(v));
  v = fmaxf(v, dpp_mov<0x140>(v));
  return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = sum16(v);
  return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}
// candle BlockQ8K::from_float for one 256-element block held by a wave, 4 values per lane
// (lane l holds elements 4l .. 4l+3): the signed value of largest |x| (first occurrence wins
// ties), iscale = -128/max, q = round-half-away(iscale * x) clamped to [-128, 127], d = 1/iscale,
// per-16 sums.  Returns the packed 4 int8 of the lane; *qsum16 = the sum of its 16-group (valid
// on every lane of the group of 4), *d = the block scale (all lanes).
__device__ __forceinline__ int q8k_block_wave(const float e[4], int* qsum16, float* d) {
  const float la = fmaxf(fmaxf(fabsf(e[0]), fabsf(e[1])), fmaxf(fabsf(e[2]), fabsf(e[3])));
  const float amax = wave_max_dpp(la);
  const float mine = fabsf(e[0]) == amax ? e[0] : fabsf(e[1]) == amax ? e[1]
                     : fabsf(e[2]) == amax ? e[2] : e[3];
  const unsigned long long hit = __ballot(la == amax);
  const int first = hit ? (int)__builtin_ctzll(hit) : 0;
  const float mx = readlane_f(mine, first);
  int packed = 0, qsum = 0;
  float dd = 0.f;
  if (amax != 0.f) {
    const float iscale = -128.f / mx;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      float r = roundf(iscale * e[j]);
      r = fminf(r, 127.f);
      r = fmaxf(r, -128.f);
      const int q = (int)r;
      qsum += q;
      packed |= (q & 0xff) << (8 * j);
    }
    dd = 1.f / iscale;
  }
  qsum += __builtin_amdgcn_update_dpp(0, qsum, 0xB1, 0xF, 0xF, false);  // groups of 4 lanes
  qsum += __builtin_amdgcn_update_dpp(0, qsum, 0x4E, 0xF, 0xF, false);
  *qsum16 = qsum;
  *d = dd;
  return packed;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
  return v;
}

// f32 total order key (f32::total_cmp) widened to an unsigned key: larger key = larger value.
__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t b = __builtin_bit_cast(uint32_t, f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// One element of a GGUF row, dequantized with candle's to_float arithmetic (bit-exact):
//   Q4_K: (d*sc)*q - dmin*m     (candle BlockQ4K::to_float; ggml dequantize_row_q4_K order)
//   Q6_K: (d*sc)*(q-32)         (candle BlockQ6K::to_float; dequant_q6k.wgsl:9-24 layout)
//   Q8_0: d*q                   (candle BlockQ8_0::to_float; dequant_q8.wgsl:3-6)
__device__ __forceinline__ float dequant_elem(int type, const uint8_t* base, int64_t i) {
  if (type == TPT_TYPE_Q4_K) {
    const uint8_t* b = base + (i >> 8) * 144;
    const int j = (int)(i & 255), g = j >> 6, l = j & 63;
    const int sub = 2 * g + (l >= 32);
    const uint8_t qb = b[16 + 32 * g + (l & 31)];
    const int q = l < 32 ? (qb & 0xF) : (qb >> 4);
    const uint8_t* s = b + 4;
    int sc, m;
    if (sub < 4) {
      sc = s[sub] & 63;
      m = s[sub + 4] & 63;
    } else {
      sc = (s[sub + 4] & 0xF) | ((s[sub - 4] >> 6) << 4);
      m = (s[sub + 4] >> 4) | ((s[sub] >> 6) << 4);
    }
    const float d = h2f(ldg_u<uint16_t>(b)), dmin = h2f(ldg_u<uint16_t>(b + 2));
    const float d1 = d * (float)sc, m1 = dmin * (float)m;
    return d1 * (float)q - m1;
  }
  if (type == TPT_TYPE_Q6_K) {
    const uint8_t* b = base + (i >> 8) * 210;
    const int j = (int)(i & 255), p = j >> 7, r = j & 127, quad = r >> 5, l = r & 31;
    const uint8_t qlb = b[64 * p + 32 * (quad & 1) + l];
    const int lo = quad >= 2 ? (qlb >> 4) : (qlb & 0xF);
    const int hi = (b[128 + 32 * p + l] >> (2 * quad)) & 3;
    const int q = (lo | (hi << 4)) - 32;
    const int sc = (int8_t)b[192 + 8 * p + (l >> 4) + 2 * quad];
    const float d = h2f(ldg_u<uint16_t>(b + 208));
    return d * (float)sc * (float)q;
  }
  if (type == TPT_TYPE_Q8_0) {
    const uint8_t* b = base + (i >> 5) * 34;
    return h2f(ldg_u<uint16_t>(b)) * (float)(int8_t)b[2 + (i & 31)];
  }
  if (type == TPT_TYPE_Q5_K) {  // Q4_K's layout plus bit (2 group + half) of qh[l]
    const uint8_t* b = base + (i >> 8) * 176;
    const int j = (int)(i & 255), g = j >> 6, half = (j >> 5) & 1, l = j & 31, sub = 2 * g + half;
    const uint8_t qb = b[48 + 32 * g + l];
    const int q = (half ? (qb >> 4) : (qb & 0xF)) + (((b[16 + l] >> sub) & 1) << 4);
    const uint8_t* s = b + 4;
    int sc, m;
    if (sub < 4) {
      sc = s[sub] & 63;
      m = s[sub + 4] & 63;
    } else {
      sc = (s[sub + 4] & 0xF) | ((s[sub - 4] >> 6) << 4);
      m = (s[sub + 4] >> 4) | ((s[sub] >> 6) << 4);
    }
    const float d = h2f(ldg_u<uint16_t>(b)), dmin = h2f(ldg_u<uint16_t>(b + 2));
    const float d1 = d * (float)sc, m1 = dmin * (float)m;
    return d1 * (float)q - m1;
  }
  if (type == TPT_TYPE_Q4_0) {  // element j < 16: low nibble of qs[j]; j + 16: its high nibble
    const uint8_t* b = base + (i >> 5) * 18;
    const int j = (int)(i & 31);
    const int q = j < 16 ? (b[2 + j] & 0xF) : (b[2 + j - 16] >> 4);
    return (float)(q - 8) * h2f(ldg_u<uint16_t>(b));
  }
  if (type == TPT_TYPE_F16) return h2f(ldg_u<uint16_t>(base + 2 * i));
  return ldg_u<float>(base + 4 * i);
}

// ---------------------------------------------------------------- errors

void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* what, const char* file, int line);

#define TPT_HIP(call)                                                   \
  do {                                                                  \
    hipError_t _e = (call);                                             \
    if (_e != hipSuccess) return ::tpt::hip_fail(_e, #call, __FILE__, __LINE__); \
  } while (0)

}  // namespace tpt

struct tpt_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  int n_cu = 0;
  char name[256] = {0};
};

namespace tpt {
int ctx_enter(tpt_ctx* c);  // hipSetDevice(c->device); status
}
