/*
 * CPU oracle -- TEST INFRASTRUCTURE ONLY (the checker; see oracle.h for the rules and the
 * per-function pinning status).  Plain C restatement of the CPU arithmetic that the
 * reference's CandleEngine (src-tauri/src/engine/candle_engine.rs:205-334) runs through
 * candle-core / candle-nn / candle-transformers 0.8.4 (src-tauri/Cargo.lock:316-370, not
 * vendored).  Built with -ffp-contract=off: Rust never contracts a*b+c into an FMA.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <fcntl.h>
#include <math.h>
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

/* ------------------------------------------------------------------ fp16 */

/* half::f16::to_f32 (exact widening) */
float orc_fp16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31, exp = (h >> 10) & 0x1f, man = h & 0x3ff, f;
  if (exp == 0) {
    if (man == 0) {
      f = sign;
    } else {
      int k = 0;
      while (!(man & 0x400)) { man <<= 1; k++; }
      f = sign | ((uint32_t)(113 - k) << 23) | ((man & 0x3ff) << 13);
    }
  } else if (exp == 31) {
    f = sign | 0x7f800000u | (man << 13);
  } else {
    f = sign | ((exp + 112) << 23) | (man << 13);
  }
  float r;
  memcpy(&r, &f, 4);
  return r;
}

/* half::f16::from_f32: round to nearest, ties to even */
uint16_t orc_f32_to_fp16(float v) {
  uint32_t x;
  memcpy(&x, &v, 4);
  uint32_t sign = (x >> 16) & 0x8000, exp = (x >> 23) & 0xff, man = x & 0x7fffff;
  if (exp == 0xff) return (uint16_t)(sign | 0x7c00 | (man ? (0x200 | (man >> 13)) : 0));
  int32_t e = (int32_t)exp - 112;
  if (e >= 0x1f) return (uint16_t)(sign | 0x7c00);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    uint32_t m = man | 0x800000, sh = (uint32_t)(14 - e);
    uint32_t h = m >> sh, rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
    if (rem > half || (rem == half && (h & 1))) h++;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((uint32_t)e << 10) | (man >> 13), rem = man & 0x1fff;
  if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) h++;
  return (uint16_t)(sign | h);
}

size_t orc_type_size(int t) {
  switch (t) {
    case ORC_F32: return 4;
    case ORC_F16: return 2;
    case ORC_Q8_0: return sizeof(orc_blk_q8_0);
    case ORC_Q4_K: return sizeof(orc_blk_q4k);
    case ORC_Q5_K: return sizeof(orc_blk_q5k);
    case ORC_Q6_K: return sizeof(orc_blk_q6k);
    case ORC_Q4_0: return sizeof(orc_blk_q4_0);
    case ORC_Q8_K: return sizeof(orc_blk_q8k);
  }
  return 0;
}

int orc_block_size(int t) {
  switch (t) {
    case ORC_F32: case ORC_F16: return 1;
    case ORC_Q8_0: case ORC_Q4_0: return ORC_QK8_0;
    case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: case ORC_Q8_K: return ORC_QK_K;
  }
  return 0;
}

/* ------------------------------------------------------------------ dequant */

/* ggml get_scale_min_k4; candle k_quants::get_scale_min_k4 (same bit layout as
 * reference shaders/dequant_q4k.wgsl:14-17,50-72) */
static inline void scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
  if (j < 4) {
    *d = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

/* candle BlockQ4K::to_float (ggml dequantize_row_q4_K): for each 64-element group the 32
 * low nibbles come first, then the 32 high nibbles of the same 32 bytes.  NOT the element
 * order of reference shaders/dequant_q4k.wgsl:9-12 (which is not ggml's). */
static void dequant_q4k(const orc_blk_q4k* x, float* y, int64_t nb) {
  for (int64_t i = 0; i < nb; i++) {
    const float d = orc_fp16_to_f32(x[i].d), min = orc_fp16_to_f32(x[i].dmin);
    const uint8_t* q = x[i].qs;
    int is = 0;
    for (int j = 0; j < ORC_QK_K; j += 64) {
      uint8_t sc, m;
      scale_min_k4(is + 0, x[i].scales, &sc, &m);
      const float d1 = d * sc, m1 = min * m;
      scale_min_k4(is + 1, x[i].scales, &sc, &m);
      const float d2 = d * sc, m2 = min * m;
      for (int l = 0; l < 32; l++) *y++ = d1 * (q[l] & 0xF) - m1;
      for (int l = 0; l < 32; l++) *y++ = d2 * (q[l] >> 4) - m2;
      q += 32;
      is += 2;
    }
  }
}

/* candle BlockQ5K::to_float (ggml dequantize_row_q5_K): Q4_K's layout and scales plus a fifth
 * bit per element from qh: for the j-th 64-element group, bit 2j of qh[l] goes to element l of
 * the low-nibble half and bit 2j+1 to element l of the high-nibble half. */
static void dequant_q5k(const orc_blk_q5k* x, float* y, int64_t nb) {
  for (int64_t i = 0; i < nb; i++) {
    const float d = orc_fp16_to_f32(x[i].d), min = orc_fp16_to_f32(x[i].dmin);
    const uint8_t* ql = x[i].qs;
    const uint8_t* qh = x[i].qh;
    int is = 0;
    uint8_t u1 = 1, u2 = 2;
    for (int j = 0; j < ORC_QK_K; j += 64) {
      uint8_t sc, m;
      scale_min_k4(is + 0, x[i].scales, &sc, &m);
      const float d1 = d * sc, m1 = min * m;
      scale_min_k4(is + 1, x[i].scales, &sc, &m);
      const float d2 = d * sc, m2 = min * m;
      for (int l = 0; l < 32; l++) *y++ = d1 * ((ql[l] & 0xF) + (qh[l] & u1 ? 16 : 0)) - m1;
      for (int l = 0; l < 32; l++) *y++ = d2 * ((ql[l] >> 4) + (qh[l] & u2 ? 16 : 0)) - m2;
      ql += 32;
      is += 2;
      u1 <<= 2;
      u2 <<= 2;
    }
  }
}

/* candle BlockQ4_0::to_float (ggml dequantize_row_q4_0): element j < 16 is the low nibble of
 * qs[j], element j + 16 its high nibble, each minus 8, times d */
static void dequant_q4_0(const orc_blk_q4_0* x, float* y, int64_t nb) {
  for (int64_t i = 0; i < nb; i++) {
    const float d = orc_fp16_to_f32(x[i].d);
    for (int j = 0; j < 16; j++) {
      y[j] = (float)((x[i].qs[j] & 0xF) - 8) * d;
      y[j + 16] = (float)((x[i].qs[j] >> 4) - 8) * d;
    }
    y += 32;
  }
}

/* candle BlockQ6K::to_float (ggml dequantize_row_q6_K; same layout as reference
 * shaders/dequant_q6k.wgsl:9-24): y = (d*sc)*q, evaluated left to right */
static void dequant_q6k(const orc_blk_q6k* x, float* y, int64_t nb) {
  for (int64_t i = 0; i < nb; i++) {
    const float d = orc_fp16_to_f32(x[i].d);
    const uint8_t* ql = x[i].ql;
    const uint8_t* qh = x[i].qh;
    const int8_t* sc = x[i].scales;
    for (int n = 0; n < ORC_QK_K; n += 128) {
      for (int l = 0; l < 32; l++) {
        int is = l / 16;
        const int8_t q1 = (int8_t)((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
        const int8_t q2 = (int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
        const int8_t q3 = (int8_t)((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
        const int8_t q4 = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
        y[l + 0] = d * (float)sc[is + 0] * (float)q1;
        y[l + 32] = d * (float)sc[is + 2] * (float)q2;
        y[l + 64] = d * (float)sc[is + 4] * (float)q3;
        y[l + 96] = d * (float)sc[is + 6] * (float)q4;
      }
      y += 128;
      ql += 64;
      qh += 32;
      sc += 8;
    }
  }
}

/* candle BlockQ8_0::to_float (reference shaders/dequant_q8.wgsl:3-6): y = d*q */
static void dequant_q8_0(const orc_blk_q8_0* x, float* y, int64_t nb) {
  for (int64_t i = 0; i < nb; i++) {
    const float d = orc_fp16_to_f32(x[i].d);
    for (int l = 0; l < ORC_QK8_0; l++) *y++ = d * (float)x[i].qs[l];
  }
}

int orc_dequant(int type, const void* src, float* dst, int64_t n) {
  int bs = orc_block_size(type);
  if (bs <= 0 || n % bs) return -1;
  switch (type) {
    case ORC_F32: memcpy(dst, src, (size_t)n * 4); return 0;
    case ORC_F16:
      for (int64_t i = 0; i < n; i++) dst[i] = orc_fp16_to_f32(((const uint16_t*)src)[i]);
      return 0;
    case ORC_Q4_K: dequant_q4k((const orc_blk_q4k*)src, dst, n / bs); return 0;
    case ORC_Q5_K: dequant_q5k((const orc_blk_q5k*)src, dst, n / bs); return 0;
    case ORC_Q4_0: dequant_q4_0((const orc_blk_q4_0*)src, dst, n / bs); return 0;
    case ORC_Q6_K: dequant_q6k((const orc_blk_q6k*)src, dst, n / bs); return 0;
    case ORC_Q8_0: dequant_q8_0((const orc_blk_q8_0*)src, dst, n / bs); return 0;
    case ORC_Q8_K: {
      const orc_blk_q8k* b = (const orc_blk_q8k*)src;
      for (int64_t i = 0; i < n / bs; i++)
        for (int l = 0; l < ORC_QK_K; l++) dst[i * ORC_QK_K + l] = b[i].d * (float)b[i].qs[l];
      return 0;
    }
  }
  return -1;
}

/* ------------------------------------------------------------------ activation quant */

/* candle BlockQ8K::from_float: the signed value with the largest |x| (first one wins),
 * iscale = -128/max, q = min(127, round(iscale*x)) with round = half away from zero,
 * d = 1/iscale, bsums = sums of 16 consecutive q. */
int orc_quantize_q8k(const float* x, int64_t k, orc_blk_q8k* y) {
  if (k % ORC_QK_K) return -1;
  for (int64_t i = 0; i < k / ORC_QK_K; i++) {
    const float* xs = x + i * ORC_QK_K;
    float max = 0.f, amax = 0.f;
    for (int j = 0; j < ORC_QK_K; j++) {
      float ax = fabsf(xs[j]);
      if (amax < ax) { amax = ax; max = xs[j]; }
    }
    if (amax == 0.f) {
      y[i].d = 0.f;
      memset(y[i].qs, 0, sizeof(y[i].qs));
      memset(y[i].bsums, 0, sizeof(y[i].bsums));  /* from_float leaves the zeroed block's bsums */
      continue;
    }
    const float iscale = -128.f / max;
    for (int j = 0; j < ORC_QK_K; j++) {
      float v = roundf(iscale * xs[j]);
      if (v > 127.f) v = 127.f;
      if (v < -128.f) v = -128.f;  /* Rust `as i8` saturates */
      y[i].qs[j] = (int8_t)v;
    }
    for (int j = 0; j < ORC_QK_K / 16; j++) {
      int s = 0;
      for (int l = 0; l < 16; l++) s += y[i].qs[j * 16 + l];
      y[i].bsums[j] = (int16_t)s;
    }
    y[i].d = 1.f / iscale;
  }
  return 0;
}

/* candle BlockQ8_0::from_float: d = amax/127 (stored as f16), id = 1/d (f32 d),
 * q = round(x*id) half away from zero, saturating cast */
int orc_quantize_q8_0(const float* x, int64_t k, orc_blk_q8_0* y) {
  if (k % ORC_QK8_0) return -1;
  for (int64_t i = 0; i < k / ORC_QK8_0; i++) {
    const float* xs = x + i * ORC_QK8_0;
    float amax = 0.f;
    for (int j = 0; j < ORC_QK8_0; j++) amax = fmaxf(amax, fabsf(xs[j]));
    const float d = amax / 127.f;
    const float id = d != 0.f ? 1.f / d : 0.f;
    y[i].d = orc_f32_to_fp16(d);
    for (int j = 0; j < ORC_QK8_0; j++) {
      float v = roundf(xs[j] * id);
      if (v > 127.f) v = 127.f;
      if (v < -128.f) v = -128.f;
      y[i].qs[j] = (int8_t)v;
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ vec_dot */

/* Summation-order variant (test instrument, off by default): when set, each super-block's
 * integer lanes are added first and one f32 term per block (d * sum - dmin * mins) joins a single
 * running sum -- the order of a SIMD kernel that reduces lanes inside the block, instead of the
 * generic path's eight f32 lane accumulators.  Same integers, different f32 rounding. */
static int g_dot_block_order = 0;

void orc_set_dot_block_order(int on) { g_dot_block_order = on != 0; }

/* candle BlockQ4K::vec_dot_unopt (ggml generic ggml_vec_dot_q4_K_q8_K): 8 integer lanes
 * per block, f32 lane sums across blocks, mins subtracted through bsums. */
static float vec_dot_q4k_q8k(int64_t n, const orc_blk_q4k* x, const orc_blk_q8k* y) {
  int8_t aux8[ORC_QK_K];
  int16_t aux16[8];
  float sums[8] = {0};
  int32_t aux32[8];
  float sumf = 0.f;
  for (int64_t i = 0; i < n / ORC_QK_K; i++) {
    const uint8_t* q4 = x[i].qs;
    const int8_t* q8 = y[i].qs;
    memset(aux32, 0, sizeof(aux32));
    int8_t* a = aux8;
    for (int j = 0; j < ORC_QK_K / 64; j++) {
      for (int l = 0; l < 32; l++) a[l] = (int8_t)(q4[l] & 0xF);
      a += 32;
      for (int l = 0; l < 32; l++) a[l] = (int8_t)(q4[l] >> 4);
      a += 32;
      q4 += 32;
    }
    uint8_t scales[8], mins[8];
    for (int j = 0; j < 8; j++) scale_min_k4(j, x[i].scales, &scales[j], &mins[j]);
    int sumi = 0;
    for (int j = 0; j < ORC_QK_K / 16; j++) sumi += y[i].bsums[j] * mins[j / 2];
    a = aux8;
    for (int j = 0; j < 8; j++) {
      int32_t scale = scales[j];
      for (int r = 0; r < 4; r++) {
        for (int l = 0; l < 8; l++) aux16[l] = (int16_t)(q8[l] * a[l]);
        for (int l = 0; l < 8; l++) aux32[l] += scale * aux16[l];
        q8 += 8;
        a += 8;
      }
    }
    const float d = orc_fp16_to_f32(x[i].d) * y[i].d;
    const float dmin = orc_fp16_to_f32(x[i].dmin) * y[i].d;
    if (g_dot_block_order) {
      int32_t t = 0;
      for (int l = 0; l < 8; l++) t += aux32[l];
      sumf += d * (float)t - dmin * (float)sumi;
      continue;
    }
    for (int l = 0; l < 8; l++) sums[l] += d * (float)aux32[l];
    sumf -= dmin * (float)sumi;
  }
  float s = 0.f;
  for (int l = 0; l < 8; l++) s += sums[l];
  return sumf + s;
}

/* candle BlockQ5K::vec_dot_unopt (ggml generic ggml_vec_dot_q5_K_q8_K): vec_dot_q4k_q8k with
 * the 5-bit values (nibble + 16 * qh bit). */
static float vec_dot_q5k_q8k(int64_t n, const orc_blk_q5k* x, const orc_blk_q8k* y) {
  int8_t aux8[ORC_QK_K];
  int16_t aux16[8];
  float sums[8] = {0};
  int32_t aux32[8];
  float sumf = 0.f;
  for (int64_t i = 0; i < n / ORC_QK_K; i++) {
    const uint8_t* q4 = x[i].qs;
    const uint8_t* hm = x[i].qh;
    const int8_t* q8 = y[i].qs;
    memset(aux32, 0, sizeof(aux32));
    int8_t* a = aux8;
    uint8_t m = 1;
    for (int j = 0; j < ORC_QK_K / 64; j++) {
      for (int l = 0; l < 32; l++) a[l] = (int8_t)(q4[l] & 0xF);
      for (int l = 0; l < 32; l++) a[l] += (hm[l] & m ? 16 : 0);
      a += 32;
      m <<= 1;
      for (int l = 0; l < 32; l++) a[l] = (int8_t)(q4[l] >> 4);
      for (int l = 0; l < 32; l++) a[l] += (hm[l] & m ? 16 : 0);
      a += 32;
      m <<= 1;
      q4 += 32;
    }
    uint8_t scales[8], mins[8];
    for (int j = 0; j < 8; j++) scale_min_k4(j, x[i].scales, &scales[j], &mins[j]);
    int sumi = 0;
    for (int j = 0; j < ORC_QK_K / 16; j++) sumi += y[i].bsums[j] * mins[j / 2];
    a = aux8;
    for (int j = 0; j < 8; j++) {
      int32_t scale = scales[j];
      for (int r = 0; r < 4; r++) {
        for (int l = 0; l < 8; l++) aux16[l] = (int16_t)(q8[l] * a[l]);
        for (int l = 0; l < 8; l++) aux32[l] += scale * aux16[l];
        q8 += 8;
        a += 8;
      }
    }
    const float d = orc_fp16_to_f32(x[i].d) * y[i].d;
    const float dmin = orc_fp16_to_f32(x[i].dmin) * y[i].d;
    if (g_dot_block_order) {
      int32_t t = 0;
      for (int l = 0; l < 8; l++) t += aux32[l];
      sumf += d * (float)t - dmin * (float)sumi;
      continue;
    }
    for (int l = 0; l < 8; l++) sums[l] += d * (float)aux32[l];
    sumf -= dmin * (float)sumi;
  }
  float s = 0.f;
  for (int l = 0; l < 8; l++) s += sums[l];
  return sumf + s;
}

/* candle BlockQ4_0::vec_dot_unopt (ggml generic ggml_vec_dot_q4_0_q8_0): per 32-block
 * sumi = sum (q_lo - 8) y[j] + (q_hi - 8) y[j + 16], sumf += (float)sumi * d_w * d_x */
static float vec_dot_q4_0_q8_0(int64_t n, const orc_blk_q4_0* x, const orc_blk_q8_0* y) {
  float sumf = 0.f;
  for (int64_t i = 0; i < n / ORC_QK8_0; i++) {
    int32_t s0 = 0, s1 = 0;
    for (int j = 0; j < 16; j++) {
      s0 += ((x[i].qs[j] & 0xF) - 8) * (int32_t)y[i].qs[j];
      s1 += ((x[i].qs[j] >> 4) - 8) * (int32_t)y[i].qs[j + 16];
    }
    sumf += (float)(s0 + s1) * orc_fp16_to_f32(x[i].d) * orc_fp16_to_f32(y[i].d);
  }
  return sumf;
}

/* candle BlockQ6K::vec_dot_unopt (ggml generic ggml_vec_dot_q6_K_q8_K); the per-lane
 * accumulator is f32 there, which holds these integer partial sums exactly. */
static float vec_dot_q6k_q8k(int64_t n, const orc_blk_q6k* x, const orc_blk_q8k* y) {
  int8_t aux8[ORC_QK_K];
  int16_t aux16[8];
  float sums[8] = {0};
  float aux32[8];
  for (int64_t i = 0; i < n / ORC_QK_K; i++) {
    const uint8_t* q4 = x[i].ql;
    const uint8_t* qh = x[i].qh;
    const int8_t* q8 = y[i].qs;
    memset(aux32, 0, sizeof(aux32));
    for (int j = 0; j < ORC_QK_K; j += 128) {
      int8_t* a = aux8 + j;
      const uint8_t* q4j = q4 + j / 2;
      const uint8_t* qhj = qh + j / 4;
      for (int l = 0; l < 32; l++) {
        a[l] = (int8_t)(((q4j[l] & 0xF) | ((qhj[l] & 3) << 4)) - 32);
        a[l + 32] = (int8_t)(((q4j[l + 32] & 0xF) | (((qhj[l] >> 2) & 3) << 4)) - 32);
        a[l + 64] = (int8_t)(((q4j[l] >> 4) | (((qhj[l] >> 4) & 3) << 4)) - 32);
        a[l + 96] = (int8_t)(((q4j[l + 32] >> 4) | (((qhj[l] >> 6) & 3) << 4)) - 32);
      }
    }
    for (int j = 0; j < 16; j++) {
      const float scale = (float)x[i].scales[j];
      const int8_t* q8j = q8 + 16 * j;
      const int8_t* aj = aux8 + 16 * j;
      for (int l = 0; l < 8; l++) aux16[l] = (int16_t)(q8j[l] * aj[l]);
      for (int l = 0; l < 8; l++) aux32[l] += scale * (float)aux16[l];
      for (int l = 0; l < 8; l++) aux16[l] = (int16_t)(q8j[8 + l] * aj[8 + l]);
      for (int l = 0; l < 8; l++) aux32[l] += scale * (float)aux16[l];
    }
    const float d = orc_fp16_to_f32(x[i].d) * y[i].d;
    if (g_dot_block_order) {
      float t = 0.f;
      for (int l = 0; l < 8; l++) t += aux32[l];
      sums[0] += t * d;
      continue;
    }
    for (int l = 0; l < 8; l++) sums[l] += aux32[l] * d;
  }
  float s = 0.f;
  for (int l = 0; l < 8; l++) s += sums[l];
  return s;
}

/* candle BlockQ8_0::vec_dot_unopt: sumf += (sum_i * d_w) * d_x per 32-block */
static float vec_dot_q8_0_q8_0(int64_t n, const orc_blk_q8_0* x, const orc_blk_q8_0* y) {
  float sumf = 0.f;
  for (int64_t i = 0; i < n / ORC_QK8_0; i++) {
    int32_t s = 0;
    for (int l = 0; l < ORC_QK8_0; l++) s += (int32_t)x[i].qs[l] * (int32_t)y[i].qs[l];
    sumf += (float)s * orc_fp16_to_f32(x[i].d) * orc_fp16_to_f32(y[i].d);
  }
  return sumf;
}

float orc_vec_dot(int type, int64_t k, const void* w_row, const void* act_q) {
  switch (type) {
    case ORC_Q4_K: return vec_dot_q4k_q8k(k, (const orc_blk_q4k*)w_row, (const orc_blk_q8k*)act_q);
    case ORC_Q5_K: return vec_dot_q5k_q8k(k, (const orc_blk_q5k*)w_row, (const orc_blk_q8k*)act_q);
    case ORC_Q6_K: return vec_dot_q6k_q8k(k, (const orc_blk_q6k*)w_row, (const orc_blk_q8k*)act_q);
    case ORC_Q4_0: return vec_dot_q4_0_q8_0(k, (const orc_blk_q4_0*)w_row, (const orc_blk_q8_0*)act_q);
    case ORC_Q8_0: return vec_dot_q8_0_q8_0(k, (const orc_blk_q8_0*)w_row, (const orc_blk_q8_0*)act_q);
  }
  return NAN;
}

static int is_quant_type(int t) {
  return t == ORC_Q4_K || t == ORC_Q5_K || t == ORC_Q6_K || t == ORC_Q8_0 || t == ORC_Q4_0;
}

/* candle k_quants::matmul: each lhs row is quantized to the weight type's VecDotType
 * (Q8_K for k-quants, Q8_0 for Q8_0), then one vec_dot per output column (rayon there,
 * OpenMP here; each column is independent so the thread count does not change results). */
int orc_matmul(int type, int64_t m, int64_t k, int64_t n, const float* lhs, const void* w,
               float* dst, int nthreads) {
  if (nthreads <= 0) nthreads = omp_get_num_procs();
  if (type == ORC_F32) {
    /* plain f32 weights (not on the Q4_K_M path): sequential dot */
    const float* W = (const float*)w;
    for (int64_t r = 0; r < m; r++) {
#pragma omp parallel for num_threads(nthreads) schedule(static)
      for (int64_t c = 0; c < n; c++) {
        float s = 0.f;
        for (int64_t i = 0; i < k; i++) s += lhs[r * k + i] * W[c * k + i];
        dst[r * n + c] = s;
      }
    }
    return 0;
  }
  if (type == ORC_F16) {
    /* QMatMul::from_arc dequantizes F16 (and F32) weights to an f32 tensor and forward runs
     * xs.matmul(w.t()): the weights widen exactly and the product is an f32 matmul.  candle's
     * f32 matmul is the gemm crate; its blocking and summation order are not restated here:
     * each output is one f32 FMA chain along k (parity unpinned; the GPU's order differs by
     * f32 rounding only, and tests bound both against an fp64 dot). */
    const uint16_t* W = (const uint16_t*)w;
    for (int64_t r = 0; r < m; r++) {
#pragma omp parallel for num_threads(nthreads) schedule(static)
      for (int64_t c = 0; c < n; c++) {
        float s = 0.f;
        for (int64_t i = 0; i < k; i++) s = fmaf(lhs[r * k + i], orc_fp16_to_f32(W[c * k + i]), s);
        dst[r * n + c] = s;
      }
    }
    return 0;
  }
  if (!is_quant_type(type)) return -1;
  const int bs = orc_block_size(type);
  if (k % bs) return -2;
  const size_t row_bytes = (size_t)(k / bs) * orc_type_size(type);
  const int act_type = type == ORC_Q8_0 || type == ORC_Q4_0 ? ORC_Q8_0 : ORC_Q8_K;
  const size_t act_row = (size_t)(k / orc_block_size(act_type)) * orc_type_size(act_type);
  uint8_t* aq = (uint8_t*)malloc(act_row * (size_t)m);
  if (!aq) return -3;
  for (int64_t r = 0; r < m; r++) {
    if (act_type == ORC_Q8_K) orc_quantize_q8k(lhs + r * k, k, (orc_blk_q8k*)(aq + r * act_row));
    else orc_quantize_q8_0(lhs + r * k, k, (orc_blk_q8_0*)(aq + r * act_row));
  }
  for (int64_t r = 0; r < m; r++) {
    const uint8_t* ar = aq + r * act_row;
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int64_t c = 0; c < n; c++)
      dst[r * n + c] = orc_vec_dot(type, k, (const uint8_t*)w + (size_t)c * row_bytes, ar);
  }
  free(aq);
  return 0;
}

int orc_gemv_f64(int type, int64_t k, int64_t n, const void* w, const double* x, double* y) {
  const int bs = orc_block_size(type);
  if (bs <= 0 || k % bs) return -1;
  const size_t row_bytes = (size_t)(k / bs) * orc_type_size(type);
  int err = 0;
#pragma omp parallel
  {
    float* row = (float*)malloc((size_t)k * 4);
    if (!row) err = -2;
#pragma omp for schedule(static)
    for (int64_t c = 0; c < n; c++) {
      if (!row) continue;
      orc_dequant(type, (const uint8_t*)w + (size_t)c * row_bytes, row, k);
      double s = 0.0;
      for (int64_t i = 0; i < k; i++) s += (double)row[i] * x[i];
      y[c] = s;
    }
    free(row);
  }
  return err;
}

/* ------------------------------------------------------------------ small ops */

/* Summation-order variant of rms_norm's sum of squares (test instrument, off by default): fused
 * multiply-add sums over runs of 16 elements, then the run sums added pairwise as a tree -- the
 * shape of a GPU reduction.  Same squares, different f32 rounding. */
static int g_rms_order = 0;

void orc_set_rms_order(int on) { g_rms_order = on != 0; }

static float sum_squares_tree(const float* x, int64_t n) {
  const int64_t m0 = n / 16;
  float* p = (float*)malloc(sizeof(float) * (size_t)m0);
  for (int64_t j = 0; j < m0; j++) {
    float s = 0.f;
    for (int i = 0; i < 16; i++) s = fmaf(x[16 * j + i], x[16 * j + i], s);
    p[j] = s;
  }
  int64_t m = m0;
  while (m > 1) {
    for (int64_t i = 0; i < m / 2; i++) p[i] = p[2 * i] + p[2 * i + 1];
    if (m & 1) p[m / 2] = p[m - 1];
    m = (m + 1) / 2;
  }
  const float t = p[0];
  free(p);
  return t;
}

/* candle_nn::ops::rms_norm CPU: sum2 sequential in f32, m = sqrt(sum2/dim + eps),
 * y = x / m * alpha */
void orc_rmsnorm(const float* x, const float* w, int64_t n, float eps, float* y) {
  float sum2 = 0.f;
  if (g_rms_order && n >= 16 && n % 16 == 0) sum2 = sum_squares_tree(x, n);
  else
    for (int64_t i = 0; i < n; i++) sum2 += x[i] * x[i];
  const float m = sqrtf(sum2 / (float)n + eps);
  for (int64_t i = 0; i < n; i++) y[i] = x[i] / m * w[i];
}

float orc_silu(float v) { return v / (1.f + expf(-v)); }

/* quantized_llama::precomput_freqs_cis: theta_i = 1/base^(2i/d) (f32 powf),
 * angle = pos*theta_i (f32), cos/sin in f32 */
static void rope_rows(int rope_dim, float base, int p_lo, int p_hi, float* cos_t, float* sin_t) {
  const int half = rope_dim / 2;
  float* theta = (float*)malloc(sizeof(float) * (size_t)half);
  for (int i = 0; i < half; i++) theta[i] = 1.f / powf(base, (float)(2 * i) / (float)rope_dim);
  for (int p = p_lo; p < p_hi; p++)
    for (int i = 0; i < half; i++) {
      const float a = (float)p * theta[i];
      cos_t[(size_t)p * half + i] = cosf(a);
      sin_t[(size_t)p * half + i] = sinf(a);
    }
  free(theta);
}

void orc_rope_tables(int rope_dim, float base, int n_pos, float* cos_t, float* sin_t) {
  rope_rows(rope_dim, base, 0, n_pos, cos_t, sin_t);
}

/* candle_nn::rotary_emb::rope_i CPU kernel: interleaved pairs (x[2i], x[2i+1]) */
void orc_rope_i(float* x, int n_heads, int hd, const float* c, const float* s) {
  for (int h = 0; h < n_heads; h++) {
    float* v = x + (size_t)h * hd;
    for (int i = 0; i < hd / 2; i++) {
      const float x0 = v[2 * i], x1 = v[2 * i + 1];
      v[2 * i] = x0 * c[i] - x1 * s[i];
      v[2 * i + 1] = x0 * s[i] + x1 * c[i];
    }
  }
}

/* quantized_llama LayerWeights::forward_attn, non-metal branch: repeat_kv (head h reads kv
 * head h / (nq/nkv)), scores = (q.k) * f32(1/sqrt(hd)), softmax_last_dim, p.v.  The two products
 * are candle's f32 matmul, i.e. the gemm crate (gemm 0.17.1, Cargo.lock), which picks its kernel
 * at run time by CPU feature: on a host with FMA (every x86-64-v3 part, which this library is
 * built for) each output accumulates fused multiply-adds in order along the reduced dimension,
 * on a host without FMA separate multiplies and adds.  fma = 1 restates the first (the default
 * of the model and of orc_attention), fma = 0 the second (a test instrument: the spread between
 * them is how far candle's own result moves between hosts). */
static void attention_impl(const float* q, const float* kc, const float* vc, int nq, int nkv, int hd,
                           int L, int L_stride, float* o, int fma) {
  const float scale = (float)(1.0 / sqrt((double)hd));
  const int rep = nq / nkv;
  /* heads are independent (each is its own matmul row in candle): one per thread, every head's
   * arithmetic in the same order as a serial run */
#pragma omp parallel for schedule(static) if (L >= 256)
  for (int h = 0; h < nq; h++) {
    float* sc = (float*)malloc(sizeof(float) * (size_t)L);
    const int g = h / rep;
    const float* qh = q + (size_t)h * hd;
    const float* K = kc + (size_t)g * L_stride * hd;
    const float* V = vc + (size_t)g * L_stride * hd;
    float mx = -INFINITY;
    for (int p = 0; p < L; p++) {
      float s = 0.f;
      for (int d = 0; d < hd; d++) s = fma ? fmaf(qh[d], K[(size_t)p * hd + d], s) : s + qh[d] * K[(size_t)p * hd + d];
      s = s * scale;
      sc[p] = s;
      if (s > mx) mx = s;
    }
    float sum = 0.f;
    for (int p = 0; p < L; p++) {
      sc[p] = expf(sc[p] - mx);
      sum += sc[p];
    }
    for (int p = 0; p < L; p++) sc[p] /= sum;
    float* oh = o + (size_t)h * hd;
    for (int d = 0; d < hd; d++) {
      float acc = 0.f;
      for (int p = 0; p < L; p++) acc = fma ? fmaf(sc[p], V[(size_t)p * hd + d], acc) : acc + sc[p] * V[(size_t)p * hd + d];
      oh[d] = acc;
    }
    free(sc);
  }
}

void orc_attention(const float* q, const float* kc, const float* vc, int nq, int nkv, int hd,
                   int L, int L_stride, float* o) {
  attention_impl(q, kc, vc, nq, nkv, hd, L, L_stride, o, 1);
}

/* f32::total_cmp key */
static inline int32_t total_key(float f) {
  int32_t b;
  memcpy(&b, &f, 4);
  return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

uint32_t orc_argmax(const float* logits, int64_t n) {
  int64_t best = 0;
  int32_t bk = total_key(logits[0]);
  for (int64_t i = 1; i < n; i++) {
    int32_t k = total_key(logits[i]);
    if (k >= bk) { bk = k; best = i; }  /* Iterator::max_by keeps the last maximum */
  }
  return (uint32_t)best;
}

void orc_repeat_penalty(float* logits, int64_t n, const uint32_t* seen, int64_t n_seen,
                        float penalty) {
  if (fabsf(penalty - 1.f) < 1.1920929e-07f) return;
  for (int64_t i = 0; i < n_seen; i++) {
    uint32_t id = seen[i];
    if ((int64_t)id < n) {
      if (logits[id] >= 0.f) logits[id] /= penalty;
      else logits[id] *= penalty;
    }
  }
}

/* ------------------------------------------------------------------ GGUF */

typedef struct {
  char name[96];
  int type;
  int n_dims;
  int64_t ne[4];
  uint64_t offset;
  const uint8_t* data;
} orc_tensor;

typedef struct {
  char key[96];
  int vtype;
  uint64_t u;
  double f;
  char s[64];
} orc_kv;

typedef struct {
  const orc_tensor *q, *k, *v, *o, *gate, *up, *down;
  const float *attn_norm, *ffn_norm;
} orc_layer;

struct orc_model {
  uint8_t* map;
  size_t map_len;
  orc_tensor* tensors;
  int n_tensors;
  orc_kv* kvs;
  int n_kvs;
  orc_model_cfg cfg;
  const orc_tensor *tok_embd, *output;
  const float* output_norm;
  orc_layer* layers;
  /* runtime state */
  int max_pos, kv_f16;
  int attn_fma; /* attention dots as fused multiply-adds (candle's gemm crate on an FMA host) */
  float *kcache, *vcache; /* [layer][kvh][max_pos][hd] */
  float* hidden;          /* last position's residual stream */
};

typedef struct {
  const uint8_t* p;
  const uint8_t* end;
  int bad;
} rd_t;

static uint64_t rd_u(rd_t* r, int nb) {
  if (r->p + nb > r->end) { r->bad = 1; return 0; }
  uint64_t v = 0;
  memcpy(&v, r->p, (size_t)nb);
  r->p += nb;
  return v;
}

static void rd_str(rd_t* r, char* out, size_t cap) {
  uint64_t len = rd_u(r, 8);
  if (r->bad || r->p + len > r->end) { r->bad = 1; return; }
  if (out) {
    size_t c = len < cap - 1 ? (size_t)len : cap - 1;
    memcpy(out, r->p, c);
    out[c] = 0;
  }
  r->p += len;
}

static int scalar_size(int t) {
  switch (t) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
  }
  return -1;
}

static void rd_value(rd_t* r, int t, orc_kv* kv) {
  if (t == 8) { rd_str(r, kv ? kv->s : NULL, 64); return; }
  if (t == 9) {
    int et = (int)rd_u(r, 4);
    uint64_t cnt = rd_u(r, 8);
    for (uint64_t i = 0; i < cnt && !r->bad; i++) rd_value(r, et, NULL);
    return;
  }
  int sz = scalar_size(t);
  if (sz < 0) { r->bad = 1; return; }
  uint64_t raw = rd_u(r, sz);
  if (!kv) return;
  kv->u = raw;
  if (t == 6) { float f; uint32_t b = (uint32_t)raw; memcpy(&f, &b, 4); kv->f = f; }
  else if (t == 12) { double d; memcpy(&d, &raw, 8); kv->f = d; }
  else if (t == 1) kv->f = (double)(int8_t)raw;
  else if (t == 3) kv->f = (double)(int16_t)raw;
  else if (t == 5) kv->f = (double)(int32_t)raw;
  else if (t == 11) kv->f = (double)(int64_t)raw;
  else kv->f = (double)raw;
}

static const orc_kv* find_kv(const orc_model* m, const char* key) {
  for (int i = 0; i < m->n_kvs; i++)
    if (!strcmp(m->kvs[i].key, key)) return &m->kvs[i];
  return NULL;
}

static const orc_tensor* find_tensor(const orc_model* m, const char* name) {
  for (int i = 0; i < m->n_tensors; i++)
    if (!strcmp(m->tensors[i].name, name)) return &m->tensors[i];
  return NULL;
}

/* candle Value::to_u32 accepts only U32-typed values (quantized_llama::from_gguf) */
static int kv_u32(const orc_model* m, const char* key, int* out) {
  const orc_kv* kv = find_kv(m, key);
  if (!kv || kv->vtype != 4) return -1;
  *out = (int)kv->u;
  return 0;
}

static int kv_f32(const orc_model* m, const char* key, float* out) {
  const orc_kv* kv = find_kv(m, key);
  if (!kv || kv->vtype != 6) return -1;
  *out = (float)kv->f;
  return 0;
}

orc_model* orc_model_open(const char* path, char* err, int errlen) {
#define FAIL(...) do { if (err) snprintf(err, (size_t)errlen, __VA_ARGS__); orc_model_close(m); return NULL; } while (0)
  orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
  if (m) m->attn_fma = 1; /* candle's gemm crate on an FMA host (the x86-64-v3 hosts this runs on) */
  int fd = open(path, O_RDONLY);
  if (fd < 0) FAIL("open %s failed", path);
  struct stat st;
  fstat(fd, &st);
  m->map_len = (size_t)st.st_size;
  m->map = (uint8_t*)mmap(NULL, m->map_len, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (m->map == MAP_FAILED) { m->map = NULL; FAIL("mmap failed"); }
  rd_t r = {m->map, m->map + m->map_len, 0};
  if (rd_u(&r, 4) != 0x46554747u) FAIL("bad GGUF magic");
  uint32_t ver = (uint32_t)rd_u(&r, 4);
  if (ver < 2 || ver > 3) FAIL("unsupported GGUF version %u", ver);
  uint64_t nt = rd_u(&r, 8), nkv = rd_u(&r, 8);
  if (r.bad || nt > 100000 || nkv > 100000) FAIL("bad GGUF counts");
  m->kvs = (orc_kv*)calloc(nkv ? nkv : 1, sizeof(orc_kv));
  m->n_kvs = (int)nkv;
  for (uint64_t i = 0; i < nkv; i++) {
    rd_str(&r, m->kvs[i].key, sizeof(m->kvs[i].key));
    m->kvs[i].vtype = (int)rd_u(&r, 4);
    rd_value(&r, m->kvs[i].vtype, &m->kvs[i]);
    if (r.bad) FAIL("truncated metadata");
  }
  m->tensors = (orc_tensor*)calloc(nt ? nt : 1, sizeof(orc_tensor));
  m->n_tensors = (int)nt;
  for (uint64_t i = 0; i < nt; i++) {
    orc_tensor* t = &m->tensors[i];
    rd_str(&r, t->name, sizeof(t->name));
    t->n_dims = (int)rd_u(&r, 4);
    if (t->n_dims < 1 || t->n_dims > 4) FAIL("bad n_dims");
    for (int d = 0; d < 4; d++) t->ne[d] = 1;
    for (int d = 0; d < t->n_dims; d++) t->ne[d] = (int64_t)rd_u(&r, 8);
    t->type = (int)rd_u(&r, 4);
    t->offset = rd_u(&r, 8);
    if (r.bad) FAIL("truncated tensor info");
  }
  uint64_t align = 32;
  const orc_kv* al = find_kv(m, "general.alignment");
  if (al && al->vtype == 4) align = al->u;
  uint64_t pos = (uint64_t)(r.p - m->map);
  uint64_t data0 = (pos + align - 1) / align * align;
  for (int i = 0; i < m->n_tensors; i++) {
    orc_tensor* t = &m->tensors[i];
    int bs = orc_block_size(t->type);
    if (bs <= 0) continue; /* types the path does not use are left unmapped */
    int64_t ne = t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3];
    uint64_t bytes = (uint64_t)(ne / bs) * orc_type_size(t->type);
    if (data0 + t->offset + bytes > m->map_len) FAIL("tensor %s extends past end of file", t->name);
    t->data = m->map + data0 + t->offset;
  }
  /* metadata required by quantized_llama::ModelWeights::from_gguf */
  orc_model_cfg* c = &m->cfg;
  if (kv_u32(m, "llama.attention.head_count", &c->n_heads) ||
      kv_u32(m, "llama.attention.head_count_kv", &c->n_kv_heads) ||
      kv_u32(m, "llama.block_count", &c->n_layers) ||
      kv_u32(m, "llama.embedding_length", &c->embed) ||
      kv_u32(m, "llama.rope.dimension_count", &c->rope_dim) ||
      kv_f32(m, "llama.attention.layer_norm_rms_epsilon", &c->eps))
    FAIL("missing llama.* metadata");
  if (kv_f32(m, "llama.rope.freq_base", &c->rope_base)) c->rope_base = 10000.f;
  if (kv_u32(m, "llama.context_length", &c->ctx_len)) c->ctx_len = 4096;
  c->head_dim = c->embed / c->n_heads;
  m->tok_embd = find_tensor(m, "token_embd.weight");
  m->output = find_tensor(m, "output.weight");
  if (!m->output) m->output = m->tok_embd; /* quantized_llama falls back to tok_embeddings */
  const orc_tensor* on = find_tensor(m, "output_norm.weight");
  if (!m->tok_embd || !on || on->type != ORC_F32) FAIL("missing token_embd/output_norm");
  m->output_norm = (const float*)on->data;
  c->vocab = (int)m->tok_embd->ne[1];
  m->layers = (orc_layer*)calloc((size_t)c->n_layers, sizeof(orc_layer));
  for (int l = 0; l < c->n_layers; l++) {
    char nm[96];
#define GET(field, suffix)                                              \
  snprintf(nm, sizeof nm, "blk.%d.%s.weight", l, suffix);               \
  m->layers[l].field = find_tensor(m, nm);                              \
  if (!m->layers[l].field) FAIL("missing tensor %s", nm);
    GET(q, "attn_q") GET(k, "attn_k") GET(v, "attn_v") GET(o, "attn_output")
    GET(gate, "ffn_gate") GET(up, "ffn_up") GET(down, "ffn_down")
    const orc_tensor *an, *fn;
    snprintf(nm, sizeof nm, "blk.%d.attn_norm.weight", l);
    an = find_tensor(m, nm);
    snprintf(nm, sizeof nm, "blk.%d.ffn_norm.weight", l);
    fn = find_tensor(m, nm);
    if (!an || !fn || an->type != ORC_F32 || fn->type != ORC_F32) FAIL("missing norms in layer %d", l);
    m->layers[l].attn_norm = (const float*)an->data;
    m->layers[l].ffn_norm = (const float*)fn->data;
#undef GET
  }
  c->ffn = (int)m->layers[0].gate->ne[1];
  return m;
#undef FAIL
}

void orc_model_close(orc_model* m) {
  if (!m) return;
  if (m->map) munmap(m->map, m->map_len);
  free(m->tensors);
  free(m->kvs);
  free(m->layers);
  free(m->kcache);
  free(m->vcache);
  free(m->hidden);
  free(m);
}

void orc_model_get_cfg(const orc_model* m, orc_model_cfg* cfg) { *cfg = m->cfg; }

const void* orc_model_tensor(const orc_model* m, const char* name, int* type, int64_t* ne0,
                             int64_t* ne1) {
  const orc_tensor* t = find_tensor(m, name);
  if (!t) return NULL;
  if (type) *type = t->type;
  if (ne0) *ne0 = t->ne[0];
  if (ne1) *ne1 = t->ne[1];
  return t->data;
}

int orc_model_set_attn_fma(orc_model* m, int on) {
  m->attn_fma = on != 0;
  return 0;
}

int orc_model_reset(orc_model* m, int max_pos, int kv_f16) {
  const orc_model_cfg* c = &m->cfg;
  free(m->kcache);
  free(m->vcache);
  size_t n = (size_t)c->n_layers * c->n_kv_heads * (size_t)max_pos * c->head_dim;
  m->kcache = (float*)calloc(n, 4);
  m->vcache = (float*)calloc(n, 4);
  if (!m->hidden) m->hidden = (float*)calloc((size_t)c->embed, 4);
  m->max_pos = max_pos;
  m->kv_f16 = kv_f16;
  return (m->kcache && m->vcache) ? 0 : -1;
}

static size_t row_bytes(const orc_tensor* t) {
  return (size_t)(t->ne[0] / orc_block_size(t->type)) * orc_type_size(t->type);
}

static int mm(const orc_tensor* w, int64_t rows, const float* x, float* y, int nt) {
  return orc_matmul(w->type, rows, w->ne[0], w->ne[1], x, w->data, y, nt);
}

/* Decoder layers [l0, l1) of quantized_llama::ModelWeights::forward on the residual rows X
 * ([n][embed], updated in place) at positions pos0..pos0+n-1, writing the layers' K/V rows;
 * trace, when given, receives the rows entering each layer of the range and leaving the last
 * ([l1 - l0 + 1][n][embed]). */
static int layers_forward(orc_model* m, float* X, int n, int pos0, int l0, int l1, int nt, float* trace) {
  const orc_model_cfg* c = &m->cfg;
  const int H = c->embed, hd = c->head_dim, nq = c->n_heads, nkv = c->n_kv_heads, F = c->ffn;
  const int qd = nq * hd, kd = nkv * hd, half = c->rope_dim / 2;
  float* XN = (float*)malloc(sizeof(float) * (size_t)n * H);
  float* Q = (float*)malloc(sizeof(float) * (size_t)n * qd);
  float* K = (float*)malloc(sizeof(float) * (size_t)n * kd);
  float* V = (float*)malloc(sizeof(float) * (size_t)n * kd);
  float* A = (float*)malloc(sizeof(float) * (size_t)n * qd);
  float* O = (float*)malloc(sizeof(float) * (size_t)n * H);
  float* G = (float*)malloc(sizeof(float) * (size_t)n * F);
  float* U = (float*)malloc(sizeof(float) * (size_t)n * F);
  float* cs = (float*)malloc(sizeof(float) * (size_t)(pos0 + n) * half);
  float* sn = (float*)malloc(sizeof(float) * (size_t)(pos0 + n) * half);
  int rc = 0;
  rope_rows(c->rope_dim, c->rope_base, pos0, pos0 + n, cs, sn);
  for (int l = l0; l < l1; l++) {
    const orc_layer* L = &m->layers[l];
    if (trace) memcpy(trace + (size_t)(l - l0) * n * H, X, sizeof(float) * (size_t)n * H);
    for (int t = 0; t < n; t++) orc_rmsnorm(X + (size_t)t * H, L->attn_norm, H, c->eps, XN + (size_t)t * H);
    if ((rc = mm(L->q, n, XN, Q, nt)) || (rc = mm(L->k, n, XN, K, nt)) || (rc = mm(L->v, n, XN, V, nt))) goto done;
    const size_t lstride = (size_t)nkv * m->max_pos * hd;
    float* kc = m->kcache + (size_t)l * lstride;
    float* vc = m->vcache + (size_t)l * lstride;
    for (int t = 0; t < n; t++) {
      const int p = pos0 + t;
      orc_rope_i(Q + (size_t)t * qd, nq, hd, cs + (size_t)p * half, sn + (size_t)p * half);
      orc_rope_i(K + (size_t)t * kd, nkv, hd, cs + (size_t)p * half, sn + (size_t)p * half);
      for (int g = 0; g < nkv; g++)
        for (int d = 0; d < hd; d++) {
          float kv = K[(size_t)t * kd + g * hd + d], vv = V[(size_t)t * kd + g * hd + d];
          if (m->kv_f16) { kv = orc_fp16_to_f32(orc_f32_to_fp16(kv)); vv = orc_fp16_to_f32(orc_f32_to_fp16(vv)); }
          kc[((size_t)g * m->max_pos + p) * hd + d] = kv;
          vc[((size_t)g * m->max_pos + p) * hd + d] = vv;
        }
    }
    /* causal: position p attends to 0..p (the masked_fill(-inf) rows are exp()=0) */
    for (int t = 0; t < n; t++)
      attention_impl(Q + (size_t)t * qd, kc, vc, nq, nkv, hd, pos0 + t + 1, m->max_pos, A + (size_t)t * qd,
                     m->attn_fma);
    if ((rc = mm(L->o, n, A, O, nt))) goto done;
    for (size_t i = 0; i < (size_t)n * H; i++) X[i] = O[i] + X[i];
    for (int t = 0; t < n; t++) orc_rmsnorm(X + (size_t)t * H, L->ffn_norm, H, c->eps, XN + (size_t)t * H);
    if ((rc = mm(L->gate, n, XN, G, nt)) || (rc = mm(L->up, n, XN, U, nt))) goto done;
    for (size_t i = 0; i < (size_t)n * F; i++) G[i] = orc_silu(G[i]) * U[i];
    if ((rc = mm(L->down, n, G, O, nt))) goto done;
    for (size_t i = 0; i < (size_t)n * H; i++) X[i] = O[i] + X[i];
  }
  if (trace) memcpy(trace + (size_t)(l1 - l0) * n * H, X, sizeof(float) * (size_t)n * H);
done:
  free(XN); free(Q); free(K); free(V); free(A); free(O); free(G); free(U); free(cs); free(sn);
  return rc;
}

/* quantized_llama::ModelWeights::forward restated for tokens at pos0..pos0+n-1; trace, when
 * given, receives the residual rows entering each layer and leaving the last
 * ([n_layers + 1][n][embed]) */
int orc_model_forward_trace(orc_model* m, const uint32_t* tok, int n, int pos0, float* logits, int nt,
                            float* trace) {
  const orc_model_cfg* c = &m->cfg;
  if (!m->kcache || pos0 + n > m->max_pos || n <= 0) return -1;
  const int H = c->embed;
  float* X = (float*)malloc(sizeof(float) * (size_t)n * H);
  float* XN = (float*)malloc(sizeof(float) * (size_t)H);
  int rc = 0;
  /* embedding: candle dequantizes token_embd to f32 and index_selects rows */
  for (int t = 0; t < n; t++) {
    if (tok[t] >= (uint32_t)c->vocab) { rc = -2; goto done; }
    orc_dequant(m->tok_embd->type, m->tok_embd->data + (size_t)tok[t] * row_bytes(m->tok_embd),
                X + (size_t)t * H, H);
  }
  if ((rc = layers_forward(m, X, n, pos0, 0, c->n_layers, nt, trace))) goto done;
  memcpy(m->hidden, X + (size_t)(n - 1) * H, sizeof(float) * H);
  orc_rmsnorm(X + (size_t)(n - 1) * H, m->output_norm, H, c->eps, XN);
  rc = mm(m->output, 1, XN, logits, nt);
done:
  free(X); free(XN);
  return rc;
}

int orc_model_run_layers(orc_model* m, const float* x_in, int n, int pos0, int l0, int l1, float* x_out,
                         int nt) {
  const orc_model_cfg* c = &m->cfg;
  if (!m->kcache || pos0 + n > m->max_pos || n <= 0 || l0 < 0 || l1 > c->n_layers || l0 > l1) return -1;
  memcpy(x_out, x_in, sizeof(float) * (size_t)n * c->embed);
  return layers_forward(m, x_out, n, pos0, l0, l1, nt, NULL);
}

int orc_model_forward(orc_model* m, const uint32_t* tok, int n, int pos0, float* logits, int nt) {
  return orc_model_forward_trace(m, tok, n, pos0, logits, nt, NULL);
}

int orc_model_kv(const orc_model* m, int layer, float* k_out, float* v_out) {
  const orc_model_cfg* c = &m->cfg;
  if (!m->kcache || layer < 0 || layer >= c->n_layers) return -1;
  const size_t n = (size_t)c->n_kv_heads * m->max_pos * c->head_dim;
  memcpy(k_out, m->kcache + (size_t)layer * n, n * sizeof(float));
  memcpy(v_out, m->vcache + (size_t)layer * n, n * sizeof(float));
  return 0;
}

/* Benchmark aid: fill K/V of positions [0, n_pos) in every layer with seeded N(0,1)-shaped
 * values (a cheap xorshift sum of uniforms), so that decode steps from position n_pos on read as
 * many cached positions as after a real prompt of that length, without its prefill.  The
 * values are not a model's; only the amount of attention work is. */
int orc_model_prime_cache(orc_model* m, int n_pos, uint64_t seed) {
  const orc_model_cfg* c = &m->cfg;
  if (!m->kcache || n_pos < 0 || n_pos > m->max_pos) return -1;
  const size_t row = (size_t)c->head_dim;
  for (int l = 0; l < c->n_layers; l++)
    for (int g = 0; g < c->n_kv_heads; g++)
      for (int p = 0; p < n_pos; p++) {
        const size_t off = (((size_t)l * c->n_kv_heads + g) * m->max_pos + p) * row;
        for (size_t d = 0; d < row; d++) {
          float kv[2];
          for (int j = 0; j < 2; j++) {
            float s = 0.f;
            for (int u = 0; u < 3; u++) {
              seed ^= seed << 13; seed ^= seed >> 7; seed ^= seed << 17;
              s += (float)(seed >> 40) * (1.f / 16777216.f);
            }
            kv[j] = (s - 1.5f) * 2.f;
          }
          m->kcache[off + d] = m->kv_f16 ? orc_fp16_to_f32(orc_f32_to_fp16(kv[0])) : kv[0];
          m->vcache[off + d] = m->kv_f16 ? orc_fp16_to_f32(orc_f32_to_fp16(kv[1])) : kv[1];
        }
      }
  return 0;
}

int orc_model_last_hidden(const orc_model* m, float* out) {
  if (!m->hidden) return -1;
  memcpy(out, m->hidden, sizeof(float) * (size_t)m->cfg.embed);
  return 0;
}
