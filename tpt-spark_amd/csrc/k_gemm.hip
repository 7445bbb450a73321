// Prefill GEMM on MFMA: Y[M,N] = X[M,K] . W[N,K]^T with W in GGUF Q4_K, Q5_K or Q6_K blocks
// (uploaded unchanged), for M >= 16 tokens at once.
//
// Replaces the prefill of the reference engines: WgpuEngine runs one whole forward pass per
// prompt position through dequant_and_gemm + gemm.wgsl at M=1 (wgpu_engine.rs:254-261,
// 581-605); CandleEngine runs a batched forward whose QMatMul quantizes every activation row
// to Q8_K and takes integer dot products (candle_engine.rs:272-273; candle 0.8.4
// k_quants::matmul).  Two modes:
//  * GEMM_Q8K (the model's prefill): candle's arithmetic.  The activation arrives as Q8_K rows
//    (int8 q, f32 d per 256, per-16 sums); the weight tile is decoded into LDS as the exact
//    integers sc_j * q (<= 63 * 15, exact in fp16).  One MFMA chain covers at most 128
//    elements, so every partial sum is an integer below 2^24 and exact in f32; the two halves
//    of a super-block add with one rounding, as (float)isum does in candle.  The mins term
//    sum_j m_j * bsum_j is one more K=16 MFMA (per-16 sums <= 2032 and mins <= 63: exact).
//    Per block, in f32 as candle: y += (d_w * d_x) * isum - (dmin_w * d_x) * msum.
//    Q6_K weights (candle's vec_dot_q6k_q8k: y += d_w d_x sum_j sc_j sum (q - 32) q8): the
//    integer w = sc_j * (q - 32) lies in [-4064, 4096], past fp16's exact range, so it is
//    split as w = 64 w1 + w0 (w1 in [-64, 64], w0 in [0, 63], both exact in fp16) and two
//    chains hi += q8 . w1, lo += q8 . w0 run over the whole super-block (|partial| < 2^22,
//    exact); isum = 64 hi + lo rounds once.
//    Q5_K weights (vec_dot_q5k_q8k: Q4_K's arithmetic with 5-bit q): w = sc_j * q <= 63 * 31 is
//    exact in fp16, but 128-element chains could pass 2^24, so w takes Q6_K's split (w = 64 w1 +
//    w0, two chains over the super-block) and the mins term Q4_K's K=16 MFMA.
//  * GEMM_Q80 (Q8_0 and Q4_0 weights: vec_dot_q8_0_q8_0 / vec_dot_q4_0_q8_0): the activation
//    arrives as Q8_0 rows (int8 q, f16-rounded d per 32); the weight tile holds the exact integers
//    q (Q8_0) or q - 8 (Q4_0).  One MFMA chain per 32-element block (|sum| <= 32 * 127 * 128,
//    exact), scaled per block as candle does, y += (isum * d_w) * d_x.
//  * GEMM_F16: the tile is dequantized into LDS as fp16 (Q4_K: d*sc*q - dmin*m, Q6_K:
//    d*sc*(q - 32), rounded to fp16; F16 weights as stored), the activation is fp16, one fp32
//    MFMA chain over all of K.  For F16 weights candle multiplies in f32: the caller runs the
//    GEMM twice, on x's fp16 rounding and on the fp16 rounding of the remainder (products exact
//    in the f32 accumulator, x carried to 2^-22 relative).
// Tiling (MI355X: 160 KB LDS, wave64, v_mfma_f32_32x32x16_f16): 512 threads, a 128 x 128 tile
// of Y per workgroup, each wave 64 x 32 (2 x 1 MFMA tiles), two waves per SIMD so that one
// wave's weight decode and block scaling run while the other's MFMAs do.  K advances half a super-block (128)
// per step through a double-buffered LDS tile: while a step's MFMAs read one buffer, the next
// step's weights are decoded into the other and the step after that is in flight from HBM, so
// the Q4_K decode overlaps the matrix cores instead of alternating with them.  The activation
// arrives as fp16 rows from act_prep_kernel (in GEMM_Q8K mode the int8 values, exact in fp16), so
// no workgroup converts it again.
// Q4_K GEMMs of at least 256 rows run on gemm_wide_kernel instead: 256 x 128 tiles, 64 x 64 per
// wave, activation tiles fetched two steps ahead by LDS DMA, one exact chain per super-block on
// the shifted integers sc * q - 480 (same results, bit for bit).
#include <hip/hip_ext.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "kernels.h"

namespace tpt {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
// native 16-byte vector (HIP's uint4 is a struct: its copies go through private memory)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int GT = 512;          // threads per workgroup
constexpr int BM = 128, BN = 128, BK = 128;
constexpr int LDG = 16;          // per-16 sums / mins row

// One K step's operands, rows of BK fp16 (256 B) without padding: the 16-byte chunk c of row r
// sits at chunk position c ^ (r % 16), so that the 16 rows one MFMA operand read touches per
// chunk column spread over all banks, and every operand read and staging write is one aligned
// 16-byte LDS access.
struct GemmTile {
  __attribute__((aligned(16))) _Float16 a[BM * BK];
  __attribute__((aligned(16))) _Float16 b[BN * BK];
};
// element index of (row r, column k) in a tile, k a multiple of 8
__device__ __forceinline__ int sw(int r, int k) { return r * BK + ((((k >> 3) ^ (r & 15))) << 3); }
struct GemmBlock {               // GEMM_Q8K: one super-block's per-row and per-column data
  _Float16 a16[BM][LDG];         // activation per-16 sums
  _Float16 b16[BN][LDG];         // weight mins, each repeated for its two 16-element halves
  float dx[BM];                  // activation block scale
  float dw[BN], dm[BN];          // weight d, dmin
};
struct GemmQ80 {                 // GEMM_Q80: one K step's block scales (4 blocks of 32)
  __attribute__((aligned(16))) float dwT[BN][4];  // weight d per tile column and block
  __attribute__((aligned(16))) float dxT[4][BM];  // activation d per block and tile row
};
struct GemmSmem {
  GemmTile t[2];                 // by step parity: the half of the super-block
  GemmBlock blk[2];              // by super-block parity
  GemmQ80 q80[2];                // by step parity
};

// Registers one thread stages for a K step (thread = row r = tid / 4, quarter qt = tid % 4 of
// the step's 128 elements): 32 fp16 activation values and the weight bytes of those 32
// elements; in the first half of a super-block also the row's block scale (and, for Q4_K, 4 of
// its per-16 sums).
//  * Q4_K: the block header (d, dmin, packed scales) and 16 qs bytes of group 2 hb + qt / 2
//    (the low nibbles are 16 elements of sub-block 2g, the high nibbles 16 of sub-block 2g + 1).
//  * Q6_K: quad qt of the half: its 32 ql bytes, the half's 32 qh bytes, the half's 8 int8
//    scales and d (210-byte blocks are only 2-byte aligned: 16-bit loads).
//  * Q5_K: Q4_K's header and 16 qs bytes, and the 16 qh bytes of the same l (bits 2g, 2g + 1
//    are the fifth bits of sub-blocks 2g, 2g + 1); 176-byte blocks stay 16-byte aligned.
template <int WT> struct Stage;
template <> struct Stage<TPT_TYPE_Q4_K> {
  u32x4 a[4];
  u32x4 h;
  u32x4 q;
  u32x2 a16;
  float dx;
};
template <> struct Stage<TPT_TYPE_Q6_K> {
  u32x4 a[4];
  u32x4 ql[2];
  u32x4 qh[2];
  u32x2 sc;
  uint32_t d;
  float dx;
};
template <> struct Stage<TPT_TYPE_Q5_K> {
  u32x4 a[4];
  u32x4 h;
  u32x4 q;
  u32x4 qh;
  u32x2 a16;
  float dx;
};
// Q8_0 / Q4_0: the 32-element block kb * 8 + 4 HB + qt of the row (its d, its quants) and the
// activation block's d; F16: the 32 weights as stored.
template <> struct Stage<TPT_TYPE_Q8_0> {
  u32x4 a[4];
  u32x4 q[2];
  uint32_t d;
  float dx;
};
template <> struct Stage<TPT_TYPE_Q4_0> {
  u32x4 a[4];
  u32x4 q;
  uint32_t d;
  float dx;
};
template <> struct Stage<TPT_TYPE_F16> {
  u32x4 a[4];
  u32x4 w[4];
};

// Q4_K and Q5_K share the header (d, dmin, packed scales and mins) and the per-16 mins term
template <int WT> constexpr bool has_mins() { return WT == TPT_TYPE_Q4_K || WT == TPT_TYPE_Q5_K; }
// Q6_K and Q5_K keep w = 64 w1 + w0 in two exact chains over the whole super-block
template <int WT> constexpr bool split_w() { return WT == TPT_TYPE_Q6_K || WT == TPT_TYPE_Q5_K; }

__device__ __forceinline__ void get_scale_min(const u32x4& h, int j, int* sc, int* m) {
  // get_scale_min_k4 (ggml/candle): scales bytes s[0..11] are h.y, h.z, h.w
  const uint32_t Y = h.y, Z = h.z, W = h.w;
  if (j < 4) {
    *sc = (Y >> (8 * j)) & 63;
    *m = (Z >> (8 * j)) & 63;
  } else {
    const int k = j - 4;
    *sc = ((W >> (8 * k)) & 0xF) | (((Y >> (8 * k + 6)) & 3) << 4);
    *m = ((W >> (8 * k + 4)) & 0xF) | (((Z >> (8 * k + 6)) & 3) << 4);
  }
}

// step = 2 kb + hb: super-block kb, half hb
template <int WT, int MODE, int HB>
__device__ __forceinline__ void stage_load(const GemmArgs& g, int m0, int n0, int kb, Stage<WT>& st) {
  const int tid = threadIdx.x, r = tid >> 2, qt = tid & 3;
  int m = m0 + r;
  if (m >= g.M) m = g.M - 1;
  int n = n0 + r;
  if (n >= g.N) n = g.N - 1;
  const u32x4* src = (const u32x4*)(g.af + (size_t)m * g.K + (size_t)kb * 256 + 128 * HB + 32 * qt);
#pragma unroll
  for (int i = 0; i < 4; i++) st.a[i] = src[i];
  if constexpr (WT == TPT_TYPE_Q4_K) {
    const uint8_t* blk = g.w + (size_t)n * g.w_stride + (size_t)kb * 144;
    st.h = *(const u32x4*)blk;
    st.q = *(const u32x4*)(blk + 16 + 32 * (2 * HB + (qt >> 1)) + 16 * (qt & 1));
    if constexpr (MODE == GEMM_Q8K && HB == 0)
      st.a16 = *(const u32x2*)(g.as16 + (size_t)m * (g.K / 16) + kb * 16 + 4 * qt);
  } else if constexpr (WT == TPT_TYPE_Q8_0 || WT == TPT_TYPE_Q4_0) {
    const int bi = kb * 8 + 4 * HB + qt;  // 34- / 18-byte blocks: 2-byte aligned
    const uint8_t* blk = g.w + (size_t)n * g.w_stride + (size_t)bi * (WT == TPT_TYPE_Q8_0 ? 34 : 18);
    st.d = ldg_u<uint16_t>(blk);
    if constexpr (WT == TPT_TYPE_Q8_0) {
      st.q[0] = ldg_u<u32x4>(blk + 2);
      st.q[1] = ldg_u<u32x4>(blk + 18);
    } else {
      st.q = ldg_u<u32x4>(blk + 2);
    }
    st.dx = g.ad[(size_t)m * (g.K / 32) + bi];
  } else if constexpr (WT == TPT_TYPE_F16) {
    const u32x4* wr = (const u32x4*)(g.w + (size_t)n * g.w_stride + ((size_t)kb * 256 + 128 * HB + 32 * qt) * 2);
#pragma unroll
    for (int i = 0; i < 4; i++) st.w[i] = wr[i];
  } else if constexpr (WT == TPT_TYPE_Q5_K) {
    const uint8_t* blk = g.w + (size_t)n * g.w_stride + (size_t)kb * 176;
    st.h = *(const u32x4*)blk;
    st.qh = *(const u32x4*)(blk + 16 + 16 * (qt & 1));
    st.q = *(const u32x4*)(blk + 48 + 32 * (2 * HB + (qt >> 1)) + 16 * (qt & 1));
    if constexpr (MODE == GEMM_Q8K && HB == 0)
      st.a16 = *(const u32x2*)(g.as16 + (size_t)m * (g.K / 16) + kb * 16 + 4 * qt);
  } else {
    // 2-byte aligned rows: 32-bit words assembled from aligned 16-bit loads
    const uint16_t* blk = (const uint16_t*)(g.w + (size_t)n * g.w_stride + (size_t)kb * 210);
    auto w32 = [&](int byte_off) {
      return (uint32_t)blk[byte_off / 2] | ((uint32_t)blk[byte_off / 2 + 1] << 16);
    };
    auto w128 = [&](int byte_off) {
      return u32x4{w32(byte_off), w32(byte_off + 4), w32(byte_off + 8), w32(byte_off + 12)};
    };
    const int qlo = 64 * HB + 32 * (qt & 1);  // ql bytes of quad qt
#pragma unroll
    for (int i = 0; i < 2; i++) st.ql[i] = w128(qlo + 16 * i);
#pragma unroll
    for (int i = 0; i < 2; i++) st.qh[i] = w128(128 + 32 * HB + 16 * i);
    st.sc = u32x2{w32(192 + 8 * HB), w32(196 + 8 * HB)};
    st.d = blk[104];
  }
  if constexpr (MODE == GEMM_Q8K && HB == 0) st.dx = g.ad[(size_t)m * (g.K / 256) + kb];
}

typedef _Float16 half2 __attribute__((ext_vector_type(2)));
typedef short short2 __attribute__((ext_vector_type(2)));

template <int WT, int MODE, int HB>
__device__ __forceinline__ void stage_store(const Stage<WT>& st, GemmTile& T, GemmBlock& B, GemmQ80& Q) {
  const int tid = threadIdx.x, r = tid >> 2, qt = tid & 3;
#pragma unroll
  for (int i = 0; i < 4; i++) *(u32x4*)&T.a[sw(r, 32 * qt + 8 * i)] = st.a[i];
  float d = 0.f, dmin = 0.f;
  if constexpr (WT == TPT_TYPE_Q8_0 || WT == TPT_TYPE_Q4_0) {
    // the block's 32 integers q (Q8_0) or q - 8 (Q4_0, element j < 16: low nibble of qs[j],
    // j + 16: its high nibble) as exact fp16: a biased byte ORed into the mantissa of 1024.0
    // and the bias subtracted in packed fp16
    const half2 bias = WT == TPT_TYPE_Q8_0 ? half2{(_Float16)1152.f, (_Float16)1152.f}
                                           : half2{(_Float16)1032.f, (_Float16)1032.f};
#pragma unroll
    for (int c = 0; c < 4; c++) {  // elements 8c .. 8c + 7 of the block
      u32x4 o;
#pragma unroll
      for (int h = 0; h < 2; h++) {
        uint32_t x;
        if constexpr (WT == TPT_TYPE_Q8_0) {
          x = st.q[c >> 1][2 * (c & 1) + h] ^ 0x80808080u;  // int8 + 128
        } else {
          const uint32_t wq = st.q[2 * (c & 1) + h];
          x = (c < 2 ? wq : wq >> 4) & 0x0F0F0F0Fu;
        }
        const uint32_t p01 = __builtin_amdgcn_perm(0u, x, 0x0c010c00u) | 0x64006400u;
        const uint32_t p23 = __builtin_amdgcn_perm(0u, x, 0x0c030c02u) | 0x64006400u;
        o[2 * h] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2, p01) - bias);
        o[2 * h + 1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2, p23) - bias);
      }
      *(u32x4*)&T.b[sw(r, 32 * qt + 8 * c)] = o;
    }
    Q.dwT[r][qt] = h2f((uint16_t)st.d);
    Q.dxT[qt][r] = st.dx;
  } else if constexpr (WT == TPT_TYPE_F16) {
#pragma unroll
    for (int c = 0; c < 4; c++) *(u32x4*)&T.b[sw(r, 32 * qt + 8 * c)] = st.w[c];
  } else if constexpr (WT == TPT_TYPE_Q4_K) {
    // weight row r, group g = 2 HB + qt / 2: qs[32g + l] holds element 64g + l (low nibble,
    // sub-block 2g) and 64g + 32 + l (high nibble, sub-block 2g + 1); this thread has
    // l = 16 (qt % 2) .. + 15, tile columns c0 + l' and c0 + 32 + l'
    const int g = 2 * HB + (qt >> 1);
    const int c0 = 64 * (qt >> 1) + 16 * (qt & 1);
    d = h2f((uint16_t)(st.h.x & 0xffff));
    dmin = h2f((uint16_t)(st.h.x >> 16));
    int sc0, m0, sc1, m1;
    get_scale_min(st.h, 2 * g, &sc0, &m0);
    get_scale_min(st.h, 2 * g + 1, &sc1, &m1);
    if constexpr (MODE == GEMM_Q8K) {
      // the integers sc * q two at a time in packed fp16, all exact: a byte pair (b, b') moved
      // to the two halves, its nibbles ORed into the mantissa of 1024.0 (0x6400) give 1024 + q;
      // one fused multiply-add (1024 + q) * sc - 1024 sc rounds once, onto the integer
      // sc * q <= 945 < 2048 (1024 sc <= 64512 is exact in fp16)
      const half2 s0 = {(_Float16)sc0, (_Float16)sc0}, s1 = {(_Float16)sc1, (_Float16)sc1};
      const half2 o0 = {(_Float16)(-1024 * sc0), (_Float16)(-1024 * sc0)};
      const half2 o1 = {(_Float16)(-1024 * sc1), (_Float16)(-1024 * sc1)};
      auto dec = [&](uint32_t pair, half2 sc, half2 off) {
        const half2 v = __builtin_bit_cast(half2, (pair & 0x000F000Fu) | 0x64006400u);
        return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(v, sc, off));
      };
#pragma unroll
      for (int c = 0; c < 2; c++) {  // 8 consecutive elements per 16-byte store
        u32x4 lo, hi;
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const uint32_t x = st.q[2 * c + h];
          const uint32_t p01 = __builtin_amdgcn_perm(0u, x, 0x0c010c00u);  // bytes 0, 1 -> halves
          const uint32_t p23 = __builtin_amdgcn_perm(0u, x, 0x0c030c02u);  // bytes 2, 3 -> halves
          lo[2 * h] = dec(p01, s0, o0);
          lo[2 * h + 1] = dec(p23, s0, o0);
          hi[2 * h] = dec(p01 >> 4, s1, o1);
          hi[2 * h + 1] = dec(p23 >> 4, s1, o1);
        }
        *(u32x4*)&T.b[sw(r, c0 + 8 * c)] = lo;
        *(u32x4*)&T.b[sw(r, c0 + 32 + 8 * c)] = hi;
      }
      // mins of sub-blocks 2g, 2g + 1, each for its two 16-element halves (16-sums 8g .. 8g+3)
      const half2 mm0 = {(_Float16)m0, (_Float16)m0}, mm1 = {(_Float16)m1, (_Float16)m1};
      *(u32x2*)&B.b16[r][4 * g] = u32x2{__builtin_bit_cast(uint32_t, mm0), __builtin_bit_cast(uint32_t, mm1)};
      if constexpr (HB == 0) {
        u32x2 v;
#pragma unroll
        for (int j = 0; j < 2; j++) {
          const half2 p = {(_Float16)(int16_t)(st.a16[j] & 0xffff), (_Float16)(int16_t)(st.a16[j] >> 16)};
          v[j] = __builtin_bit_cast(uint32_t, p);
        }
        *(u32x2*)&B.a16[r][4 * qt] = v;
      }
    } else {
      const float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
      const float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
#pragma unroll
      for (int c = 0; c < 2; c++) {  // 8 consecutive elements per half8 store
        half8 lo, hi;
#pragma unroll
        for (int t = 0; t < 8; t++) {
          const uint32_t byte = (st.q[2 * c + t / 4] >> (8 * (t % 4))) & 0xff;
          lo[t] = (_Float16)(d1 * (float)(byte & 0xF) - mm1);
          hi[t] = (_Float16)(d2 * (float)(byte >> 4) - mm2);
        }
        *(half8*)&T.b[sw(r, c0 + 8 * c)] = lo;
        *(half8*)&T.b[sw(r, c0 + 32 + 8 * c)] = hi;
      }
    }
  } else if constexpr (WT == TPT_TYPE_Q5_K) {
    // as Q4_K (group g = 2 HB + qt / 2, l = 16 (qt % 2) .. + 15), q = nibble + 16 * bit 2g (low)
    // or 2g + 1 (high) of qh[l]
    const int g = 2 * HB + (qt >> 1);
    const int c0 = 64 * (qt >> 1) + 16 * (qt & 1);
    d = h2f((uint16_t)(st.h.x & 0xffff));
    dmin = h2f((uint16_t)(st.h.x >> 16));
    int sc0, m0, sc1, m1;
    get_scale_min(st.h, 2 * g, &sc0, &m0);
    get_scale_min(st.h, 2 * g + 1, &sc1, &m1);
#pragma unroll
    for (int c = 0; c < 2; c++) {  // 8 consecutive elements (two qs / qh words) per store
      uint32_t vlo[2], vhi[2];
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const uint32_t x = st.q[2 * c + h], hb = st.qh[2 * c + h];
        vlo[h] = (x & 0x0F0F0F0Fu) | (((hb >> (2 * g)) & 0x01010101u) << 4);
        vhi[h] = ((x >> 4) & 0x0F0F0F0Fu) | (((hb >> (2 * g + 1)) & 0x01010101u) << 4);
      }
      if constexpr (MODE == GEMM_Q8K) {
        // w = sc * q <= 1953 as w + 4096 = 64 u + w0 stored as the bytes (w0, u), the layout of
        // the Q6_K tile (the MFMA operands are then u - 64 and w0)
        auto split = [&](const uint32_t (&v)[2], int sc) {
          const short2 s2 = {(short)sc, (short)sc}, c2 = {(short)4096, (short)4096};
          u32x4 o;
#pragma unroll
          for (int h = 0; h < 2; h++) {
            const uint32_t p01 = __builtin_amdgcn_perm(0u, v[h], 0x0c010c00u);
            const uint32_t p23 = __builtin_amdgcn_perm(0u, v[h], 0x0c030c02u);
            const uint32_t w01 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(short2, p01) * s2 + c2);
            const uint32_t w23 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(short2, p23) * s2 + c2);
            o[2 * h] = ((w01 << 2) & 0xFF00FF00u) | (w01 & 0x003F003Fu);
            o[2 * h + 1] = ((w23 << 2) & 0xFF00FF00u) | (w23 & 0x003F003Fu);
          }
          return o;
        };
        *(u32x4*)&T.b[sw(r, c0 + 8 * c)] = split(vlo, sc0);
        *(u32x4*)&T.b[sw(r, c0 + 32 + 8 * c)] = split(vhi, sc1);
      } else {
        const float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
        const float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
        half8 lo, hi;
#pragma unroll
        for (int t = 0; t < 8; t++) {
          lo[t] = (_Float16)(d1 * (float)((vlo[t / 4] >> (8 * (t % 4))) & 0xff) - mm1);
          hi[t] = (_Float16)(d2 * (float)((vhi[t / 4] >> (8 * (t % 4))) & 0xff) - mm2);
        }
        *(half8*)&T.b[sw(r, c0 + 8 * c)] = lo;
        *(half8*)&T.b[sw(r, c0 + 32 + 8 * c)] = hi;
      }
    }
    if constexpr (MODE == GEMM_Q8K) {
      const half2 mm0 = {(_Float16)m0, (_Float16)m0}, mm1 = {(_Float16)m1, (_Float16)m1};
      *(u32x2*)&B.b16[r][4 * g] = u32x2{__builtin_bit_cast(uint32_t, mm0), __builtin_bit_cast(uint32_t, mm1)};
      if constexpr (HB == 0) {
        u32x2 v;
#pragma unroll
        for (int j = 0; j < 2; j++) {
          const half2 p = {(_Float16)(int16_t)(st.a16[j] & 0xffff), (_Float16)(int16_t)(st.a16[j] >> 16)};
          v[j] = __builtin_bit_cast(uint32_t, p);
        }
        *(u32x2*)&B.a16[r][4 * qt] = v;
      }
    }
  } else {
    // Q6_K half HB of a super-block, elements 32 Q + l of the half (quad Q, l < 32):
    //   q = ((ql[32 (Q & 1) + l] >> 4 (Q >= 2)) & 15) | ((qh[l] >> 2 Q) & 3) << 4,
    //   scale sc[2 Q + l / 16], weight d * scale * (q - 32).
    // Thread qt holds quad Q = qt (tile columns 32 qt + l).
    d = h2f((uint16_t)st.d);
    const int sh = 4 * (qt >> 1), shh = 2 * qt;
    const uint32_t scw = qt >= 2 ? st.sc[1] : st.sc[0];  // scales 4 (qt / 2) .. + 3
    const int sA = (int)(int8_t)(scw >> (16 * (qt & 1))), sB = (int)(int8_t)(scw >> (16 * (qt & 1) + 8));
#pragma unroll
    for (int c = 0; c < 4; c++) {   // elements 8c .. 8c + 7 of the quad
      const int s = c < 2 ? sA : sB;
      uint32_t qv[2];
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const int wi = 2 * c + h;  // ql / qh word of elements 4 wi .. 4 wi + 3
        const uint32_t x = st.ql[wi / 4][wi % 4], hb = st.qh[wi / 4][wi % 4];
        qv[h] = ((x >> sh) & 0x0F0F0F0Fu) | (((hb >> shh) & 0x03030303u) << 4);
      }
      if constexpr (MODE == GEMM_Q8K) {
        // w = s * (q - 32) in [-4064, 4096] as w + 4096 = 64 u + w0 (u <= 128, w0 < 64), stored
        // per element as the bytes (w0, u): the MFMA operands w1 = u - 64 and w0 are then exact
        // fp16 values with w = 64 w1 + w0
        const short2 s2 = {(short)s, (short)s}, c2 = {(short)(4096 - 32 * s), (short)(4096 - 32 * s)};
        u32x4 o;
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const uint32_t p01 = __builtin_amdgcn_perm(0u, qv[h], 0x0c010c00u);
          const uint32_t p23 = __builtin_amdgcn_perm(0u, qv[h], 0x0c030c02u);
          const uint32_t w01 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(short2, p01) * s2 + c2);
          const uint32_t w23 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(short2, p23) * s2 + c2);
          o[2 * h] = ((w01 << 2) & 0xFF00FF00u) | (w01 & 0x003F003Fu);
          o[2 * h + 1] = ((w23 << 2) & 0xFF00FF00u) | (w23 & 0x003F003Fu);
        }
        *(u32x4*)&T.b[sw(r, 32 * qt + 8 * c)] = o;
      } else {
        const float ds = d * (float)s;
        half8 v;
#pragma unroll
        for (int t = 0; t < 8; t++) v[t] = (_Float16)(ds * (float)((int)((qv[t / 4] >> (8 * (t % 4))) & 0xff) - 32));
        *(half8*)&T.b[sw(r, 32 * qt + 8 * c)] = v;
      }
    }
  }
  if constexpr (MODE == GEMM_Q8K && HB == 0) {
    // the four threads of the row hold the same values: the duplicate stores keep the step one
    // basic block for the scheduler
    B.dx[r] = st.dx;
    B.dw[r] = d;
    B.dm[r] = dmin;
  }
}

// One K step of MFMAs on tile T (each wave: 64 x 32 as 2 x 1 tiles of 32 x 32).  Q4_K and the
// fp16 mode: acc += A . B.  Q6_K in GEMM_Q8K mode: the B tile holds the bytes (w0, u) of each
// weight; two exact chains, hi += A . (u - 64) and lo += A . w0.  FRESH: the chains start here
// (the first MFMA takes a zero accumulator operand, so no registers are cleared per block).
template <int WT, int MODE, bool FRESH = false>
__device__ __forceinline__ void mfma_step(const GemmTile& T, floatx16 (&acc)[2], floatx16 (&lo)[2]) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = wid >> 2, wn = wid & 3;
  const int lr = lane & 31, lk = 8 * (lane >> 5);
#pragma unroll
  for (int kk = 0; kk < BK; kk += 16) {
    half8 a[2];
#pragma unroll
    for (int i = 0; i < 2; i++) a[i] = *(const half8*)&T.a[sw(64 * wm + 32 * i + lr, kk + lk)];
    if constexpr (split_w<WT>() && MODE == GEMM_Q8K) {
      const u32x4 raw = *(const u32x4*)&T.b[sw(32 * wn + lr, kk + lk)];
      const half2 k1088 = {(_Float16)1088.f, (_Float16)1088.f}, k1024 = {(_Float16)1024.f, (_Float16)1024.f};
      u32x4 h, l;
#pragma unroll
      for (int c = 0; c < 4; c++) {  // bytes (w0, u) of two weights -> fp16 1024 + u, 1024 + w0
        h[c] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2, __builtin_amdgcn_perm(0x64646464u, raw[c], 0x04030401u)) - k1088);
        l[c] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2, __builtin_amdgcn_perm(0x64646464u, raw[c], 0x04020400u)) - k1024);
      }
      const half8 bh = __builtin_bit_cast(half8, h), bl = __builtin_bit_cast(half8, l);
#pragma unroll
      for (int i = 0; i < 2; i++) {
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bh, FRESH && kk == 0 ? floatx16{} : acc[i], 0, 0, 0);
        lo[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bl, FRESH && kk == 0 ? floatx16{} : lo[i], 0, 0, 0);
      }
    } else {
      const half8 b = *(const half8*)&T.b[sw(32 * wn + lr, kk + lk)];
#pragma unroll
      for (int i = 0; i < 2; i++)
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b, FRESH && kk == 0 ? floatx16{} : acc[i], 0, 0, 0);
    }
  }
}

// GEMM_Q80: one K step = four 32-element blocks; per block one exact chain of two MFMAs, then
// y += (isum * d_w) * d_x per element (the last multiply fused with the add).
__device__ __forceinline__ void mfma_step_q80(const GemmTile& T, const GemmQ80& Q, floatx16 (&out)[2]) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = wid >> 2, wn = wid & 3;
  const int lr = lane & 31, lk = 8 * (lane >> 5);
  const float4 dw4 = *(const float4*)&Q.dwT[32 * wn + lr][0];
  const float dw[4] = {dw4.x, dw4.y, dw4.z, dw4.w};
#pragma unroll
  for (int j = 0; j < 4; j++) {
    floatx16 c[2];
#pragma unroll
    for (int t = 0; t < 2; t++) {
      const int kk = 32 * j + 16 * t;
      half8 a[2];
#pragma unroll
      for (int i = 0; i < 2; i++) a[i] = *(const half8*)&T.a[sw(64 * wm + 32 * i + lr, kk + lk)];
      const half8 b = *(const half8*)&T.b[sw(32 * wn + lr, kk + lk)];
#pragma unroll
      for (int i = 0; i < 2; i++) c[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b, t == 0 ? floatx16{} : c[i], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
      float dxs[16];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float4 v = *(const float4*)&Q.dxT[j][64 * wm + 32 * i + q * 8 + (lane >> 5) * 4];
        dxs[4 * q] = v.x; dxs[4 * q + 1] = v.y; dxs[4 * q + 2] = v.z; dxs[4 * q + 3] = v.w;
      }
#pragma unroll
      for (int e = 0; e < 16; e++) out[i][e] = fmaf(c[i][e] * dw[j], dxs[e], out[i][e]);
    }
  }
}

// GEMM_Q8K end of a super-block, per element in f32: candle's y += d_x (d_w isum - dmin_w msum)
// with the integers exact (the same terms as candle's (d_w d_x) isum - (dmin_w d_x) msum; the
// f32 roundings differ by an ulp).  Q4_K: isum = the two exact 128-element chains added once,
// the mins term sum_j m_j * bsum_j on the matrix cores (K = 16, exact); per element one add and
// three (fused) multiplies.  Q6_K: isum = 64 hi + lo (64 hi exact, one rounding); no mins term.
template <int WT>
__device__ __forceinline__ void block_end(const GemmBlock& B, floatx16 (&acc0)[2], floatx16 (&acc1)[2],
                                          floatx16 (&out)[2]) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = wid >> 2, wn = wid & 3;
  const int lr = lane & 31, lk = 8 * (lane >> 5);
  const int col = 32 * wn + lr;
  const float dw = B.dw[col];
  half8 b;
  float dm = 0.f;
  if constexpr (has_mins<WT>()) {
    b = *(const half8*)&B.b16[col][lk];
    dm = B.dm[col];
  }
#pragma unroll
  for (int i = 0; i < 2; i++) {
    // the lane's 16 rows of tile i are 4 runs of 4 consecutive rows: one float4 each
    float dxs[16];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const float4 v = *(const float4*)&B.dx[64 * wm + 32 * i + q * 8 + (lane >> 5) * 4];
      dxs[4 * q] = v.x; dxs[4 * q + 1] = v.y; dxs[4 * q + 2] = v.z; dxs[4 * q + 3] = v.w;
    }
    if constexpr (has_mins<WT>()) {
      const half8 a = *(const half8*)&B.a16[64 * wm + 32 * i + lr][lk];
      const floatx16 accm = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, floatx16{}, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 16; e++) {
        // Q4_K: the two exact half chains; Q5_K: 64 hi + lo
        const float isum = split_w<WT>() ? fmaf(64.f, acc0[i][e], acc1[i][e]) : acc0[i][e] + acc1[i][e];
        const float t = fmaf(dw, isum, -(dm * accm[e]));
        out[i][e] = fmaf(dxs[e], t, out[i][e]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const float isum = fmaf(64.f, acc0[i][e], acc1[i][e]);
        out[i][e] = fmaf(dxs[e], dw * isum, out[i][e]);
      }
    }
  }
}

template <int WT, int MODE>
__global__ void __launch_bounds__(GT, 1) gemm_kernel(const GemmArgs g) {
  __shared__ GemmSmem s;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = wid >> 2, wn = wid & 3;  // wave tile: rows 64 wm .., cols 32 wn ..
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  // split-K (small M): split blockIdx.z of gridDim.z takes super-blocks [kb0, kb1)
  const int nkb_all = g.K / 256, ns = gridDim.z, sz = blockIdx.z;
  const int kb0 = sz * nkb_all / ns, nkb = (sz + 1) * nkb_all / ns;
  const int lr = lane & 31;
  // chains: Q4_K q8k acc0 / acc1 = the two halves of a super-block; Q6_K q8k acc0 / acc1 =
  // hi / lo over the whole super-block; fp16 mode: out directly
  constexpr bool Q6 = split_w<WT>();  // Q6_K, Q5_K: hi / lo chains over the super-block

  floatx16 out[2], acc0[2], acc1[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    out[i] = floatx16{};
    acc0[i] = floatx16{};
    acc1[i] = floatx16{};
  }

  // prologue: step 0 in LDS, step 1 in registers
  Stage<WT> st;
  stage_load<WT, MODE, 0>(g, m0, n0, kb0, st);
  stage_store<WT, MODE, 0>(st, s.t[0], s.blk[kb0 & 1], s.q80[0]);
  stage_load<WT, MODE, 1>(g, m0, n0, kb0, st);
  __syncthreads();
  for (int kb = kb0; kb < nkb; kb++) {
    // past the last block the next block is the last one again (clamped), staged into the tile
    // and block buffer that are not read again
    const int kn = kb + 1 < nkb ? kb + 1 : kb;
    // first half of super-block kb (tile t[0]): stage the second half, fetch the next block's
    // first half
    stage_store<WT, MODE, 1>(st, s.t[1], s.blk[kb & 1], s.q80[1]);
    stage_load<WT, MODE, 0>(g, m0, n0, kn, st);
    if constexpr (MODE == GEMM_Q8K) mfma_step<WT, MODE, true>(s.t[0], acc0, acc1);
    else if constexpr (MODE == GEMM_Q80) mfma_step_q80(s.t[0], s.q80[0], out);
    else mfma_step<WT, MODE>(s.t[0], out, out);
    __syncthreads();
    // second half (tile t[1]): stage the next block's first half, fetch its second half
    stage_store<WT, MODE, 0>(st, s.t[0], s.blk[(kb + 1) & 1], s.q80[0]);
    stage_load<WT, MODE, 1>(g, m0, n0, kn, st);
    if constexpr (MODE == GEMM_Q8K) {
      if constexpr (Q6) mfma_step<WT, MODE>(s.t[1], acc0, acc1);
      else mfma_step<WT, MODE, true>(s.t[1], acc1, acc1);
    } else if constexpr (MODE == GEMM_Q80) {
      mfma_step_q80(s.t[1], s.q80[1], out);
    } else {
      mfma_step<WT, MODE>(s.t[1], out, out);
    }
    if constexpr (MODE == GEMM_Q8K) block_end<WT>(s.blk[kb & 1], acc0, acc1, out);
    __syncthreads();
  }

  // epilogue: y[m][n] = out (+ resid[m][n]); split-K: this split's partial sums
  const int n = n0 + 32 * wn + lr;
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int e = 0; e < 16; e++) {
      const int m = m0 + 64 * wm + 32 * i + (e / 4) * 8 + (lane >> 5) * 4 + (e % 4);
      if (m < g.M && n < g.N) {
        float v = out[i][e];
        if (ns > 1) {
          g.part[((size_t)sz * g.M + m) * g.N + n] = v;
        } else {
          if (g.resid) v = v + g.resid[(size_t)m * g.ldr + n];
          g.y[(size_t)m * g.ldy + n] = v;
        }
      }
    }
}

// ---------------------------------------------------------------------------------------------
// Q4_K weights with M > 128: 256 x 128 tiles.  Each wave computes 64 x 64 of Y (2 x 2 MFMA
// tiles), so a K step reads 4 KB of LDS operands per 4 MFMAs (the 128 x 128 kernel: 3 KB per 2)
// and one decoded weight tile serves 256 activation rows.  K advances 64 per step, one Q4_K group
// (the low and high nibbles of 32 qs bytes: sub-blocks 2g and 2g + 1), four steps per super-block,
// through a double-buffered tile of 128-byte rows.
// GEMM_Q8K: one exact chain per super-block.  The tile holds w - 480 for w = sc * q in [0, 945],
// so every partial sum is an integer of magnitude at most 256 * 128 * 480 < 2^24 (exact in f32),
// and isum = chain + 480 * sum(q8) is formed by one more MFMA on the chain (two exact products,
// one rounding): the rounding of the exact integer, the value the two half chains of the 128 x
// 128 kernel give.  The rest of the block arithmetic is
// that kernel's, so both produce the same bits.
constexpr int WBM = 256, WBN = 128, WBK = 64;
constexpr int WOFF = 480;  // a multiple of 32: 1024 sc + WOFF is exact in fp16 up to sc = 63
// Rows of 64 fp16 (128 bytes, half of gfx950's 64 LDS banks): the 16-byte chunk c of row r sits
// at c ^ f((r / 2) % 8), f a permutation.  One 16-lane group of an MFMA operand read covers rows
// r0 .. r0 + 15 at one chunk column: the even rows fill one half of the banks, the odd rows the
// other, and within each half f gives the 8 rows 8 distinct chunk positions.  A rows: f =
// identity (written by DMA, whole 1 KB runs).  B rows: f(x) = 4 (x % 2) + x / 2, so that the two
// rows of equal parity in one 16-lane store group (4 rows, 4 threads each writing one chunk of
// the same half of a row) land in opposite halves of the chunk positions.
__device__ __forceinline__ int swa(int r, int k) { return r * WBK + (((k >> 3) ^ ((r >> 1) & 7)) << 3); }
__device__ __forceinline__ int swb(int r, int k) {
  const int x = (r >> 1) & 7;
  return r * WBK + (((k >> 3) ^ (((x & 1) << 2) | (x >> 1))) << 3);
}
struct WideBlock {               // GEMM_Q8K: one super-block's per-row and per-column data
  _Float16 a16[WBM][LDG];        // activation per-16 sums
  _Float16 b16[WBN][LDG];        // weight mins, each repeated for its two 16-element halves
  float dx[WBM];                 // activation block scale
  uint32_t sx[WBM];              // the activation row's sum of q8 over the super-block, S = 64 h + l
                                 // (h, l of S's sign, |h| <= 512, |l| <= 63), as the fp16 pair (h, l)
  float dw[WBN], dm[WBN];        // weight d, dmin
};
// 158 KB: activation tiles by step mod 3 (the DMA runs two steps ahead), weight tiles by step
// parity, block data by super-block parity
struct WideSmem {
  __attribute__((aligned(16))) _Float16 a[3][WBM * WBK];
  __attribute__((aligned(16))) _Float16 b[2][WBN * WBK];
  WideBlock blk[2];
};
// Registers a thread stages for a K step: weight row tid / 4, qs bytes 8 (tid % 4) .. + 7 of the
// step's group.  With the super-block's first step also that weight row's header (d, dmin,
// scales: kept for the other three steps) and, in GEMM_Q8K mode, 8 of the per-16 sums of
// activation row tid / 2 (sums 8 (tid % 2) .. + 7) and its block scale.  The activation tile
// goes from memory to LDS directly (wide_dma_a).
struct WideStage {
  u32x2 q;
  u32x4 h;
  u32x4 a16;
  float dx;
};
// A thread's byte offsets from the operand bases, fixed over the K loop (32-bit: the launcher
// keeps every operand below 4 GiB, so loads take a uniform base plus one offset register): its
// DMA lane's offset within a group of 8 activation rows (row l / 8 and the chunk that position
// l % 8 holds, for groups of even (a0) and odd (a1) index), its weight row, its activation row's
// per-16 sums and block scales.  The tile's rows and columns all lie inside the matrices (the
// last tiles are shifted back, see gemm_wide_kernel), so no index is clamped.
struct WideOff {
  uint32_t a0, a1, w, s16, sd;
};
__device__ __forceinline__ WideOff wide_offsets(const GemmArgs& g, int m0, int n0) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int p = lane & 7, rr = lane >> 3;
  WideOff o;
  // row 8 k + rr of the tile: (row / 2) % 8 = 4 (k % 2) + rr / 2
  o.a0 = (uint32_t)rr * (uint32_t)g.K * 2u + 16u * (uint32_t)(p ^ (rr >> 1));
  o.a1 = (uint32_t)rr * (uint32_t)g.K * 2u + 16u * (uint32_t)(p ^ ((rr >> 1) + 4));
  const uint32_t m = (uint32_t)(m0 + (tid >> 1)), n = (uint32_t)(n0 + (tid >> 2));
  o.w = n * (uint32_t)g.w_stride;
  o.s16 = m * (uint32_t)(g.K / 16) * 2u + 16u * (uint32_t)(tid & 1);
  o.sd = m * (uint32_t)(g.K / 256) * 4u;
  return o;
}

template <int MODE, int S>
__device__ __forceinline__ void wide_load(const GemmArgs& g, const WideOff& o, int kb, WideStage& st) {
  const uint32_t bo = o.w + (uint32_t)kb * 144u;
  if constexpr (S == 0) st.h = *(const u32x4*)(g.w + bo);
  st.q = *(const u32x2*)(g.w + (bo + 16u + 32u * S + 8u * (threadIdx.x & 3)));
  if constexpr (MODE == GEMM_Q8K && S == 0) {
    st.a16 = *(const u32x4*)((const char*)g.as16 + (o.s16 + (uint32_t)kb * 32u));
    st.dx = *(const float*)((const char*)g.ad + (o.sd + (uint32_t)kb * 4u));
  }
}

// The activation tile of step S of super-block kb, by LDS DMA (global_load_lds_dwordx4: lane l of
// a wave writes the 16 bytes at LDS offset 16 l of the instruction's 1 KB): wave w's instruction i
// fills rows 8 (4 w + i) .. + 7, lane l position l % 8 of row 8 (4 w + i) + l / 8, which holds
// the chunk swa places there.  Complete once the wave's vector memory count drains.
template <int S>
__device__ __forceinline__ void wide_dma_a(const GemmArgs& g, const WideOff& o, int m0, int kb, _Float16* A) {
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar bases
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t r0 = (uint32_t)(m0 + 8 * (4 * w + i));  // the instruction's first row
    const char* base = (const char*)g.af + (r0 * (uint32_t)g.K * 2u + (uint32_t)kb * 512u + 2u * WBK * S);
    __builtin_amdgcn_global_load_lds(base + (i & 1 ? o.a1 : o.a0), (__attribute__((address_space(3))) void*)&A[8 * WBK * (4 * w + i)], 16, 0, 0);
  }
}

// s_waitcnt vmcnt(N): at most N of this wave's global loads (LDS DMA included) are in flight;
// vector memory loads complete in issue order
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 16, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

template <int MODE, int S>
__device__ __forceinline__ void wide_store(const WideStage& st, _Float16* Bt, WideBlock& B) {
  const int tid = threadIdx.x, ra = tid >> 1, ha = tid & 1, rb = tid >> 2, qt = tid & 3;
  // qs byte 32 S + l holds element l of sub-block 2 S (low nibble) and of 2 S + 1 (high); this
  // thread has l = 8 qt .. + 7: tile columns 8 qt .. and 32 + 8 qt ..
  int sc0, m0, sc1, m1;
  get_scale_min(st.h, 2 * S, &sc0, &m0);
  get_scale_min(st.h, 2 * S + 1, &sc1, &m1);
  const float d = h2f((uint16_t)(st.h.x & 0xffff)), dmin = h2f((uint16_t)(st.h.x >> 16));
  if constexpr (MODE == GEMM_Q8K) {
    // sc * q - 480 two at a time: (1024 + q) * sc - (1024 sc + 480) in one packed fp16 fma,
    // whose single rounding lands on the exact integer (|sc q - 480| <= 480)
    const half2 s0 = {(_Float16)sc0, (_Float16)sc0}, s1 = {(_Float16)sc1, (_Float16)sc1};
    const half2 o0 = {(_Float16)(-1024 * sc0 - WOFF), (_Float16)(-1024 * sc0 - WOFF)};
    const half2 o1 = {(_Float16)(-1024 * sc1 - WOFF), (_Float16)(-1024 * sc1 - WOFF)};
    auto dec = [&](uint32_t pair, half2 sc, half2 off) {
      const half2 v = __builtin_bit_cast(half2, (pair & 0x000F000Fu) | 0x64006400u);
      return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(v, sc, off));
    };
    u32x4 lo, hi;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const uint32_t x = st.q[h];
      const uint32_t p01 = __builtin_amdgcn_perm(0u, x, 0x0c010c00u);  // bytes 0, 1 -> halves
      const uint32_t p23 = __builtin_amdgcn_perm(0u, x, 0x0c030c02u);  // bytes 2, 3 -> halves
      lo[2 * h] = dec(p01, s0, o0);
      lo[2 * h + 1] = dec(p23, s0, o0);
      hi[2 * h] = dec(p01 >> 4, s1, o1);
      hi[2 * h + 1] = dec(p23 >> 4, s1, o1);
    }
    *(u32x4*)&Bt[swb(rb, 8 * qt)] = lo;
    *(u32x4*)&Bt[swb(rb, 32 + 8 * qt)] = hi;
    if constexpr (S == 0) {
      // the weight row's d, dmin and mins (this thread: sub-blocks 2 qt, 2 qt + 1); the four
      // threads of the row store the same d and dmin
      // get_scale_min_k4's mins for j = 2 qt + c: byte j of Z (low 6 bits) for j < 4, else the
      // high nibble of W's byte j - 4 with Z's byte j - 4's top two bits (selected, not branched)
      auto min_of = [&](int c) {
        const int sh = 8 * ((2 * qt + c) & 3);
        const int lo = (int)((st.h.z >> sh) & 63);
        const int hi = (int)(((st.h.w >> (sh + 4)) & 0xF) | (((st.h.z >> (sh + 6)) & 3) << 4));
        return qt < 2 ? lo : hi;
      };
      const int ma = min_of(0), mb = min_of(1);
      const half2 mma = {(_Float16)ma, (_Float16)ma}, mmb = {(_Float16)mb, (_Float16)mb};
      *(u32x2*)&B.b16[rb][4 * qt] = u32x2{__builtin_bit_cast(uint32_t, mma), __builtin_bit_cast(uint32_t, mmb)};
      B.dw[rb] = d;
      B.dm[rb] = dmin;
      // the activation row's per-16 sums (exact fp16), block scale and 480 * sum(q8); the row's
      // two threads are adjacent lanes
      u32x4 v;
      int s = 0;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int lo16 = (int16_t)(st.a16[j] & 0xffff), hi16 = (int16_t)(st.a16[j] >> 16);
        const half2 p = {(_Float16)lo16, (_Float16)hi16};
        v[j] = __builtin_bit_cast(uint32_t, p);
        s += lo16 + hi16;
      }
      *(u32x4*)&B.a16[ra][8 * ha] = v;
      const float fs = (float)s;               // |s| <= 128 * 128: exact
      const float tot = fs + dpp_mov<0xB1>(fs);  // + the other half of the row (lane ^ 1), exact
      B.dx[ra] = st.dx;
      const int sum = (int)tot, h = sum / 64, l = sum - 64 * h;  // truncating: l has the sum's sign
      const half2 hl = {(_Float16)h, (_Float16)l};
      B.sx[ra] = __builtin_bit_cast(uint32_t, hl);
    }
  } else {
    const float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
    const float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
    half8 lo, hi;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      const uint32_t byte = (st.q[t / 4] >> (8 * (t % 4))) & 0xff;
      lo[t] = (_Float16)(d1 * (float)(byte & 0xF) - mm1);
      hi[t] = (_Float16)(d2 * (float)(byte >> 4) - mm2);
    }
    *(half8*)&Bt[swb(rb, 8 * qt)] = lo;
    *(half8*)&Bt[swb(rb, 32 + 8 * qt)] = hi;
  }
}

// One K step of MFMAs on tiles A, Bt: wave (wm, wn) = (wid / 2, wid % 2) computes rows 64 wm ..
// + 63, columns 64 wn .. + 63 as 2 x 2 tiles.  FRESH: the chains start here (zero accumulator
// operand).
template <bool FRESH>
__device__ __forceinline__ void wide_mfma(const _Float16* A, const _Float16* Bt, floatx16 (&acc)[2][2]) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = wid >> 1, wn = wid & 1;
  const int lr = lane & 31, lk = 8 * (lane >> 5);
#pragma unroll
  for (int kk = 0; kk < WBK; kk += 16) {
    half8 a[2], b[2];
#pragma unroll
    for (int i = 0; i < 2; i++) a[i] = *(const half8*)&A[swa(64 * wm + 32 * i + lr, kk + lk)];
#pragma unroll
    for (int j = 0; j < 2; j++) b[j] = *(const half8*)&Bt[swb(64 * wn + 32 * j + lr, kk + lk)];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int j = 0; j < 2; j++)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], FRESH && kk == 0 ? floatx16{} : acc[i][j], 0, 0, 0);
  }
}

// GEMM_Q8K end of a super-block, per element in f32 as the 128 x 128 kernel's block_end:
// isum = chain + 480 sum(q8) (one rounding), y += d_x * fma(d_w, isum, -d_min * msum), the mins
// term msum on the matrix cores (K = 16, exact).  The 480 sum(q8) term is added on the matrix
// cores too: one MFMA with the chain as accumulator and two nonzero products per element,
// 30720 h + 480 l = 480 (64 h + l) (exact, same sign as the sum), in place of an f32 add per
// element.
__device__ __forceinline__ void wide_block_end(const WideBlock& B, floatx16 (&acc)[2][2], floatx16 (&out)[2][2]) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = wid >> 1, wn = wid & 1;
  const int lr = lane & 31, lk = 8 * (lane >> 5);
  half8 bsx = {};  // B operand of the 480 sum(q8) MFMA: rows k = 0, 1 hold 64 * 480 and 480
  if (lane < 32) {
    bsx[0] = (_Float16)(64 * WOFF);
    bsx[1] = (_Float16)WOFF;
  }
  // isum = chain + 480 sum(q8), in place, for the four tiles first
#pragma unroll
  for (int i = 0; i < 2; i++) {
    half8 asx = {};  // A operand: row 64 wm + 32 i + lr's pair (h, l) at k = 0, 1
    if (lane < 32) {
      const half2 hl = __builtin_bit_cast(half2, B.sx[64 * wm + 32 * i + lr]);
      asx[0] = hl[0];
      asx[1] = hl[1];
    }
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(asx, bsx, acc[i][j], 0, 0, 0);
  }
  float dw[2], dm[2];
  half8 bm[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int col = 64 * wn + 32 * j + lr;
    dw[j] = B.dw[col];
    dm[j] = B.dm[col];
    bm[j] = *(const half8*)&B.b16[col][lk];
  }
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int r0 = 64 * wm + 32 * i;
    // the lane's 16 rows of tile i are 4 runs of 4 consecutive rows: one float4 each
    float dxs[16];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int r = r0 + q * 8 + (lane >> 5) * 4;
      const float4 v = *(const float4*)&B.dx[r];
      dxs[4 * q] = v.x; dxs[4 * q + 1] = v.y; dxs[4 * q + 2] = v.z; dxs[4 * q + 3] = v.w;
    }
    const half8 am = *(const half8*)&B.a16[r0 + lr][lk];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const floatx16 accm = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bm[j], floatx16{}, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const float t = fmaf(dw[j], acc[i][j][e], -(dm[j] * accm[e]));
        out[i][j][e] = fmaf(dxs[e], t, out[i][j][e]);
      }
    }
  }
}

// Workgroup barrier of the K loop: this wave's LDS stores complete, then s_barrier, in one asm
// statement with a memory clobber (no memory access moves across it).  __syncthreads() would add
// a release fence, which also waits for every LDS DMA in flight: the tiles fetched ahead.
__device__ __forceinline__ void wide_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Vector memory operations one phase issues: 4 DMA and the weight loads of the step two ahead
// (its qs bytes; with a super-block's first step also the header and, in GEMM_Q8K mode, the
// activation sums and scale)
template <int MODE, int S>
constexpr int phase_vm() {
  return 4 + 1 + ((S + 2) % 4 == 0 ? (MODE == GEMM_Q8K ? 3 : 1) : 0);
}

// Step p = (kb, S) of the K loop: this step's MFMAs (at S = 3 also the super-block's end), the
// weight tile of step p + 1 from the registers loaded one phase earlier, then the activation DMA
// of step p + 2 into its tile and the weight registers of step p + 2; the barrier follows once
// every load issued before this phase has landed (this phase's own stay in flight).  The DMA is
// issued after the phase's LDS stores: the compiler makes an LDS store wait for every LDS DMA in
// flight (it cannot tell their addresses apart), which here are the previous phase's, landed by
// then.  ia: this step's activation tile; kn: the next super-block (clamped).
template <int MODE, int S>
__device__ __forceinline__ void wide_phase(const GemmArgs& g, const WideOff& o, int m0, int kb, int kn, int ia,
                                           WideSmem& s, WideStage& st, floatx16 (&acc)[2][2], floatx16 (&out)[2][2]) {
  constexpr bool Q8 = MODE == GEMM_Q8K;
  const int ia2 = ia == 0 ? 2 : ia - 1;  // (ia + 2) % 3
  const int kb2 = S < 2 ? kb : kn;       // the super-block of step p + 2
  if constexpr (Q8) wide_mfma<S == 0>(s.a[ia], s.b[S & 1], acc);
  else wide_mfma<false>(s.a[ia], s.b[S & 1], out);
  if constexpr (Q8 && S == 3) wide_block_end(s.blk[kb & 1], acc, out);
  wide_store<MODE, (S + 1) % 4>(st, s.b[(S + 1) & 1], s.blk[S == 3 ? (kb + 1) & 1 : kb & 1]);
  wide_dma_a<(S + 2) % 4>(g, o, m0, kb2, s.a[ia2]);
  wide_load<MODE, (S + 2) % 4>(g, o, kb2, st);
  // the two waves of a SIMD reach the barrier together, so their MFMAs and their VALU work
  // (the next tile's decode, the block end) cannot overlap each other; inside each wave, seven
  // VALU instructions after every MFMA keep the VALU busy while the matrix core runs
  // (q8k M=2048: +2-3% against the compiler's own order with six; since the 480 sum(q8) term
  // moved onto the matrix cores seven gain 2-3% more on gate|up and down; 4, 5, 8, 9 measured
  // lower)
#pragma unroll
  for (int i = 0; i < 16; i++) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    __builtin_amdgcn_sched_group_barrier(0x002, 7, 0);  // seven VALU
  }
  wait_vm<phase_vm<MODE, S>()>();
  wide_barrier();
}

template <int MODE>
__global__ void __launch_bounds__(GT, 1) gemm_wide_kernel(const GemmArgs g) {
  __shared__ WideSmem s;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = wid >> 1, wn = wid & 1;
  // the tile's output rows / columns [m_lo, ..), [n_lo, ..); the last tiles are computed from
  // origins shifted back so that every row and column read lies inside the matrices (M >= 256,
  // N >= 128), and store only their own part
  const int m_lo = blockIdx.y * WBM, n_lo = blockIdx.x * WBN;
  const int m0 = min(m_lo, g.M - WBM), n0 = min(n_lo, g.N - WBN);
  // split-K (small grids): split blockIdx.z of gridDim.z takes super-blocks [kb0, kb1)
  const int nkb_all = g.K / 256, ns = gridDim.z, sz = blockIdx.z;
  const int kb0 = sz * nkb_all / ns, nkb = (sz + 1) * nkb_all / ns;
  const int lr = lane & 31;

  floatx16 out[2][2], acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) out[i][j] = floatx16{};

  // prologue: step 0 in LDS, step 1's activation DMA in flight and its weights in registers
  const WideOff o = wide_offsets(g, m0, n0);
  WideStage st;
  wide_dma_a<0>(g, o, m0, kb0, s.a[0]);
  wide_load<MODE, 0>(g, o, kb0, st);
  wide_store<MODE, 0>(st, s.b[0], s.blk[kb0 & 1]);
  wide_dma_a<1>(g, o, m0, kb0, s.a[1]);
  wide_load<MODE, 1>(g, o, kb0, st);
  wait_vm<5>();  // step 0's DMA has landed
  __syncthreads();
  int ia = 0;
  auto next = [](int i) { return i == 2 ? 0 : i + 1; };
  for (int kb = kb0; kb < nkb; kb++) {
    // past the last block the next block is the last one again (clamped), staged into tiles and
    // a block buffer that are not read again
    const int kn = kb + 1 < nkb ? kb + 1 : kb;
    wide_phase<MODE, 0>(g, o, m0, kb, kn, ia, s, st, acc, out);
    ia = next(ia);
    wide_phase<MODE, 1>(g, o, m0, kb, kn, ia, s, st, acc, out);
    ia = next(ia);
    wide_phase<MODE, 2>(g, o, m0, kb, kn, ia, s, st, acc, out);
    ia = next(ia);
    wide_phase<MODE, 3>(g, o, m0, kb, kn, ia, s, st, acc, out);
    ia = next(ia);
  }
  wait_vm<0>();  // the DMA of the steps past the end lands before the workgroup's LDS is released

  // epilogue: y[m][n] = out (+ resid[m][n]); split-K: this split's partial sums
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int n = n0 + 64 * wn + 32 * j + lr;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int m = m0 + 64 * wm + 32 * i + (e / 4) * 8 + (lane >> 5) * 4 + (e % 4);
        if (m >= m_lo && n >= n_lo) {
          float v = out[i][j][e];
          if (ns > 1) {
            g.part[((size_t)sz * g.M + m) * g.N + n] = v;
          } else {
            if (g.resid) v = v + g.resid[(size_t)m * g.ldr + n];
            g.y[(size_t)m * g.ldy + n] = v;
          }
        }
      }
  }
}

// Split-K sum: y[m][n] = sum over splits s = 0, 1, .. of part[s][m][n] (+ resid[m][n])
__global__ void __launch_bounds__(256) gemm_split_reduce_kernel(const GemmArgs g, int ns) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x, mn = (size_t)g.M * g.N;
  if (i >= mn) return;
  const int m = (int)(i / g.N), n = (int)(i % g.N);
  float v = g.part[i];
  for (int k = 1; k < ns; k++) v = v + g.part[(size_t)k * mn + i];
  if (g.resid) v = v + g.resid[(size_t)m * g.ldr + n];
  g.y[(size_t)m * g.ldy + n] = v;
}

// One workgroup (4 waves) per activation row: optional SwiGLU (candle: silu(w1 x) * (w3 x)),
// optional rms_norm (m = sqrt(sum(x^2)/K + eps), y = x / m * w), then per 256-block the Q8_K
// quantization of BlockQ8K::from_float (the GEMV prologue's arithmetic) or fp16 conversion.
__global__ void __launch_bounds__(256) act_prep_kernel(const ActPrepArgs a) {
  __shared__ float red[4];
  const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int K = a.K, nb = K / 256;
  const float4* xr = (const float4*)(a.x + (size_t)m * a.ldx);
  const float4* ur = a.x2 ? (const float4*)(a.x2 + (size_t)m * a.ldx) : nullptr;
  auto value = [&](int i) {  // element group i (4 floats) after SwiGLU
    float4 v = xr[i];
    if (ur) {
      const float4 u = ur[i];
      v.x = silu_mul(v.x, u.x);
      v.y = silu_mul(v.y, u.y);
      v.z = silu_mul(v.z, u.z);
      v.w = silu_mul(v.w, u.w);
    }
    return v;
  };
  float rms = 1.f;
  if (a.norm_w) {
    float ss = 0.f;
    for (int i = tid; i < K / 4; i += 256) {
      const float4 v = value(i);
      ss = fmaf(v.x, v.x, ss);
      ss = fmaf(v.y, v.y, ss);
      ss = fmaf(v.z, v.z, ss);
      ss = fmaf(v.w, v.w, ss);
    }
    ss = wave_sum_dpp(ss);
    if (lane == 0) red[wid] = ss;
    __syncthreads();
    rms = sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)K + a.eps);
  }
  const float4* nw = (const float4*)a.norm_w;
  for (int b = wid; b < nb; b += 4) {
    float4 v = value(b * 64 + lane);
    if (nw) {
      const float4 w = nw[b * 64 + lane];
      v.x = v.x / rms * w.x;
      v.y = v.y / rms * w.y;
      v.z = v.z / rms * w.z;
      v.w = v.w / rms * w.w;
    }
    const float e[4] = {v.x, v.y, v.z, v.w};
    uint2* dst = (uint2*)(a.af + (size_t)m * K + (size_t)b * 256) + lane;
    if (a.mode == GEMM_Q8K) {  // the int8 values, stored as (exact) fp16 for the MFMA operand
      int qsum;
      float d;
      const int packed = q8k_block_wave(e, &qsum, &d);
      uint2 h;
      h.x = (uint32_t)f2h((float)(int8_t)(packed & 0xff)) | ((uint32_t)f2h((float)(int8_t)((packed >> 8) & 0xff)) << 16);
      h.y = (uint32_t)f2h((float)(int8_t)((packed >> 16) & 0xff)) | ((uint32_t)f2h((float)(int8_t)(packed >> 24)) << 16);
      *dst = h;
      if ((lane & 3) == 0) a.as16[(size_t)m * (K / 16) + b * 16 + (lane >> 2)] = (int16_t)qsum;
      if (lane == 0) a.ad[(size_t)m * nb + b] = d;
    } else if (a.mode == GEMM_Q80) {
      // BlockQ8_0::from_float per 32 (8 lanes): d = amax / 127 (stored rounded to f16),
      // q = round(x / d) through id = 1 / d of the unrounded d -- the decode GEMV's prologue
      float amax = fmaxf(fmaxf(fabsf(e[0]), fabsf(e[1])), fmaxf(fabsf(e[2]), fabsf(e[3])));
      amax = fmaxf(amax, dpp_mov<0xB1>(amax));   // max over the 8 lanes of the block
      amax = fmaxf(amax, dpp_mov<0x4E>(amax));
      amax = fmaxf(amax, dpp_mov<0x141>(amax));
      const float d = amax / 127.f;
      const float id = d != 0.f ? 1.f / d : 0.f;
      uint16_t q[4];
#pragma unroll
      for (int j = 0; j < 4; j++) q[j] = f2h(fminf(fmaxf(roundf(e[j] * id), -128.f), 127.f));
      *dst = make_uint2((uint32_t)q[0] | ((uint32_t)q[1] << 16), (uint32_t)q[2] | ((uint32_t)q[3] << 16));
      if ((lane & 7) == 0) a.ad[(size_t)m * (K / 32) + b * 8 + (lane >> 3)] = h2f(f2h(d));
    } else {
      uint16_t h[4], l[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        h[j] = f2h(e[j]);
        l[j] = f2h(e[j] - h2f(h[j]));  // exact difference, rounded once
      }
      *dst = make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
      if (a.af2)
        ((uint2*)(a.af2 + (size_t)m * K + (size_t)b * 256))[lane] =
            make_uint2((uint32_t)l[0] | ((uint32_t)l[1] << 16), (uint32_t)l[2] | ((uint32_t)l[3] << 16));
    }
  }
}

}  // namespace

int launch_act_prep(const ActPrepArgs& a, hipStream_t s) {
  if (a.M <= 0 || a.K <= 0 || a.K % 256 || a.ldx < a.K || a.ldx % 4) return fail(TPT_ERR_INVALID, "act_prep: bad shape");
  if (!a.x) return fail(TPT_ERR_INVALID, "act_prep: null input");
  if (a.mode != GEMM_Q8K && a.mode != GEMM_F16 && a.mode != GEMM_Q80) return fail(TPT_ERR_INVALID, "act_prep: bad mode");
  if (!a.af || (a.mode == GEMM_Q8K && (!a.ad || !a.as16)) || (a.mode == GEMM_Q80 && !a.ad))
    return fail(TPT_ERR_INVALID, "act_prep: null output");
  hipLaunchKernelGGL(act_prep_kernel, dim3((unsigned)a.M), dim3(256), 0, s, a);
  TPT_HIP(hipGetLastError());
  return TPT_OK;
}

int launch_gemm(const GemmArgs& g, hipStream_t s) { return launch_gemm_timed(g, s, nullptr, nullptr); }

namespace {

// Q4_K GEMMs of at least 256 rows and 128 columns take the 256 x 128 kernel (its last tiles are
// shifted back inside the matrices), when every operand offset fits 32 bits; TPT_HIP_GEMM_TILE=
// narrow forces the 128 x 128 kernel (comparisons and timing).
bool gemm_wide(const GemmArgs& g) {
  if (g.wtype != TPT_TYPE_Q4_K || g.M < WBM || g.N < WBN) return false;
  if ((uint64_t)g.M * (uint64_t)g.K * 2u >= (1ull << 32) || (uint64_t)g.N * g.w_stride >= (1ull << 32)) return false;
  const char* e = getenv("TPT_HIP_GEMM_TILE");
  return !(e && !strcmp(e, "narrow"));
}

constexpr int kRound = 256;  // workgroups the device runs at once (one per CU)

// Splits of K for a grid of `tiles` output tiles that cannot fill the 256 CUs: the most that
// still run in one round (tiles x splits <= 256), at least two super-blocks per split, at most 8.
int splits_for(int tiles, int nkb) {
  if (tiles > 128 || nkb < 4) return 1;
  int ns = 256 / tiles;
  ns = std::min(ns, nkb / 2);
  return std::min(ns, 8);
}

}  // namespace

int launch_gemm_timed(const GemmArgs& g, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  if (g.M <= 0 || g.N <= 0 || g.K <= 0 || g.K % 256) return fail(TPT_ERR_INVALID, "gemm: K must be a positive multiple of 256, M and N positive");
  const bool kq = g.wtype == TPT_TYPE_Q4_K || g.wtype == TPT_TYPE_Q5_K || g.wtype == TPT_TYPE_Q6_K;
  const bool q80 = g.wtype == TPT_TYPE_Q8_0 || g.wtype == TPT_TYPE_Q4_0;
  if (!kq && !q80 && g.wtype != TPT_TYPE_F16)
    return fail(TPT_ERR_UNSUPPORTED, "gemm: weight type must be Q4_K, Q5_K, Q6_K, Q8_0, Q4_0 or F16");
  if ((kq && g.mode != GEMM_Q8K && g.mode != GEMM_F16) || (q80 && g.mode != GEMM_Q80) ||
      (g.wtype == TPT_TYPE_F16 && g.mode != GEMM_F16))
    return fail(TPT_ERR_INVALID, "gemm: activation mode does not match the weight type");
  if (!g.w || !g.y) return fail(TPT_ERR_INVALID, "gemm: null weight/output pointer");
  if (!g.af) return fail(TPT_ERR_INVALID, "gemm: null activation rows");
  if ((g.mode == GEMM_Q8K && (!g.ad || (g.wtype != TPT_TYPE_Q6_K && !g.as16))) || (g.mode == GEMM_Q80 && !g.ad))
    return fail(TPT_ERR_INVALID, "gemm: quantized activations need block scales (and per-16 sums for Q4_K and Q5_K)");
  if (((uintptr_t)g.af % 16) || ((uintptr_t)g.as16 % 16))
    return fail(TPT_ERR_INVALID, "gemm: activation rows and per-16 sums must be 16-byte aligned");
  if (g.w_stride < row_bytes(g.wtype, g.K))
    return fail(TPT_ERR_INVALID, "gemm: weight row stride shorter than a row");
  const bool a16 = g.wtype == TPT_TYPE_Q4_K || g.wtype == TPT_TYPE_Q5_K || g.wtype == TPT_TYPE_F16;
  if (a16 && ((g.w_stride % 16) || ((uintptr_t)g.w % 16)))
    return fail(TPT_ERR_INVALID, "gemm: Q4_K, Q5_K and F16 weight rows must be 16-byte aligned");
  if (!a16 && ((g.w_stride % 2) || ((uintptr_t)g.w % 2)))
    return fail(TPT_ERR_INVALID, "gemm: Q6_K, Q8_0 and Q4_0 weight rows must be 2-byte aligned");
  const bool wide = gemm_wide(g);
  const int tm = wide ? WBM : BM;
  const int tiles = ((g.N + BN - 1) / BN) * ((g.M + tm - 1) / tm);
  int ns = splits_for(tiles, g.K / 256);
  if (!g.part || g.part_floats < (size_t)ns * g.M * g.N) ns = 1;  // no workspace: one pass over K
  if (wide && ns == 1 && g.mode == GEMM_Q8K) {
    // Whole rounds of 256 x 128 tiles plus at most half a round more (M = 2048: N = 6144 or
    // 14336): the columns of the last partial round go to the 128 x 128 kernel instead, one
    // round of tiles with half the work each.  Both kernels give the same bits.  (In f16 mode
    // the half round of wide tiles is as fast.)
    const int rows_w = (g.M + WBM - 1) / WBM, rows_n = (g.M + BM - 1) / BM, cols = (g.N + BN - 1) / BN;
    const int full = tiles / kRound, rem = tiles % kRound;
    if (full >= 1 && rem > 0 && rem <= kRound / 2 && (full * kRound) % rows_w == 0) {
      const int cols_w = full * kRound / rows_w, cols_n = cols - cols_w;
      if (cols_n >= 1 && cols_n * rows_n <= kRound) {
        GemmArgs a = g, b = g;
        a.N = cols_w * BN;
        const size_t c0 = (size_t)cols_w * BN;
        b.N = g.N - (int)c0;
        b.w = g.w + c0 * g.w_stride;
        b.y = g.y + c0;
        if (g.resid) b.resid = g.resid + c0;
        const dim3 ga((unsigned)cols_w, (unsigned)rows_w), gb((unsigned)cols_n, (unsigned)rows_n);
        hipExtLaunchKernelGGL((gemm_wide_kernel<GEMM_Q8K>), ga, dim3(GT), 0, s, ev0, nullptr, 0, a);
        hipExtLaunchKernelGGL((gemm_kernel<TPT_TYPE_Q4_K, GEMM_Q8K>), gb, dim3(GT), 0, s, nullptr, ev1, 0, b);
        TPT_HIP(hipGetLastError());
        return TPT_OK;
      }
    }
  }
  const dim3 grid((unsigned)((g.N + BN - 1) / BN), (unsigned)((g.M + tm - 1) / tm), (unsigned)ns);
  hipEvent_t e1 = ns > 1 ? nullptr : ev1;  // split-K: the stop event goes on the sum kernel
  if (wide) {
    if (g.mode == GEMM_Q8K) hipExtLaunchKernelGGL((gemm_wide_kernel<GEMM_Q8K>), grid, dim3(GT), 0, s, ev0, e1, 0, g);
    else hipExtLaunchKernelGGL((gemm_wide_kernel<GEMM_F16>), grid, dim3(GT), 0, s, ev0, e1, 0, g);
  } else if (g.wtype == TPT_TYPE_Q4_K) {
    if (g.mode == GEMM_Q8K) hipExtLaunchKernelGGL((gemm_kernel<TPT_TYPE_Q4_K, GEMM_Q8K>), grid, dim3(GT), 0, s, ev0, e1, 0, g);
    else hipExtLaunchKernelGGL((gemm_kernel<TPT_TYPE_Q4_K, GEMM_F16>), grid, dim3(GT), 0, s, ev0, e1, 0, g);
  } else if (g.wtype == TPT_TYPE_Q5_K) {
    if (g.mode == GEMM_Q8K) hipExtLaunchKernelGGL((gemm_kernel<TPT_TYPE_Q5_K, GEMM_Q8K>), grid, dim3(GT), 0, s, ev0, e1, 0, g);
    else hipExtLaunchKernelGGL((gemm_kernel<TPT_TYPE_Q5_K, GEMM_F16>), grid, dim3(GT), 0, s, ev0, e1, 0, g);
  } else if (g.wtype == TPT_TYPE_Q8_0) {
    hipExtLaunchKernelGGL((gemm_kernel<TPT_TYPE_Q8_0, GEMM_Q80>), grid, dim3(GT), 0, s, ev0, e1, 0, g);
  } else if (g.wtype == TPT_TYPE_Q4_0) {
    hipExtLaunchKernelGGL((gemm_kernel<TPT_TYPE_Q4_0, GEMM_Q80>), grid, dim3(GT), 0, s, ev0, e1, 0, g);
  } else if (g.wtype == TPT_TYPE_F16) {
    hipExtLaunchKernelGGL((gemm_kernel<TPT_TYPE_F16, GEMM_F16>), grid, dim3(GT), 0, s, ev0, e1, 0, g);
  } else {
    if (g.mode == GEMM_Q8K) hipExtLaunchKernelGGL((gemm_kernel<TPT_TYPE_Q6_K, GEMM_Q8K>), grid, dim3(GT), 0, s, ev0, e1, 0, g);
    else hipExtLaunchKernelGGL((gemm_kernel<TPT_TYPE_Q6_K, GEMM_F16>), grid, dim3(GT), 0, s, ev0, e1, 0, g);
  }
  TPT_HIP(hipGetLastError());
  if (ns > 1) {
    const size_t mn = (size_t)g.M * g.N;
    hipExtLaunchKernelGGL(gemm_split_reduce_kernel, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, s,
                          nullptr, ev1, 0, g, ns);
    TPT_HIP(hipGetLastError());
  }
  return TPT_OK;
}

// Split-K workspace bound for an M x N x K GEMM: the larger split count of the two tile shapes
// (the launch uses the count of the kernel it picks).
int gemm_splits(int M, int N, int K) {
  const int cols = (N + BN - 1) / BN, nkb = K / 256;
  return std::max(splits_for(cols * ((M + BM - 1) / BM), nkb), splits_for(cols * ((M + WBM - 1) / WBM), nkb));
}

}  // namespace tpt
