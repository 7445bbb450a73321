// Causal multi-query GQA attention (the batched prompt forward) on the matrix cores, fp16 KV cache.
//
// candle's batched prompt forward (candle_engine.rs:272-273 hands the whole prompt to one
// quantized_llama forward) computes for query t at position p0 + t, head h, kv head
// h / (Nq/Nkv):  s_j = (q . k_j) * f32(1/sqrt(hd)) for j <= p0 + t (the causal mask),
// o = softmax(s) . V.  The reference's wgpu engine runs attention.wgsl once per position instead
// (attention.wgsl:31-170, dispatch_attention wgpu_engine.rs:666-726); the values are the same.
//
// Flash form, one workgroup per (kv head, block of 32 query positions), one wave per query head
// of the group: the workgroup streams the kv head's key blocks 0 .. (last query's position) / 32
// through LDS once for all G heads (double-buffered: block b+1 is fetched while block b is
// computed), and every wave keeps its 32 queries' running max, sum and output in registers.
//
// Products on v_mfma_f32_32x32x16_f16 at f32 accuracy.  The cache is fp16, so K and V are exact
// MFMA operands; the f32 operands q and p are split into fp16 pairs hi + lo (hi = q rounded
// toward zero, lo = q - hi rounded toward zero: |q - hi - lo| < 2^-20 |q|), and every product is
// two MFMAs (hi, lo) accumulated in f32.  Per 32-key block and wave:
//   S^T[key][query] = K . (q * scale * log2 e)^T   (A = K rows from LDS, B = q pairs in registers)
//   p = exp2(S^T - m), m the running max of the query's scores up to a slack of 8 (one lane per
//       query: each lane holds 16 of a query's 32 scores, the other half-wave the other 16)
//   O^T[d][query] = O^T * exp2(m_old - m) + V^T . P^T   (A = V^T from LDS, B = the p pairs)
// The score tile's register layout is used directly as the B operand of the second product: the
// 16-key reduction slots of a lane are its own 8 scores of the step, and the V^T rows are read in
// that key order (keys 16j + 4h .. +3 and 16j + 8 + 4h .. +3 for half-wave h), so no score moves
// between lanes.  V is transposed into LDS while it is staged ([d][key], two keys per 32-bit
// write).  Scores are formed in the log2 domain (q pre-scaled by scale * log2 e), the same
// softmax as exp(s - max) up to f32 rounding.  Query magnitudes must stay below the fp16 range
// after that scaling (|q| < 4.5e5 at head_dim 128).
#include "attn_dev.h"

namespace tpt {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int QB = 32;  // query positions per workgroup (the MFMA N of both products)
constexpr int KB = 32;  // keys per block (the MFMA M of the score tile)

// (x0, x1) -> packed fp16 hi and lo words with hi + lo = x to 2^-20 relative (the remainders
// x - hi are exact: mixed-precision fused multiply-adds on the fp16 hi)
__device__ __forceinline__ void split_pair(float x0, float x1, uint32_t& hi, uint32_t& lo) {
  const auto h = __builtin_amdgcn_cvt_pkrtz(x0, x1);
  const float r0 = __builtin_fmaf((float)h[0], -1.f, x0), r1 = __builtin_fmaf((float)h[1], -1.f, x1);
  hi = __builtin_bit_cast(uint32_t, h);
  lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(r0, r1));
}

// Slack of the running max (log2 units): the max moves only when a block's scores pass it by
// more than this, so the output rescale is rare; p = 2^(s - m) then stays below 2^8.
constexpr float MAX_SLACK = 8.f;

template <int HD, int G>
__global__ void __launch_bounds__(64 * G, 2) attn_causal_kernel(const AttnArgs a, const float qscale) {
  constexpr int NT = 64 * G;
  constexpr int KS = HD / 16;                // 16-dim steps of the score product
  constexpr int OT = HD / 32;                // 32-dim tiles of the output
  constexpr int KRS = HD + 8;                // K tile row stride (halves)
  constexpr int VRS = KB + 4;                // V^T tile row stride (halves)
  constexpr int KU = KB * HD / 8;            // 16-byte units of a K block
  constexpr int VU = (KB / 2) * (HD / 8);    // (key pair, 8 dims) units of a V block
  constexpr int KPT = (KU + NT - 1) / NT, VPT = (VU + NT - 1) / NT;
  __shared__ __attribute__((aligned(16))) uint16_t sK[2][KB * KRS];
  __shared__ __attribute__((aligned(16))) uint16_t sV[2][HD * VRS];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int n = lane & 31, hh = lane >> 5;
  const int kvh = blockIdx.y;
  const int t0 = (gridDim.x - 1 - blockIdx.x) * QB;  // the longest key ranges start first
  const int tlast = min(t0 + QB, a.nqb) - 1;
  const int p0 = a.L_host - 1;                       // query t sits at position p0 + t
  const int kend = p0 + tlast + 1;                   // keys [0, kend) are read
  const int nkb = (kend + KB - 1) / KB;
  const int head = kvh * G + w;
  const int t = t0 + n;

  const uint16_t* Kg = (const uint16_t*)a.kc + (size_t)kvh * a.L_stride * HD;
  const uint16_t* Vg = (const uint16_t*)a.vc + (size_t)kvh * a.L_stride * HD;

  // ---- staging: global -> registers (rows past kend read as zero) -> LDS
  u32x4 kr[KPT], vr[VPT][2];
  auto gload = [&](int kb) {
#pragma unroll
    for (int i = 0; i < KPT; i++) {
      const int u = tid + i * NT;
      if (KU % NT == 0 || u < KU) {
        const int key = kb * KB + u / (HD / 8), c = u % (HD / 8);
        kr[i] = key < kend ? *(const u32x4*)(Kg + (size_t)key * HD + 8 * c) : u32x4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int i = 0; i < VPT; i++) {
      const int u = tid + i * NT;
      if (VU % NT == 0 || u < VU) {
        const int key = kb * KB + 2 * (u % (KB / 2)), dg = u / (KB / 2);
        const uint16_t* src = Vg + (size_t)key * HD + 8 * dg;
        vr[i][0] = key < kend ? *(const u32x4*)src : u32x4{0, 0, 0, 0};
        vr[i][1] = key + 1 < kend ? *(const u32x4*)(src + HD) : u32x4{0, 0, 0, 0};
      }
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < KPT; i++) {
      const int u = tid + i * NT;
      if (KU % NT == 0 || u < KU)
        *(u32x4*)&sK[buf][(u / (HD / 8)) * KRS + 8 * (u % (HD / 8))] = kr[i];
    }
#pragma unroll
    for (int i = 0; i < VPT; i++) {
      const int u = tid + i * NT;
      if (VU % NT == 0 || u < VU) {
        const int kp = u % (KB / 2), dg = u / (KB / 2);
        uint16_t* dst = &sV[buf][(8 * dg) * VRS + 2 * kp];
#pragma unroll
        for (int j = 0; j < 4; j++) {  // dims 8dg + 2j, 8dg + 2j + 1 of keys 2kp, 2kp + 1
          const uint32_t x0 = vr[i][0][j], x1 = vr[i][1][j];
          *(uint32_t*)(dst + (2 * j) * VRS) = (x0 & 0xffffu) | (x1 << 16);
          *(uint32_t*)(dst + (2 * j + 1) * VRS) = (x0 >> 16) | (x1 & 0xffff0000u);
        }
      }
    }
  };

  gload(0);

  // ---- the wave's 32 query rows (rows past the batch repeat its last row; they are not stored)
  half8 qh[KS], ql[KS];
  {
    const float* qrow = a.q + (size_t)min(t, a.nqb - 1) * a.ldq + (size_t)head * HD + 8 * hh;
#pragma unroll
    for (int s = 0; s < KS; s++) {
      const float4 x0 = *(const float4*)(qrow + 16 * s), x1 = *(const float4*)(qrow + 16 * s + 4);
      const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      u32x4 hi, lo;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        uint32_t h, l;
        split_pair(x[2 * i] * qscale, x[2 * i + 1] * qscale, h, l);
        hi[i] = h;
        lo[i] = l;
      }
      qh[s] = __builtin_bit_cast(half8, hi);
      ql[s] = __builtin_bit_cast(half8, lo);
    }
  }

  sstore(0);
  __syncthreads();

  floatx16 o[OT];
#pragma unroll
  for (int i = 0; i < OT; i++) o[i] = floatx16{};
  float m = -INFINITY, l = 0.f;  // running max (log2 domain) and this half-wave's running sum

  for (int kb = 0; kb < nkb; kb++) {
    const int b = kb & 1;
    if (kb + 1 < nkb) gload(kb + 1);

    // S^T = K . q^T
    floatx16 sacc = floatx16{};
#pragma unroll
    for (int s = 0; s < KS; s++) {
      const half8 ka = *(const half8*)&sK[b][n * KRS + 16 * s + 8 * hh];
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qh[s], sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, ql[s], sacc, 0, 0, 0);
    }
    // causal mask: key j is visible to query t iff j <= p0 + t (only blocks that reach past the
    // first query's position hold masked keys)
    const int kbase = kb * KB;
    if (kbase + KB - 1 > p0 + t0) {
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int key = kbase + (e / 4) * 8 + hh * 4 + (e % 4);
        if (key > p0 + t) sacc[e] = -INFINITY;
      }
    }
    // online softmax: lane (n, hh) holds 16 of query n's 32 scores
    float mx = sacc[0];
#pragma unroll
    for (int e = 1; e < 16; e++) mx = fmaxf(mx, sacc[e]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // finite after the first block: key 0 is visible to every query
    const float mnew = mx > m + MAX_SLACK ? mx : m;
    // 2^(m - mnew) and 2^(s - mnew) on v_exp_f32 directly: the arguments are <= 8, and results
    // below 2^-126 (flushed or not) are negligible against the running sum
    const float alpha = __builtin_amdgcn_exp2f(m - mnew);
    m = mnew;
    float ps = 0.f;
#pragma unroll
    for (int e = 0; e < 16; e++) {
      sacc[e] = __builtin_amdgcn_exp2f(sacc[e] - mnew);
      ps += sacc[e];
    }
    l = l * alpha + ps;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
      for (int i = 0; i < OT; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) o[i][e] *= alpha;
    }
    // O^T += V^T . P^T over the two 16-key steps
#pragma unroll
    for (int j = 0; j < 2; j++) {
      u32x4 hi, lo;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        uint32_t h, lw;
        split_pair(sacc[8 * j + 2 * i], sacc[8 * j + 2 * i + 1], h, lw);
        hi[i] = h;
        lo[i] = lw;
      }
      const half8 ph = __builtin_bit_cast(half8, hi), pl = __builtin_bit_cast(half8, lo);
#pragma unroll
      for (int i = 0; i < OT; i++) {
        const uint16_t* vp = &sV[b][(32 * i + n) * VRS + 16 * j + 4 * hh];
        const u32x2 v0 = *(const u32x2*)vp, v1 = *(const u32x2*)(vp + 8);
        const half8 va = __builtin_bit_cast(half8, u32x4{v0[0], v0[1], v1[0], v1[1]});
        o[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, ph, o[i], 0, 0, 0);
        o[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pl, o[i], 0, 0, 0);
      }
    }
    if (kb + 1 < nkb) sstore(b ^ 1);
    __syncthreads();
  }

  // o = O^T / l; lane (n, hh) holds dims 32i + 8g + 4hh .. +3 of query n
  const float lt = l + __shfl_xor(l, 32);
  if (t <= tlast) {
    float* orow = a.o + (size_t)t * a.ldo + (size_t)head * HD + 4 * hh;
#pragma unroll
    for (int i = 0; i < OT; i++)
#pragma unroll
      for (int g = 0; g < 4; g++)
        *(float4*)(orow + 32 * i + 8 * g) =
            float4{o[i][4 * g] / lt, o[i][4 * g + 1] / lt, o[i][4 * g + 2] / lt, o[i][4 * g + 3] / lt};
  }
}

template <int HD>
int launch_hd(const AttnArgs& a, float qscale, hipStream_t s) {
  const dim3 grid((unsigned)((a.nqb + QB - 1) / QB), (unsigned)a.nkv);
  switch (a.nq / a.nkv) {
    case 1: hipLaunchKernelGGL((attn_causal_kernel<HD, 1>), grid, dim3(64), 0, s, a, qscale); break;
    case 2: hipLaunchKernelGGL((attn_causal_kernel<HD, 2>), grid, dim3(128), 0, s, a, qscale); break;
    case 4: hipLaunchKernelGGL((attn_causal_kernel<HD, 4>), grid, dim3(256), 0, s, a, qscale); break;
    case 8: hipLaunchKernelGGL((attn_causal_kernel<HD, 8>), grid, dim3(512), 0, s, a, qscale); break;
    default: return fail(TPT_ERR_UNSUPPORTED, "causal attention: Nq/Nkv must be 1, 2, 4 or 8");
  }
  TPT_HIP(hipGetLastError());
  return TPT_OK;
}

}  // namespace

bool attn_causal_mfma_supported(const AttnArgs& a) {
  const int g = a.nkv > 0 ? a.nq / a.nkv : 0;
  return a.kv_type == TPT_TYPE_F16 && (a.hd == 64 || a.hd == 128) && (g == 1 || g == 2 || g == 4 || g == 8) &&
         a.nq % a.nkv == 0;
}

int launch_attn_causal_mfma(const AttnArgs& a, hipStream_t s) {
  if (a.nq <= 0 || a.nkv <= 0 || a.nq % a.nkv) return fail(TPT_ERR_INVALID, "causal attention: bad head counts");
  if (!attn_causal_mfma_supported(a))
    return fail(TPT_ERR_UNSUPPORTED, "causal attention on the matrix cores: fp16 cache, head_dim 64 or 128, "
                                     "Nq/Nkv 1, 2, 4 or 8");
  if (a.state || a.nqb < 1 || a.L_host < 1 || a.L_host + a.nqb - 1 > a.L_stride)
    return fail(TPT_ERR_INVALID, "causal attention: queries past the cache");
  if (a.ldq < a.nq * a.hd || a.ldo < a.nq * a.hd || a.ldq % 4 || a.ldo % 4 || ((uintptr_t)a.q & 15) ||
      ((uintptr_t)a.o & 15) || ((uintptr_t)a.kc & 15) || ((uintptr_t)a.vc & 15))
    return fail(TPT_ERR_INVALID, "causal attention: rows must be 16-byte aligned");
  const float qscale = (float)(1.4426950408889634 / __builtin_sqrt((double)a.hd));
  return a.hd == 64 ? launch_hd<64>(a, qscale, s) : launch_hd<128>(a, qscale, s);
}

}  // namespace tpt
