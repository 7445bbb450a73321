// KV-cache row access of the decode attention kernels: an fp16 or f32 row of head_dim elements is
// read as LPP lanes x 16 bytes (EPL elements per lane).
#pragma once
#include "kernels.h"

namespace tpt {
namespace attn {

// KV element traits: 16 bytes per lane per row => LPP lanes per position.
template <typename T> struct KvTraits;
template <> struct KvTraits<uint16_t> { static constexpr int LPP = 16; };
template <> struct KvTraits<float> { static constexpr int LPP = 32; };

template <int EPL>
__device__ __forceinline__ void load_row(const uint16_t* p, float* out) {
  if constexpr (EPL == 8) {
    const uint4 v = *(const uint4*)p;
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      out[2 * i] = h2f((uint16_t)(w[i] & 0xffff));
      out[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
    }
  } else if constexpr (EPL == 6) {
    const uint32_t* q = (const uint32_t*)p;
    const uint32_t w[3] = {q[0], q[1], q[2]};
#pragma unroll
    for (int i = 0; i < 3; i++) {
      out[2 * i] = h2f((uint16_t)(w[i] & 0xffff));
      out[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
    }
  } else {
    static_assert(EPL == 4, "fp16 rows: head_dim 64, 96 or 128");
    const uint2 v = *(const uint2*)p;
    const uint32_t w[2] = {v.x, v.y};
#pragma unroll
    for (int i = 0; i < 2; i++) {
      out[2 * i] = h2f((uint16_t)(w[i] & 0xffff));
      out[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
    }
  }
}

template <int EPL>
__device__ __forceinline__ void load_row(const float* p, float* out) {
  if constexpr (EPL == 4) {
    const float4 v = *(const float4*)p;
    out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
  } else if constexpr (EPL == 3) {
    out[0] = p[0]; out[1] = p[1]; out[2] = p[2];
  } else {
    static_assert(EPL == 2, "f32 rows: head_dim 64, 96 or 128");
    const float2 v = *(const float2*)p;
    out[0] = v.x; out[1] = v.y;
  }
}

}  // namespace attn
}  // namespace tpt
