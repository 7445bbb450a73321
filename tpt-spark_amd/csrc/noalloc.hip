// tpt_attn_decode_noalloc: the decode attention of tpt_attn_decode without any device
// allocation, for callers that cannot allocate (code under HIP graph capture, serving loops that
// must not call hipMalloc, harnesses that forbid it).
//
// The split-K partition's chunk records (per kv head, chunk and query head: the unnormalised
// output row, its running max and its sum) live in `scratch`, a file-scope device array of a fixed
// size that every GPU the library runs on holds until the process ends.  In host code the name
// `scratch` is only a host-side stand-in for the symbol: its device address on each GPU comes from
// hipGetSymbolAddress, looked up once per device (with that device current) on the first call
// there, and only that address is ever passed to a kernel.
//
// Every call on one GPU shares that GPU's array: two calls that overlap on the same GPU (other
// streams, other contexts, other threads) race on the records.  Nothing in the records has to
// start at zero (each chunk that holds positions writes its whole record before the merge reads
// it; chunks past the length write nothing and are not read), so no clearing is issued.
#include <mutex>

#include "kernels.h"

namespace tpt {
namespace {

// 4 MiB of chunk records: e.g. 32 query heads of head_dim 128 over up to 252 chunks, more than the
// default partition of any length the kernels support uses (at most 512 chunk-heads of kv heads).
constexpr size_t kScratchFloats = size_t(1) << 20;
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
float* g_ptr[kMaxDevices] = {};  // device address of `scratch` on each GPU, once looked up

// The device address of this device's `scratch` (the caller has made `device` current).
int scratch_on(int device, float** out) {
  if (device < 0 || device >= kMaxDevices) return fail(TPT_ERR_UNSUPPORTED, "attn_decode_noalloc: device index out of range");
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_ptr[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)", __FILE__, __LINE__);
    if (!p) return fail(TPT_ERR_HIP, "attn_decode_noalloc: no device address for the scratch array");
    g_ptr[device] = (float*)p;
  }
  *out = g_ptr[device];
  return TPT_OK;
}

}  // namespace
}  // namespace tpt

using namespace tpt;

extern "C" int tpt_attn_decode_noalloc(tpt_ctx* c, const float* q, const void* k_cache,
                                       const void* v_cache, int kv_type, float* o, int nq, int nkv,
                                       int hd, int L, int L_stride, int n_chunks) {
  int rc = ctx_enter(c);
  if (rc) return rc;
  if (!q || !k_cache || !v_cache || !o) return fail(TPT_ERR_INVALID, "attention: null pointer");
  if (nkv <= 0 || nq <= 0 || nq % nkv) return fail(TPT_ERR_INVALID, "attention: bad head counts");
  if (hd <= 0 || hd > 128 || nq > 4096) return fail(TPT_ERR_UNSUPPORTED, "attention: head_dim or head count out of range");
  if (L <= 0 || L > L_stride) return fail(TPT_ERR_INVALID, "attention: L must be in [1, L_stride]");
  if (L > attn_max_len()) return fail(TPT_ERR_UNSUPPORTED, "attention: cache longer than the split-K partition supports");
  if (n_chunks < 0 || n_chunks > 256) return fail(TPT_ERR_INVALID, "attention: chunk count must be in [1, 256] (0: default)");
  AttnArgs a;
  a.q = q;
  a.kc = k_cache;
  a.vc = v_cache;
  a.kv_type = kv_type;
  a.o = o;
  a.nq = nq;
  a.nkv = nkv;
  a.hd = hd;
  a.L_stride = L_stride;
  a.L_host = L;
  a.n_chunks = n_chunks > 0 ? n_chunks : attn_default_chunks(L, nkv);
  a.chunk_len = attn_chunk_len(L, a.n_chunks);
  const size_t need = (size_t)attn_part_floats(nq, nkv, hd, a.n_chunks);
  if (need > kScratchFloats)
    return fail(TPT_ERR_UNSUPPORTED, "attn_decode_noalloc: the chunk records need " + std::to_string(need * 4) +
                                         " bytes, more than the fixed 4 MiB scratch (fewer chunks, or tpt_attn_decode)");
  float* part = nullptr;
  if ((rc = scratch_on(c->device, &part))) return rc;
  a.part = part;
  return launch_attn_decode(a, c->stream);
}
