"""tpt_attn_decode_noalloc (the allocation-free decode attention) through the C ABI against
tpt_attn_decode on the same inputs: the same kernels over the same split-K partition, so the
outputs are bit-identical.  Two calls in a row on one GPU, the second with a smaller input
(fewer positions, other head counts and head_dim, fewer chunks), then the size limit."""
import ctypes as C

import numpy as np
import pytest

import tpthip

pytestmark = pytest.mark.gpu


def _case(ctx, nq, nkv, hd, L, n_chunks, seed, kv_type):
    rng = np.random.default_rng(seed)
    dt = np.float16 if kv_type == tpthip.TYPE_F16 else np.float32
    q = ctx.to_device(rng.standard_normal(nq * hd).astype(np.float32))
    k = ctx.to_device(rng.standard_normal((nkv, L, hd)).astype(dt))
    v = ctx.to_device(rng.standard_normal((nkv, L, hd)).astype(dt))
    outs = []
    for fn in (tpthip.lib().tpt_attn_decode, tpthip.lib().tpt_attn_decode_noalloc):
        o = ctx.alloc(nq * hd * 4)
        tpthip.check(fn(ctx.h, q.ptr, k.ptr, v.ptr, kv_type, o.ptr, nq, nkv, hd, L, L, n_chunks))
        outs.append(o.download(np.float32, nq * hd))
        o.free()
    for b in (q, k, v):
        b.free()
    return outs


def test_noalloc_equals_allocating_entry_point(ctx):
    # first call: 8B heads over 4096 positions, the default partition
    ref, got = _case(ctx, 32, 8, 128, 4096, 0, seed=1, kv_type=tpthip.TYPE_F16)
    assert np.isfinite(ref).all() and np.array_equal(got, ref)
    # second call, smaller: MHA hd 96 over 300 positions in 5 chunks (the array keeps the first
    # call's records past what this call writes; none of them may leak into its output)
    ref, got = _case(ctx, 32, 32, 96, 300, 5, seed=2, kv_type=tpthip.TYPE_F16)
    assert np.isfinite(ref).all() and np.array_equal(got, ref)
    # and an f32 cache, 2 kv heads, one chunk
    ref, got = _case(ctx, 8, 2, 64, 17, 1, seed=3, kv_type=tpthip.TYPE_F32)
    assert np.array_equal(got, ref)


def test_noalloc_rejects_partitions_past_its_array(ctx):
    # 32 heads x 256 chunks x (128 + 2) floats = 4,259,840 bytes > 4 MiB
    q = ctx.alloc(32 * 128 * 4)
    kv = ctx.alloc(8 * 32768 * 128 * 2)
    o = ctx.alloc(32 * 128 * 4)
    try:
        rc = tpthip.lib().tpt_attn_decode_noalloc(ctx.h, q.ptr, kv.ptr, kv.ptr, tpthip.TYPE_F16,
                                                  o.ptr, 32, 8, 128, 32768, 32768, 256)
        assert rc == tpthip.ERR_UNSUPPORTED
        assert b"4 MiB" in tpthip.lib().tpt_last_error()
    finally:
        for b in (q, kv, o):
            b.free()
