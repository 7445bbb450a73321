"""The persistent decode step (embedding + every layer in one launch, grid barriers between the
phases) against the per-op launches and against the oracle.

Both device paths run the same arithmetic in the same order (the GEMV rows share their lane
groups and reductions, and the per-op attention kernels sum position groups and chunk records
in the persistent kernel's order), so their logits and greedy tokens are bit-identical; the
per-op path's oracle parity then carries over, and the persistent path is also checked against
the oracle directly.
Shapes: the tiny test model (hd 64, GQA 2), and a 2-layer model of the Llama-3 8B width (hidden
4096, 32/8 heads, hd 128, FFN 14336) that runs the 8B instantiation of the kernel; its long
prompts exercise attention partitions of more than one item per workgroup."""
import os

import numpy as np
import pytest

import oracle
import tpthip
from tpthip import synth

pytestmark = pytest.mark.gpu

PROMPT = [11, 500, 7, 1023, 42, 99, 3]
KV_TYPE = {"f16": tpthip.TYPE_F16, "f32": tpthip.TYPE_F32}


@pytest.fixture(scope="module", params=["f16", "f32"])
def kv(request):
    return request.param


def decode_both(m, prompt, n, logits_at):
    """Greedy tokens (prefill + n-1 graph-replayed steps) and the logits of step logits_at
    through the single-step path, on the model's current decode path."""
    first = m.prefill(prompt, 0)
    toks = [first] + m.decode_greedy(first, len(prompt), n - 1)
    m.prefill(prompt, 0)
    for i in range(logits_at):
        m.decode_step(toks[i], len(prompt) + i)
    _, lg = m.decode_step(toks[logits_at], len(prompt) + logits_at, logits=True)
    return toks, lg


def test_decode_path_selection(ctx, tiny_gguf):
    m = tpthip.Model(ctx, tiny_gguf, max_ctx=256)
    try:
        assert m.decode_path == m.DECODE_KERNELS
        m.decode_path = m.DECODE_PERSISTENT
        assert m.decode_path == m.DECODE_PERSISTENT
        with pytest.raises(tpthip.TptError):
            m.decode_path = 7
    finally:
        m.close()


def test_tiny_paths_agree(ctx, tiny_gguf, kv):
    """60 greedy tokens (crossing the 64- and 128-position attention buckets) on both paths."""
    m = tpthip.Model(ctx, tiny_gguf, max_ctx=256, kv_type=KV_TYPE[kv])
    try:
        m.decode_path = m.DECODE_KERNELS
        t_k, lg_k = decode_both(m, PROMPT, 60, 57)
        m.decode_path = m.DECODE_PERSISTENT
        t_p, lg_p = decode_both(m, PROMPT, 60, 57)
    finally:
        m.close()
    assert t_p == t_k
    assert np.array_equal(lg_p, lg_k)


def test_tiny_persistent_matches_oracle(ctx, tiny_gguf, kv):
    """The candle bar on the persistent path: identical first 32 greedy tokens (all 40 with the
    f32 cache, candle's), logits of step 32 within 1e-2 max-abs (f32 cache)."""
    n = 40
    om = oracle.Model(tiny_gguf)
    try:
        want, lref = om.greedy(PROMPT, n, kv_f16=(kv == "f16"), return_logits=(1, 32))
    finally:
        om.close()
    m = tpthip.Model(ctx, tiny_gguf, max_ctx=256, kv_type=KV_TYPE[kv])
    try:
        m.decode_path = m.DECODE_PERSISTENT
        got, lg = decode_both(m, PROMPT, n, 31)
    finally:
        m.close()
    assert got[:32] == want[:32]
    if kv == "f32":
        assert got == want
        assert np.abs(lg - lref[32]).max() < 1e-2


WIDE = dict(n_layers=2, embed=4096, n_heads=32, n_kv_heads=8, ffn=14336, vocab=4096,
            context_length=4096, rope_base=500000.0, rms_eps=1e-5)


@pytest.fixture(scope="module")
def wide_gguf(tmp_path_factory):
    """Two layers at the Llama-3 8B width (the 8B instantiation of the persistent kernel)."""
    path = str(tmp_path_factory.mktemp("wide") / "llama-8b-width-2l.gguf")
    synth.write_llama(path, WIDE, seed=99, nthreads=min(os.cpu_count() or 1, 16))
    yield path
    os.remove(path)


@pytest.mark.parametrize("plen", [5, 600, 3000])
def test_wide_paths_agree(ctx, wide_gguf, kv, plen):
    """Prompt lengths in the 64-position bucket, the 1024 bucket (16 chunks per kv head) and
    the 3072 bucket (48 chunks per kv head: 384 attention items, two per workgroup)."""
    prompt = [int(t) for t in np.random.default_rng(plen).integers(0, WIDE["vocab"], plen)]
    m = tpthip.Model(ctx, wide_gguf, max_ctx=4096, kv_type=KV_TYPE[kv])
    try:
        m.decode_path = m.DECODE_KERNELS
        t_k, lg_k = decode_both(m, prompt, 12, 9)
        m.decode_path = m.DECODE_PERSISTENT
        t_p, lg_p = decode_both(m, prompt, 12, 9)
    finally:
        m.close()
    print(plen, kv, "max-abs logits persistent vs per-op", float(np.abs(lg_p - lg_k).max()))
    assert t_p == t_k
    assert np.array_equal(lg_p, lg_k)


def _oracle_forced(path, prompt, toks, fma=True, block_order=False):
    """Oracle logits after feeding each of toks (teacher-forced, f32 cache)."""
    om = oracle.Model(path)
    try:
        om.set_attn_fma(fma)
        oracle.set_dot_block_order(block_order)
        om.reset(len(prompt) + len(toks) + 1, kv_f16=False)
        om.forward(prompt, 0)
        return [om.forward([t], len(prompt) + i) for i, t in enumerate(toks)]
    finally:
        oracle.set_dot_block_order(False)
        om.close()


def test_wide_persistent_matches_oracle(ctx, wide_gguf):
    """8B-width layers on the persistent path against the oracle (f32 cache, candle's), both
    fed the oracle's greedy tokens.  This random-init model amplifies rounding (every matmul
    requantizes its input to Q8_K), so as at the 1B shape the bar is the oracle's own spread S:
    the largest max-abs distance, over the 8 steps, between the oracle and the oracle under
    candle's other two plausible summation orders (attention without FMA; block-reduced k-quant
    dots); the device logits after each step stay within S."""
    prompt = [int(t) for t in np.random.default_rng(5).integers(0, WIDE["vocab"], 40)]
    om = oracle.Model(wide_gguf)
    try:
        toks, _ = om.greedy(prompt, 8, kv_f16=False)
    finally:
        om.close()
    ref = _oracle_forced(wide_gguf, prompt, toks)
    alt = [_oracle_forced(wide_gguf, prompt, toks, fma=False),
           _oracle_forced(wide_gguf, prompt, toks, block_order=True)]
    S = max(float(np.abs(a[i] - ref[i]).max()) for a in alt for i in range(len(toks)))
    m = tpthip.Model(ctx, wide_gguf, max_ctx=256, kv_type=tpthip.TYPE_F32)
    try:
        m.decode_path = m.DECODE_PERSISTENT
        m.prefill(prompt, 0)
        got = [m.decode_step(t, len(prompt) + i, logits=True)[1] for i, t in enumerate(toks)]
    finally:
        m.close()
    for i in range(len(toks)):
        dev = float(np.abs(got[i] - ref[i]).max())
        print(f"step {i}: gpu-oracle {dev:.4f}, oracle spread S {S:.4f}")
        assert dev <= S, (i, dev, S)


def test_kv_cache_rows_agree(ctx, tiny_gguf):
    """The K/V rows the persistent kernel appends are bit-identical to the per-op path's."""
    caches = {}
    for path in ("kernels", "persistent"):
        m = tpthip.Model(ctx, tiny_gguf, max_ctx=128, kv_type=tpthip.TYPE_F32)
        try:
            m.decode_path = m.DECODE_KERNELS if path == "kernels" else m.DECODE_PERSISTENT
            first = m.prefill(PROMPT, 0)
            m.decode_greedy(first, len(PROMPT), 20)
            caches[path] = [m.kv(l) for l in range(2)]
        finally:
            m.close()
    n = len(PROMPT) + 20
    for l in range(2):
        for a, b in zip(caches["kernels"][l], caches["persistent"][l]):
            assert np.array_equal(a[:, :n], b[:, :n])
