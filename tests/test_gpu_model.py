"""Model- and engine-level parity on the GPU: greedy decode of seeded random-init Llama GGUFs
against the oracle's quantized_llama restatement, and the LlmEngine semantics of the reference
engines (stop rules, cancellation, prefix reuse, error paths)."""
import os
import shutil

import numpy as np
import pytest

import oracle
import tpthip
from tpthip import synth

pytestmark = pytest.mark.gpu

PROMPT = [11, 500, 7, 1023, 42, 99, 3]


@pytest.fixture(scope="module", params=["f16", "f32"])
def kv(request):
    """KV cache element type: fp16 (the default engine layout) and f32 (candle's cache)."""
    return request.param


KV_TYPE = {"f16": tpthip.TYPE_F16, "f32": tpthip.TYPE_F32}

# fp16 K/V rounding can flip under f32 summation-order differences, and a flipped K/V entry
# feeds every later position: over a 150-token prompt the oracle itself moves by 0.011 (block-
# reduced dot products) to 0.013 (fused-multiply-add attention) in max-abs logits with the fp16
# cache, and by 2e-7 with the f32 cache.  Logit bars in the fp16 mode are set to that spread.
FP16_LOGIT_TOL = 4e-2


@pytest.fixture(scope="module")
def tiny_model(ctx, tiny_gguf, kv):
    m = tpthip.Model(ctx, tiny_gguf, max_ctx=256, kv_type=KV_TYPE[kv])
    yield m
    m.close()


@pytest.fixture(scope="module")
def tiny_oracle(tiny_gguf):
    return oracle.Model(tiny_gguf)


def test_describe(tiny_model, kv):
    d = tiny_model.desc
    assert (d["n_layers"], d["embed"], d["n_heads"], d["n_kv_heads"], d["head_dim"], d["ffn"],
            d["vocab"]) == (2, 256, 4, 2, 64, 512, 1024)
    assert d["type_q"] == tpthip.TYPE_Q4_K and d["type_out"] == tpthip.TYPE_Q6_K
    assert d["max_ctx"] == 256 and d["kv_type"] == KV_TYPE[kv]


def test_prefill_logits_match_oracle(tiny_model, tiny_oracle, kv):
    """Same cache values as the oracle's mode: only f32 summation order differs (< 1e-3).
    The f32 cache is candle's: its logits meet the candle bar (max-abs < 1e-2)."""
    nxt, lg = tiny_model.prefill(PROMPT, 0, logits=True)
    tiny_oracle.reset(64, kv_f16=(kv == "f16"))
    ref = tiny_oracle.forward(PROMPT, 0)
    assert np.abs(lg - ref).max() < 1e-3
    assert nxt == oracle.argmax(lg) == oracle.argmax(ref)
    if kv == "f32":
        tiny_oracle.reset(64, kv_f16=False)
        assert np.abs(lg - tiny_oracle.forward(PROMPT, 0)).max() < 1e-2


def test_greedy_tokens_match_oracle(tiny_model, tiny_oracle, kv):
    """Greedy tokens identical to the oracle in the same cache mode: the first 32 (the bar; for
    the f32 cache that is candle's greedy sequence) and, with the f32 cache, all 40.  An fp16
    cache entry can round the other way under an f32 summation-order difference, and such a flip
    can move a later token, so past the bar the fp16 mode is not held to identity."""
    n = 40
    toks_ref, logits_ref = tiny_oracle.greedy(PROMPT, n, kv_f16=(kv == "f16"), return_logits=(1, 32))
    first = tiny_model.prefill(PROMPT, 0)
    got = [first] + tiny_model.decode_greedy(first, len(PROMPT), n - 1)
    assert got[:32] == toks_ref[:32]
    if kv == "f32":
        assert got == toks_ref
    # logits of a later step through the single-step path
    pos = len(PROMPT)
    tiny_model.prefill(PROMPT, 0)
    for i in range(31):
        tiny_model.decode_step(got[i], pos + i)
    _, lg = tiny_model.decode_step(got[31], pos + 31, logits=True)
    assert np.abs(lg - logits_ref[32]).max() < (1e-2 if kv == "f32" else FP16_LOGIT_TOL)


def test_graph_decode_equals_stepwise(tiny_model):
    first = tiny_model.prefill(PROMPT, 0)
    fast = tiny_model.decode_greedy(first, len(PROMPT), 24)
    tiny_model.prefill(PROMPT, 0)
    slow, tok = [], first
    for i in range(24):
        tok = tiny_model.decode_step(tok, len(PROMPT) + i)
        slow.append(tok)
    assert fast == slow


def test_decode_greedy_stop_token(tiny_model):
    first = tiny_model.prefill(PROMPT, 0)
    full = tiny_model.decode_greedy(first, len(PROMPT), 30)
    stop = full[10]
    cut = tiny_model.decode_greedy(first, len(PROMPT), 30, stop_token=stop)
    assert cut == full[:full.index(stop) + 1]


def test_prefix_prefill_equals_full(tiny_model):
    full = tiny_model.prefill(PROMPT, 0)
    tiny_model.prefill(PROMPT[:4], 0)
    part = tiny_model.prefill(PROMPT[4:], 4)
    assert full == part


def test_kv_cache_matches_oracle(tiny_model, tiny_oracle, kv):
    """The K/V rows the prompt and 10 decode steps append, read back with tpt_model_kv_read,
    against the oracle's cache fed the same tokens: layout [kv head][position][head_dim], K after
    RoPE, V as projected.  f32 cache: within f32 rounding of the GEMV's summation order.  fp16
    cache: layer 0 (the same embedding rows on both sides) the oracle's fp16-rounded values, at
    most one fp16 ulp apart where an f32 ordering difference moves a value across a rounding
    boundary; layer 1 reads layer 0's output through an fp16 cache and a Q8_K requantization,
    where such a one-ulp flip grows to a few ulp: relative L2 below 2e-3 (fp16's own rounding is
    4.9e-4 relative)."""
    n = len(PROMPT)
    first = tiny_model.prefill(PROMPT, 0)
    toks = [first] + tiny_model.decode_greedy(first, n, 10)[:9]  # fed at positions n .. n+9
    tiny_oracle.reset(64, kv_f16=(kv == "f16"))
    tiny_oracle.forward(PROMPT, 0)
    for i, t in enumerate(toks):
        tiny_oracle.forward([t], n + i)
    L = n + len(toks)
    for layer in range(2):
        for g, o in zip(tiny_model.kv(layer), tiny_oracle.kv(layer)):
            g, o = g[:, :L], o[:, :L]
            if kv == "f32":
                assert np.linalg.norm(g - o) / np.linalg.norm(o) < 1e-5, layer
            elif layer == 0:
                ulp = np.spacing(np.abs(o).astype(np.float16)).astype(np.float32)
                d = np.abs(g - o)
                assert np.all(d <= ulp) and np.mean(d > 0) < 0.01, (layer, float((d / ulp).max()))
            else:
                assert np.linalg.norm(g - o) / np.linalg.norm(o) < 2e-3, layer


def test_context_bounds(tiny_model):
    with pytest.raises(tpthip.TptError) as e:
        tiny_model.prefill([1, 2], 255)
    assert e.value.code == tpthip.ERR_INVALID
    with pytest.raises(tpthip.TptError):
        tiny_model.prefill([5000], 0)  # id outside the vocabulary


# ---------------------------------------------------------------- engine (LlmEngine mirror)

@pytest.fixture(scope="module")
def engine(tiny_gguf):
    """The engine in candle's cache mode (f32 KV), so its greedy output is candle's."""
    e = tpthip.HipEngine(0, kv_type=tpthip.TYPE_F32)
    info = e.load(tiny_gguf)
    assert info.backend.startswith("hip-gfx")
    yield e
    e.close()


def run(engine, params):
    events = []
    engine.infer(params, events.append)
    assert events[-1].done and all(not ev.done for ev in events[:-1])
    return [ev.token_id for ev in events[:-1]]


def test_engine_lifecycle(tiny_gguf):
    e = tpthip.HipEngine(0)
    assert not e.is_loaded() and e.model_info() is None
    seen = []
    info = e.load(tiny_gguf, on_progress=lambda d, t: seen.append((d, t)))
    assert e.is_loaded() and info.name == "tiny" and info.size_bytes == os.path.getsize(tiny_gguf)
    assert seen[-1][0] == seen[-1][1] and len(seen) == seen[-1][1]
    assert e.model_info() == info
    e.unload()
    assert not e.is_loaded()
    with pytest.raises(tpthip.TptError) as ex:
        e.infer(tpthip.greedy_params(PROMPT, 4), lambda ev: None)
    assert ex.value.code == tpthip.ERR_STATE
    e.close()


def test_engine_greedy_matches_oracle(engine, tiny_oracle):
    engine.reset_cache()
    toks = run(engine, tpthip.greedy_params(PROMPT, 20))
    ref, _ = tiny_oracle.greedy(PROMPT, 20)
    assert toks == ref
    st = engine.last_stats
    assert st.generated == 20 and st.prompt_tokens == len(PROMPT)


def test_engine_eos_and_max_tokens(engine, tiny_oracle):
    ref, _ = tiny_oracle.greedy(PROMPT, 20)
    engine.reset_cache()
    eos = ref[6]
    toks = run(engine, tpthip.greedy_params(PROMPT, 20, eos_token_id=eos))
    assert toks == ref[:ref.index(eos)]
    engine.reset_cache()
    assert run(engine, tpthip.greedy_params(PROMPT, 3)) == ref[:3]
    engine.reset_cache()
    assert run(engine, tpthip.greedy_params(PROMPT, 0)) == []


def test_engine_cancellation(engine, tiny_oracle):
    ref, _ = tiny_oracle.greedy(PROMPT, 20)
    engine.reset_cache()
    events = []

    class Stop(Exception):
        pass

    def cb(ev):
        events.append(ev)
        if not ev.done and len(events) == 4:
            raise Stop()

    with pytest.raises(Stop):
        engine.infer(tpthip.greedy_params(PROMPT, 20), cb)
    assert [ev.token_id for ev in events[:4]] == ref[:4]
    assert events[-1].done and len(events) == 5  # done:true still delivered
    # the cancelled token was not fed: the cache holds the prompt + the first 3 tokens
    assert engine.cached_prefix_len(PROMPT + ref[:3] + [9999]) == len(PROMPT) + 3


def test_engine_prefix_reuse(engine, tiny_oracle):
    engine.reset_cache()
    first = run(engine, tpthip.greedy_params(PROMPT, 8))
    turn2 = PROMPT + first + [77, 78]
    toks = run(engine, tpthip.greedy_params(turn2, 8))
    assert engine.last_stats.cached_prefix == len(PROMPT) + len(first)
    ref, _ = tiny_oracle.greedy(turn2, 8)
    assert toks == ref
    # identical prompt again: everything cached, the last position is recomputed
    toks2 = run(engine, tpthip.greedy_params(turn2, 8))
    assert toks2 == ref and engine.last_stats.cached_prefix == len(turn2) - 1


def test_engine_reset_cache(engine, tiny_oracle):
    """KvCache::reset through the engine (the reference's test_reset_clears_tokens,
    wgpu_kvcache.rs:126-132): after tpt_engine_reset_cache nothing of the previous turn is
    reusable, the next infer recomputes the whole prompt, and its output is still candle's."""
    engine.reset_cache()
    first = run(engine, tpthip.greedy_params(PROMPT, 6))
    assert engine.cached_prefix_len(PROMPT + first) == len(PROMPT) + 6  # every emitted token was fed
    engine.reset_cache()
    assert engine.cached_prefix_len(PROMPT + first) == 0
    assert engine.cached_prefix_len(PROMPT) == 0
    again = run(engine, tpthip.greedy_params(PROMPT, 6))
    assert engine.last_stats.cached_prefix == 0 and engine.last_stats.prompt_tokens == len(PROMPT)
    ref, _ = tiny_oracle.greedy(PROMPT, 6)
    assert again == first == ref


def test_engine_repeat_penalty_path(engine, tiny_oracle):
    """Non-greedy settings take the host-sampling path; with temperature 0 and a penalty the
    result is deterministic and follows apply_repeat_penalty (candle_engine.rs:87-101)."""
    engine.reset_cache()
    p = tpthip.InferenceParams(prompt=PROMPT, max_tokens=10, temperature=0.0, top_p=1.0,
                               repeat_penalty=1.3)
    toks = run(engine, p)
    tiny_oracle.reset(64)
    seen = list(PROMPT)
    lg = oracle.repeat_penalty(tiny_oracle.forward(PROMPT, 0), seen, 1.3)
    ref, pos = [], len(PROMPT)
    nxt = oracle.argmax(lg)
    for _ in range(10):
        ref.append(nxt)
        seen.append(nxt)
        lg = oracle.repeat_penalty(tiny_oracle.forward([nxt], pos), seen, 1.3)
        nxt = oracle.argmax(lg)
        pos += 1
    assert toks == ref


def test_engine_prompt_truncation(engine):
    engine.reset_cache()
    long_prompt = [int(t) for t in np.random.default_rng(0).integers(0, 1024, 600)]
    toks = run(engine, tpthip.greedy_params(long_prompt, 10))
    # the tiny model's context_length is 512: the prompt keeps its last 512 - 10 ids
    assert engine.last_stats.prompt_tokens == 512 - 10 and len(toks) == 10


def test_load_errors(ctx, tiny_gguf, tmp_path):
    with pytest.raises(tpthip.TptError) as e:
        tpthip.Model(ctx, str(tmp_path / "missing.gguf"))
    assert e.value.code == tpthip.ERR_IO
    trunc = str(tmp_path / "trunc.gguf")
    data = open(tiny_gguf, "rb").read()
    open(trunc, "wb").write(data[:len(data) - 1000])
    with pytest.raises(tpthip.TptError) as e:
        tpthip.Model(ctx, trunc)
    assert e.value.code == tpthip.ERR_FORMAT and "past end of file" in str(e.value)
    arch = str(tmp_path / "arch.gguf")
    open(arch, "wb").write(data.replace(b"\x05\x00\x00\x00\x00\x00\x00\x00llama", b"\x05\x00\x00\x00\x00\x00\x00\x00gemma", 1))
    with pytest.raises(tpthip.TptError) as e:
        tpthip.Model(ctx, arch)
    assert e.value.code == tpthip.ERR_UNSUPPORTED
    bad = str(tmp_path / "bad.gguf")
    open(bad, "wb").write(b"GGUX" + data[4:])
    with pytest.raises(tpthip.TptError) as e:
        tpthip.Model(ctx, bad)
    assert e.value.code == tpthip.ERR_FORMAT


# ---------------------------------------------------------------- batched prefill

LONG_TOL = {"f32": 1e-3, "f16": FP16_LOGIT_TOL}


def test_batched_prefill_equals_steps(ctx, tiny_gguf, kv):
    """The MFMA prefill and the one-decode-step-per-position prefill compute the same Q8_K
    integer products; only f32 summation order differs."""
    prompt = [int(t) for t in np.random.default_rng(5).integers(0, 1024, 150)]
    m_b = tpthip.Model(ctx, tiny_gguf, max_ctx=256, kv_type=KV_TYPE[kv])
    os.environ["TPT_HIP_PREFILL"] = "steps"
    try:
        m_s = tpthip.Model(ctx, tiny_gguf, max_ctx=256, kv_type=KV_TYPE[kv])
    finally:
        del os.environ["TPT_HIP_PREFILL"]
    try:
        nb, lb = m_b.prefill(prompt, 0, logits=True)
        ns, ls = m_s.prefill(prompt, 0, logits=True)
        print("batched vs steps max-abs", np.abs(lb - ls).max())
        assert nb == ns
        assert np.abs(lb - ls).max() < LONG_TOL[kv]
        if kv == "f32":  # the caches agree: the next greedy tokens match
            assert m_b.decode_greedy(nb, len(prompt), 12) == m_s.decode_greedy(ns, len(prompt), 12)
    finally:
        m_b.close()
        m_s.close()


def test_tiny_long_prompt_matches_oracle(ctx, tiny_gguf, tiny_oracle, kv):
    """150-token prompt (several attention chunks on the step path) on both prefill paths."""
    prompt = [int(t) for t in np.random.default_rng(5).integers(0, 1024, 150)]
    tiny_oracle.reset(256, kv_f16=(kv == "f16"))
    ref = tiny_oracle.forward(prompt, 0)
    for path in ("batched", "steps"):
        if path == "steps":
            os.environ["TPT_HIP_PREFILL"] = "steps"
        try:
            m = tpthip.Model(ctx, tiny_gguf, max_ctx=256, kv_type=KV_TYPE[kv])
        finally:
            os.environ.pop("TPT_HIP_PREFILL", None)
        try:
            nxt, lg = m.prefill(prompt, 0, logits=True)
        finally:
            m.close()
        print(path, "max-abs vs oracle", np.abs(lg - ref).max())
        assert np.abs(lg - ref).max() < LONG_TOL[kv], path
        assert nxt == oracle.argmax(ref)


@pytest.fixture(scope="module")
def mixed_gguf(tmp_path_factory):
    """The tiny model typed as a real Q4_K_M file is: attn_v and ffn_down Q6_K in the layers
    llama.cpp's recipe gives more bits (here layer 1), everything else Q4_K."""
    path = str(tmp_path_factory.mktemp("mixed") / "tiny-q4_k_m-mixed.gguf")
    synth.write_llama(path, synth.TINY, seed=8, type_more_bits=tpthip.TYPE_Q6_K)
    return path


def test_mixed_q4k_q6k_prefill(ctx, mixed_gguf):
    """Q6_K layer matrices stay on the batched MFMA prefill (the Q6_K GEMM):
    * the layer holding Q6_K attn_v / ffn_down equals the step path on the same rows;
    * each layer, fed the oracle's own residual rows of a 150-token prompt (teacher-forced, f32
      cache: candle's), gives the oracle's next rows on both prefill paths within 1e-3
      relative L2 (only f32 rounding differs on identical inputs).
    End to end, 150 positions of this random-init model carry an occasional Q8_K rounding flip
    (under any f32 ordering difference) to the logits, which are therefore only reported."""
    prompt = [int(t) for t in np.random.default_rng(6).integers(0, 1024, 150)]
    om = oracle.Model(mixed_gguf)
    try:
        om.reset(256, kv_f16=False)
        ref, tr = om.forward_trace(prompt, 0)
    finally:
        om.close()
    m_b = tpthip.Model(ctx, mixed_gguf, max_ctx=256, kv_type=tpthip.TYPE_F32)
    os.environ["TPT_HIP_PREFILL"] = "steps"
    try:
        m_s = tpthip.Model(ctx, mixed_gguf, max_ctx=256, kv_type=tpthip.TYPE_F32)
    finally:
        del os.environ["TPT_HIP_PREFILL"]
    try:
        rows = np.random.default_rng(2).standard_normal((40, m_b.desc["embed"])).astype(np.float32)
        yb = m_b.run_layers(rows, 0, 1, 2, path=0)
        ys = m_s.run_layers(rows, 0, 1, 2, path=1)
        assert _rel_l2(yb, ys) < 1e-4
        errs = []
        for layer in range(tr.shape[0] - 1):
            for mm_, path in ((m_b, 0), (m_s, 1)):
                errs.append(_rel_l2(mm_.run_layers(tr[layer], 0, layer, layer + 1, path=path), tr[layer + 1]))
        _, lb = m_b.prefill(prompt, 0, logits=True)
        _, ls = m_s.prefill(prompt, 0, logits=True)
        print("layer 1 batched vs steps rel-l2", _rel_l2(yb, ys), "| teacher-forced layers rel-l2",
              [f"{e:.1e}" for e in errs], "| end to end max-abs vs oracle: batched",
              float(np.abs(lb - ref).max()), "steps", float(np.abs(ls - ref).max()))
        assert max(errs) < 1e-3, errs
    finally:
        m_b.close()
        m_s.close()


@pytest.mark.parametrize("qtype", [tpthip.TYPE_Q5_K, tpthip.TYPE_Q4_0, tpthip.TYPE_F16])
def test_other_quant_types_match_oracle(ctx, tmp_path, qtype):
    """A tiny model whose layer matrices are Q5_K, Q4_0 or F16 (token_embd / output Q6_K)
    against the oracle, f32 cache: prompt logits within 1e-3 and the first 16 greedy tokens
    identical.  Then a 150-token prompt through the batched MFMA prefill of the type (Q8_K
    activations for Q5_K, Q8_0 for Q4_0, the f32 split for F16), each layer fed the oracle's
    own input rows: for F16, where no activation is quantized, within 1e-5 relative L2; for the
    quantized types within 1e-2, the bar of the 1B teacher-forced layers -- over 150 positions
    an activation that sits on a rounding boundary of its Q8 quantization can round the other
    way under a different f32 summation order of the RMSNorm (4.6e-3 measured at layer 0 of
    the Q4_0 model, on the batched and the step-by-step path alike)."""
    path = str(tmp_path / f"tiny-{qtype}.gguf")
    synth.write_llama(path, synth.TINY, seed=9, type_matrix=qtype)
    om = oracle.Model(path)
    try:
        om.reset(64, kv_f16=False)
        ref = om.forward(PROMPT, 0)
        want = om.greedy(PROMPT, 16, kv_f16=False)[0]
    finally:
        om.close()
    m = tpthip.Model(ctx, path, max_ctx=64, kv_type=tpthip.TYPE_F32)
    try:
        nxt, lg = m.prefill(PROMPT, 0, logits=True)
        got = [nxt] + m.decode_greedy(nxt, len(PROMPT), 15)
    finally:
        m.close()
    print(qtype, "logits max-abs vs oracle", float(np.abs(lg - ref).max()))
    assert np.abs(lg - ref).max() < 1e-3
    assert got == want
    prompt = [int(t) for t in np.random.default_rng(5).integers(0, 1024, 150)]
    om = oracle.Model(path)
    try:
        om.reset(256, kv_f16=False)
        _, tr = om.forward_trace(prompt, 0)
    finally:
        om.close()
    m_b = tpthip.Model(ctx, path, max_ctx=256, kv_type=tpthip.TYPE_F32)
    try:
        errs = [_rel_l2(m_b.run_layers(tr[l], 0, l, l + 1, path=0), tr[l + 1]) for l in range(tr.shape[0] - 1)]
    finally:
        m_b.close()
    print(qtype, "batched 150-token prompt, teacher-forced layers rel-l2", [f"{e:.1e}" for e in errs])
    assert max(errs) < (1e-5 if qtype == tpthip.TYPE_F16 else 1e-2)


@pytest.fixture(scope="module")
def gguf_1b(tmp_path_factory):
    """Llama 1B shape (16 layers, hidden 2048, 32/8 heads, head_dim 64, FFN 8192, vocab 128256,
    theta 500000), Q4_K_M, weights N(0, 0.02), norms 1."""
    path = str(tmp_path_factory.mktemp("m1b") / "llama-1b-shape-q4_k_m.gguf")
    synth.write_llama(path, synth.LLAMA_1B, seed=1234, nthreads=min(os.cpu_count() or 1, 16))
    yield path
    os.remove(path)


PROMPT_1B = [int(t) for t in np.random.default_rng(128).integers(0, 128256, 128)]
_TRACES = {}


def oracle_trace_1b(path, kv_mode):
    """The oracle's residual stream at every layer boundary for the 128-token prompt (batched
    forward), then for one greedy decode token at position 128; cached per cache mode."""
    if kv_mode not in _TRACES:
        om = oracle.Model(path)
        om.reset(256, kv_f16=(kv_mode == "f16"))
        nt = min(os.cpu_count() or 1, 16)
        logits, tr = om.forward_trace(PROMPT_1B, 0, nt)
        tok = oracle.argmax(logits)
        _, tr2 = om.forward_trace([tok], len(PROMPT_1B), nt)
        kvs = [om.kv(l) for l in range(tr.shape[0] - 1)]
        om.close()
        _TRACES[kv_mode] = (logits, tr, tok, tr2, kvs)
    return _TRACES[kv_mode]


def _rel_l2(a, b):
    return float(np.linalg.norm((a - b).ravel()) / np.linalg.norm(b.ravel()))


def _row_rel(a, b):
    return np.linalg.norm(a - b, axis=-1) / np.linalg.norm(b, axis=-1)


@pytest.mark.timeout(900)
def test_1b_ops_on_oracle_layer_inputs(ctx, gguf_1b):
    """Every operation of a decoder layer at the 1B shape, fed the oracle's own intermediate
    values of layers 0, 5 and 15 (128 positions), against the oracle on the same values:
    RMSNorm, the Q4_K GEMV (Q8_K activations quantized on the GPU) and the MFMA GEMM for
    Q, Wo, gate and down, RoPE, attention over the oracle's cache, SwiGLU.  Identical inputs
    leave only f32 rounding: per-row relative error <= 2e-6 (attention 1e-5); SiLU equal but
    for < 0.1% of elements, which differ by at most two ulp (the host libm's expf is not
    correctly rounded for every argument; the device rounds the f64 exponential once, and a
    last-place change of exp(-g) passes through 1 + e and the divide)."""
    _, tr, _, _, kvs = oracle_trace_1b(gguf_1b, "f32")
    om = oracle.Model(gguf_1b)
    H, hd, nq, nkv, F, eps, n = 2048, 64, 32, 8, 8192, 1e-5, len(PROMPT_1B)
    cos_t, sin_t = oracle.rope_tables(hd, 500000.0, 256)
    dcos, dsin = ctx.to_device(cos_t), ctx.to_device(sin_t)
    worst = {}

    def check(name, got, want, tol=2e-6):
        e = float(_row_rel(got, want).max())
        worst[name] = max(worst.get(name, 0.0), e)
        assert e <= tol, (name, e)

    try:
        for layer in (0, 5, 15):
            X = tr[layer]
            t = {k: om.tensor(f"blk.{layer}.{k}.weight") for k in
                 ("attn_q", "attn_output", "ffn_gate", "ffn_down")}
            an = om.tensor(f"blk.{layer}.attn_norm.weight")[3].view(np.float32)
            fn = om.tensor(f"blk.{layer}.ffn_norm.weight")[3].view(np.float32)
            dan, dfn = ctx.to_device(an), ctx.to_device(fn)
            XN = np.stack([oracle.rmsnorm(x, an, eps) for x in X])
            check("rmsnorm", np.stack([ctx.rmsnorm(ctx.to_device(x), dan, H, eps) for x in X]), XN)

            def mat(key, A, N):
                qt, _, _, raw = t[key]
                want = oracle.matmul(qt, A, raw, N, 16)
                dw = ctx.to_device(raw)
                K = A.shape[1]
                check(key + " gemv", np.stack([ctx.gemv(qt, dw, ctx.to_device(a), K, N) for a in A[:32]]),
                      want[:32])
                check(key + " gemm", ctx.gemm(qt, dw, ctx.to_device(A), A.shape[0], K, N), want)
                return want

            Q = mat("attn_q", XN, nq * hd)
            Qr = np.stack([oracle.rope_i(Q[i], nq, hd, cos_t[i], sin_t[i]) for i in range(n)])
            check("rope", np.stack([ctx.rope(ctx.to_device(Q[i].copy()), nq, hd, i, dcos, dsin)
                                    for i in range(n)]), Qr)
            kc, vc = kvs[layer]
            dk, dv = ctx.to_device(kc), ctx.to_device(vc)
            A = np.stack([oracle.attention(Qr[i], kc, vc, nq, nkv, hd, i + 1) for i in range(n)])
            check("attention", np.stack([ctx.attn_decode(ctx.to_device(Qr[i]), dk, dv, nq, nkv, hd, i + 1,
                                                         kc.shape[1], kv_type=tpthip.TYPE_F32)
                                         for i in range(n)]), A, tol=1e-5)
            Xm = mat("attn_output", A, H) + X
            XN2 = np.stack([oracle.rmsnorm(x, fn, eps) for x in Xm])
            G = mat("ffn_gate", XN2, F)
            U = np.random.default_rng(layer).standard_normal(G.shape).astype(np.float32)
            S = np.stack([np.array([oracle.silu(v) for v in G[i]], np.float32) for i in range(8)])
            got = ctx.swiglu(ctx.to_device(G[:8]), ctx.to_device(np.ones_like(G[:8])), 8 * F).reshape(8, F)
            ulps = float((np.abs(got - S) / np.spacing(np.abs(S))).max())
            worst["silu ulp"] = max(worst.get("silu ulp", 0.0), ulps)
            worst["silu differs"] = max(worst.get("silu differs", 0.0), float(np.mean(got != S)))
            assert ulps <= 2 and np.mean(got != S) < 1e-3, ("silu", ulps, np.mean(got != S))
            want = S * U[:8]
            mat("ffn_down", want, H)
    finally:
        om.close()
    print({k: f"{v:.1e}" for k, v in worst.items()})


@pytest.mark.timeout(900)
def test_1b_layers_teacher_forced(ctx, gguf_1b, kv):
    """Each decoder layer at the 1B shape, fed the oracle's residual rows, against the oracle's
    next rows: the 128 prompt positions through the batched MFMA kernels and through the
    decode-step kernels, then position 128 on the decode path over the cache the batched run
    left.  The ops agree to f32 rounding on identical inputs (the test above); here the Q8_K
    activation quantization (and, in the fp16 mode, the fp16 K/V rounding) can flip under
    those rounding differences, and a flip in one position's K/V input reaches every later
    position through attention.  The oracle moves by the same amount under a change of its own
    dot-product summation order (block-reduced instead of candle's eight f32 lanes), so the bar
    is that size: relative L2 over the layer output <= 1e-2 (f32 cache) / 2e-2 (fp16 cache)."""
    _, tr, _, tr2, _ = oracle_trace_1b(gguf_1b, kv)
    tol = 1e-2 if kv == "f32" else 2e-2
    n_layers = tr.shape[0] - 1
    errs = {"batched": [], "steps": [], "decode": []}
    mb = tpthip.Model(ctx, gguf_1b, max_ctx=256, kv_type=KV_TYPE[kv])
    ms = tpthip.Model(ctx, gguf_1b, max_ctx=256, kv_type=KV_TYPE[kv])
    try:
        for l in range(n_layers):
            errs["batched"].append(_rel_l2(mb.run_layers(tr[l], 0, l, l + 1, path=0), tr[l + 1]))
            errs["steps"].append(_rel_l2(ms.run_layers(tr[l], 0, l, l + 1, path=1), tr[l + 1]))
        for l in range(n_layers):
            errs["decode"].append(_rel_l2(mb.run_layers(tr2[l], len(PROMPT_1B), l, l + 1, path=1),
                                          tr2[l + 1]))
    finally:
        mb.close()
        ms.close()
    print({k: f"{max(v):.2e}" for k, v in errs.items()})
    for k, v in errs.items():
        assert max(v) < tol, (k, v)


_FORCED = {}


def _forced_logits(path, prompt, toks, fma=True, block_order=False, nthreads=16, kv_f16=False,
                   rms_order=False):
    """Oracle logits at every step of a teacher-forced run (f32 cache, candle's, unless kv_f16):
    step 0 after the prompt, step i after feeding toks[i-1].  Cached per arguments."""
    key = (path, tuple(prompt), tuple(toks), fma, block_order, kv_f16, rms_order)
    if key not in _FORCED:
        _FORCED[key] = _forced_logits_run(path, prompt, toks, fma, block_order, nthreads, kv_f16,
                                          rms_order)
    return _FORCED[key]


def _forced_logits_run(path, prompt, toks, fma, block_order, nthreads, kv_f16, rms_order=False):
    om = oracle.Model(path)
    try:
        om.set_attn_fma(fma)
        oracle.set_dot_block_order(block_order)
        oracle.set_rms_order(rms_order)
        om.reset(len(prompt) + len(toks) + 1, kv_f16=kv_f16)
        out = [om.forward(prompt, 0, nthreads)]
        for i, t in enumerate(toks[:-1]):
            out.append(om.forward([t], len(prompt) + i, nthreads))
        return np.stack(out)
    finally:
        oracle.set_dot_block_order(False)
        oracle.set_rms_order(False)
        om.close()


def _margin(l):
    top = np.sort(l)[-2:]
    return float(top[1] - top[0])


_GREEDY = {}


def _greedy_1b(path, nt):
    """The oracle's (candle's, f32 cache) 128 greedy tokens after the 1B prompt."""
    if path not in _GREEDY:
        om = oracle.Model(path)
        try:
            _GREEDY[path] = om.greedy(PROMPT_1B, 128, kv_f16=False, nthreads=nt)[0]
        finally:
            om.close()
    return _GREEDY[path]


def _gpu_forced(ctx, path, toks, kv_type):
    """GPU logits and greedy tokens at every step of the teacher-forced 1B run."""
    m = tpthip.Model(ctx, path, max_ctx=512, kv_type=kv_type)
    try:
        nxt, lg = m.prefill(PROMPT_1B, 0, logits=True)
        got, gtok = [lg], [nxt]
        for i, t in enumerate(toks[:-1]):
            nxt, lg = m.decode_step(t, len(PROMPT_1B) + i, logits=True)
            got.append(lg)
            gtok.append(nxt)
    finally:
        m.close()
    return np.stack(got), gtok


@pytest.mark.timeout(1200)
def test_1b_teacher_forced_decode(ctx, gguf_1b):
    """Config 1 end to end against candle's arithmetic: the 128-token prompt, then the 128 greedy
    tokens of the oracle's own run (candle_engine.rs:269-324), teacher-forced into both sides,
    f32 cache (candle's).  The oracle's summation order inside candle's dot products is unpinned,
    and this random-init model amplifies any order change (a Q8_K activation value that rounds
    the other way moves the next layer), so the bar is the oracle's own spread S: the largest
    max-abs logit distance, over all 128 steps, between the oracle and the oracle run with the
    other plausible orders (separate multiply-adds in attention, as the gemm crate on a host
    without FMA; block-reduced k-quant dot products; RMSNorm's sum of squares in the tree order
    a GPU reduction takes; all three at once, as the device changes every reduction's order
    together).  Every step: GPU logits within S of
    the oracle, and the GPU's greedy token equal to the oracle's wherever the oracle's top-two
    margin exceeds S (a margin below S is a token candle itself could pick either way).  Then
    free-running: the GPU's greedy tokens equal the oracle's up to the first such close step, and
    over at least the first 32 tokens when no close step comes earlier."""
    nt = min(os.cpu_count() or 1, 16)
    ref_toks = _greedy_1b(gguf_1b, nt)
    ref = _forced_logits(gguf_1b, PROMPT_1B, ref_toks, nthreads=nt)
    alt_fma = _forced_logits(gguf_1b, PROMPT_1B, ref_toks, fma=False, nthreads=nt)
    alt_blk = _forced_logits(gguf_1b, PROMPT_1B, ref_toks, block_order=True, nthreads=nt)
    alt_rms = _forced_logits(gguf_1b, PROMPT_1B, ref_toks, rms_order=True, nthreads=nt)
    alt_all = _forced_logits(gguf_1b, PROMPT_1B, ref_toks, fma=False, block_order=True, rms_order=True,
                             nthreads=nt)
    spread = np.max([np.abs(a - ref).max(axis=1) for a in (alt_fma, alt_blk, alt_rms, alt_all)], axis=0)
    S = float(spread.max())
    m = tpthip.Model(ctx, gguf_1b, max_ctx=512, kv_type=tpthip.TYPE_F32)
    try:
        nxt, lg = m.prefill(PROMPT_1B, 0, logits=True)
        got, gtok = [lg], [nxt]
        for i, t in enumerate(ref_toks[:-1]):
            nxt, lg = m.decode_step(t, len(PROMPT_1B) + i, logits=True)
            got.append(lg)
            gtok.append(nxt)
        got = np.stack(got)
        first = m.prefill(PROMPT_1B, 0)
        free = [first] + m.decode_greedy(first, len(PROMPT_1B), 127)
    finally:
        m.close()
    dev = np.abs(got - ref).max(axis=1)
    rel = np.linalg.norm(got - ref, axis=1) / np.linalg.norm(ref, axis=1)
    margins = np.array([_margin(l) for l in ref])
    close = margins <= S
    print(f"1B teacher-forced, 128 steps: gpu-oracle max-abs logits max {dev.max():.4f} "
          f"median {np.median(dev):.4f}, rel-l2 max {rel.max():.4f}; oracle spread S {S:.4f} (per step median "
          f"{np.median(spread):.4f}); logit std {float(ref.std()):.3f}; steps with top-2 margin "
          f"<= S: {int(close.sum())} {np.flatnonzero(close).tolist()}; tokens equal where gated-in: "
          f"{int(sum(g == r for g, r, c in zip(gtok, ref_toks, close) if not c))}/{int((~close).sum())}")
    assert dev.max() <= S, (dev.max(), S)
    for i in np.flatnonzero(~close):
        assert gtok[i] == ref_toks[i], (i, gtok[i], ref_toks[i], margins[i])
    n_ok = int(np.flatnonzero(close)[0]) if close.any() else 128
    assert free[:n_ok] == ref_toks[:n_ok]
    if n_ok >= 32:
        assert free[:32] == ref_toks[:32]


@pytest.mark.timeout(1200)
def test_1b_teacher_forced_decode_fp16_cache(ctx, gguf_1b):
    """Config 1 with the library's default fp16 KV cache, teacher-forced with candle's greedy
    tokens (the oracle with candle's f32 cache).  Two bars:
      * against the oracle run with the same fp16 rounding of the cache: GPU logits within S16,
        the largest max-abs distance over all steps between that run and the same run in
        the other plausible orders (no FMA in attention; block-reduced dots; tree-ordered
        RMSNorm sum of squares; all three at once);
      * against candle itself (f32 cache): the fp16 cache is a different arithmetic, and on this
        model it moves candle's logits by D, the largest distance over all steps between any of
        the oracle's five fp16-cache runs and candle's f32 run.  The GPU's greedy token equals
        candle's at every step whose top-two margin exceeds D."""
    nt = min(os.cpu_count() or 1, 16)
    ref_toks = _greedy_1b(gguf_1b, nt)
    ref32 = _forced_logits(gguf_1b, PROMPT_1B, ref_toks, nthreads=nt)
    ref16 = _forced_logits(gguf_1b, PROMPT_1B, ref_toks, nthreads=nt, kv_f16=True)
    alt16 = [_forced_logits(gguf_1b, PROMPT_1B, ref_toks, fma=False, nthreads=nt, kv_f16=True),
             _forced_logits(gguf_1b, PROMPT_1B, ref_toks, block_order=True, nthreads=nt, kv_f16=True),
             _forced_logits(gguf_1b, PROMPT_1B, ref_toks, rms_order=True, nthreads=nt, kv_f16=True),
             _forced_logits(gguf_1b, PROMPT_1B, ref_toks, fma=False, block_order=True, rms_order=True,
                            nthreads=nt, kv_f16=True)]
    S16 = max(float(np.abs(a - ref16).max()) for a in alt16)
    D = max(float(np.abs(c - ref32).max()) for c in [ref16] + alt16)
    got, gtok = _gpu_forced(ctx, gguf_1b, ref_toks, tpthip.TYPE_F16)
    dev16 = np.abs(got - ref16).max(axis=1)
    dev32 = np.abs(got - ref32).max(axis=1)
    margins = np.array([_margin(l) for l in ref32])
    decisive = np.flatnonzero(margins > D)
    print(f"1B fp16 cache, 128 steps: gpu vs oracle(fp16 cache) max {dev16.max():.4f} median "
          f"{np.median(dev16):.4f}, S16 {S16:.4f}; gpu vs candle(f32 cache) max {dev32.max():.4f} "
          f"median {np.median(dev32):.4f}, D {D:.4f}; tokens equal at "
          f"{int(sum(gtok[i] == ref_toks[i] for i in decisive))}/{decisive.size} steps with margin > D")
    assert dev16.max() <= S16, (dev16.max(), S16)
    for i in decisive:
        assert gtok[i] == ref_toks[i], (i, gtok[i], ref_toks[i], margins[i])


@pytest.mark.timeout(900)
def test_1b_kv_cache_matches_oracle(ctx, gguf_1b, kv):
    """K/V cache contents of every layer at the 1B shape, read back with tpt_model_kv_read,
    against the oracle's cache after the 128-token prompt, each layer fed the oracle's own input
    rows (teacher-forced, through the batched prefill and through the decode-step kernels), so
    that each layer's K/V rows come from identical inputs: layout [kv head][position][head_dim]
    with RoPE applied to K, in the mode's element type, within 2e-4 relative L2 (the f32 order
    of the RMSNorm and GEMV sums can move a Q8_K activation value by one step, a K/V element by
    ~5e-4 of its size; fp16's own rounding is 4.9e-4); positions past the prompt untouched."""
    _, tr, _, _, kvs = oracle_trace_1b(gguf_1b, kv)
    n = len(PROMPT_1B)
    worst = {}
    for path in (0, 1):
        m = tpthip.Model(ctx, gguf_1b, max_ctx=256, kv_type=KV_TYPE[kv])
        try:
            for layer in range(16):
                m.run_layers(tr[layer], 0, layer, layer + 1, path=path)
                for g, o, name in zip(m.kv(layer), kvs[layer], "KV"):
                    assert g.shape == o.shape == (8, 256, 64)
                    assert not np.any(g[:, n:]), "positions past the prompt were written"
                    e = _rel_l2(g[:, :n], o[:, :n])
                    worst[(path, name)] = max(worst.get((path, name), 0.0), e)
                    assert e < 2e-4, (path, layer, name, e)
        finally:
            m.close()
    print(kv, "kv rel-l2, worst layer:", {f"{'batched' if p == 0 else 'steps'} {n_}": f"{e:.1e}"
                                          for (p, n_), e in worst.items()})
