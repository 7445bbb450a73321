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
    """40 greedy tokens identical to the oracle in the same cache mode; for the f32 cache that
    is candle's greedy sequence (the bar: the first 32 identical, logits within 1e-2)."""
    n = 40
    toks_ref, logits_ref = tiny_oracle.greedy(PROMPT, n, kv_f16=(kv == "f16"), return_logits=(1, 32))
    first = tiny_model.prefill(PROMPT, 0)
    got = [first] + tiny_model.decode_greedy(first, len(PROMPT), n - 1)
    assert got[:32] == toks_ref[:32]
    assert got == toks_ref
    # logits of a later step through the single-step path
    pos = len(PROMPT)
    tiny_model.prefill(PROMPT, 0)
    for i in range(31):
        tiny_model.decode_step(got[i], pos + i)
    _, lg = tiny_model.decode_step(got[31], pos + 31, logits=True)
    assert np.abs(lg - logits_ref[32]).max() < 1e-2


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
