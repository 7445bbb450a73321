"""The oracle's model composition (quantized_llama::ModelWeights::forward restated in
oracle/oracle.c layers_forward / orc_model_forward_trace) pinned by closed forms on the CPU.

The per-op functions are pinned elsewhere (tests/test_oracle_golden.py).  Here, weight tensors of
a seeded tiny Llama GGUF are replaced so that the forward pass collapses to an expression of
those pinned primitives, which the reference's op order fixes (candle_engine.rs:272-273 runs
quantized_llama's forward; wgpu_engine.rs:339-490 gives the same op sequence without the
residual adds):

* attn_output = ffn_down = 0: both residual branches add exactly zero, so every layer leaves the
  residual rows equal to the embedding rows bit for bit, and the logits are
  output . rmsnorm(embed(last token), output_norm);
* ffn_down = 0, one-token prompt: attention over one position returns v, so each layer maps x
  to x + Wo . (Wv . rmsnorm(x, attn_norm));
* attn_output = 0: each layer maps x to x + Wdown . (silu(Wgate . n) * (Wup . n)) with
  n = rmsnorm(x, ffn_norm);
* any prompt: the logits come from the last position's residual row only.

Every norm weight vector is replaced by distinct random values, so a norm applied with the
wrong weights (or not at all) changes the result, and each closed form is checked to differ
from what a plausible composition mistake would give (k for v, gate/up swapped, the wrong
norm, the first position instead of the last)."""
import numpy as np
import pytest

import oracle
from gguf_edit import Gguf
from tpthip import synth

CFG = synth.TINY
H, F, V, NL = CFG["embed"], CFG["ffn"], CFG["vocab"], CFG["n_layers"]
NQ, NKV = CFG["n_heads"], CFG["n_kv_heads"]
HD = H // NQ
EPS = CFG["rms_eps"]


def _model(tmp_path, name, zero=()):
    """The tiny model with random norm weights and the named matrices zeroed in every layer."""
    src = str(tmp_path / "src.gguf")
    synth.write_llama(src, CFG, seed=21)
    g = Gguf(src)
    rng = np.random.default_rng(22)
    for t in g.tensors:
        if t["name"].endswith("norm.weight"):
            g.set_payload(t["name"], rng.uniform(0.5, 1.5, t["ne"][0]).astype(np.float32).tobytes())
        if any(t["name"].endswith(z + ".weight") for z in zero):
            g.zero(t["name"])
    return oracle.Model(g.write(str(tmp_path / name)))


def _w(m, name):
    t, n0, n1, raw = m.tensor(name)
    return t, n1, raw


def _mm(m, name, x):
    t, n, raw = _w(m, name)
    return oracle.matmul(t, x, raw, n, 1)


def _norm(m, name, x):
    return np.stack([oracle.rmsnorm(r, _w(m, name)[2].view(np.float32), EPS) for r in np.atleast_2d(x)])


def _embed(m, tok):
    t, _, raw = _w(m, "token_embd.weight")
    rb = oracle.row_bytes(t, H)
    return oracle.dequant(t, raw[tok * rb:(tok + 1) * rb], H)


def _silu(a):
    return np.array([oracle.silu(v) for v in a.ravel()], np.float32).reshape(a.shape)


def test_zero_branches_keep_the_embedding(tmp_path):
    m = _model(tmp_path, "zero_both.gguf", zero=("attn_output", "ffn_down"))
    prompt = [3, 500, 17]
    m.reset(8)
    logits, tr = m.forward_trace(prompt, 0, 1)
    emb = np.stack([_embed(m, t) for t in prompt])
    for l in range(NL + 1):
        assert np.array_equal(tr[l], emb), l
    want = _mm(m, "output.weight", _norm(m, "output_norm.weight", emb[-1]))[0]
    assert np.array_equal(logits, want)
    # the closed form discriminates: the first position, or no final norm, give other logits
    assert not np.array_equal(logits, _mm(m, "output.weight", _norm(m, "output_norm.weight", emb[0]))[0])
    assert not np.array_equal(logits, _mm(m, "output.weight", emb[-1:])[0])
    assert not np.array_equal(logits, _mm(m, "output.weight", _norm(m, "blk.0.attn_norm.weight", emb[-1]))[0])


@pytest.mark.parametrize("kv_f16", [False, True])
def test_single_position_attention_layer(tmp_path, kv_f16):
    m = _model(tmp_path, "zero_ffn.gguf", zero=("ffn_down",))
    m.reset(8, kv_f16=kv_f16)
    logits, tr = m.forward_trace([77], 0, 1)
    assert np.array_equal(tr[0][0], _embed(m, 77))
    for l in range(NL):
        x = tr[l]
        n = _norm(m, f"blk.{l}.attn_norm.weight", x)
        v = _mm(m, f"blk.{l}.attn_v.weight", n)
        if kv_f16:  # the cache holds v rounded to fp16, and attention returns the cached row
            v = v.astype(np.float16).astype(np.float32)  # round to nearest even, as the cache
        got = tr[l + 1]
        # repeat_kv: query head h reads kv head h // (nq / nkv), and with one position its
        # attention output is that head's v row
        rep = NQ // NKV
        attn = np.concatenate([v[:, (h // rep) * HD:(h // rep + 1) * HD] for h in range(NQ)], axis=1)
        assert np.array_equal(got, x + _mm(m, f"blk.{l}.attn_output.weight", attn)), l
        # mistakes the form would catch: the kv head h % nkv, k in place of v, the ffn norm
        wrong = np.concatenate([v[:, (h % NKV) * HD:(h % NKV + 1) * HD] for h in range(NQ)], axis=1)
        assert not np.array_equal(got, x + _mm(m, f"blk.{l}.attn_output.weight", wrong))
        k = _mm(m, f"blk.{l}.attn_k.weight", n)
        ka = np.concatenate([k[:, (h // rep) * HD:(h // rep + 1) * HD] for h in range(NQ)], axis=1)
        assert not np.array_equal(got, x + _mm(m, f"blk.{l}.attn_output.weight", ka))
        n2 = _norm(m, f"blk.{l}.ffn_norm.weight", x)
        v2 = _mm(m, f"blk.{l}.attn_v.weight", n2)
        a2 = np.concatenate([v2[:, (h // rep) * HD:(h // rep + 1) * HD] for h in range(NQ)], axis=1)
        assert not np.array_equal(got, x + _mm(m, f"blk.{l}.attn_output.weight", a2))
    want = _mm(m, "output.weight", _norm(m, "output_norm.weight", tr[NL][-1]))[0]
    assert np.array_equal(logits, want)


def test_feed_forward_layer(tmp_path):
    m = _model(tmp_path, "zero_attn.gguf", zero=("attn_output",))
    prompt = [5, 900, 12, 44]
    m.reset(8)
    logits, tr = m.forward_trace(prompt, 0, 1)
    for l in range(NL):
        x = tr[l]
        n = _norm(m, f"blk.{l}.ffn_norm.weight", x)
        g = _mm(m, f"blk.{l}.ffn_gate.weight", n)
        u = _mm(m, f"blk.{l}.ffn_up.weight", n)
        got = tr[l + 1]
        assert np.array_equal(got, x + _mm(m, f"blk.{l}.ffn_down.weight", _silu(g) * u)), l
        # silu on the up projection instead of the gate, or the attention norm, differ
        assert not np.array_equal(got, x + _mm(m, f"blk.{l}.ffn_down.weight", g * _silu(u)))
        na = _norm(m, f"blk.{l}.attn_norm.weight", x)
        ga, ua = _mm(m, f"blk.{l}.ffn_gate.weight", na), _mm(m, f"blk.{l}.ffn_up.weight", na)
        assert not np.array_equal(got, x + _mm(m, f"blk.{l}.ffn_down.weight", _silu(ga) * ua))
    assert np.array_equal(logits, _mm(m, "output.weight", _norm(m, "output_norm.weight", tr[NL][-1]))[0])


def test_logits_come_from_the_last_position(tmp_path):
    m = _model(tmp_path, "full.gguf")
    prompt = [8, 300, 1000, 2, 640]
    m.reset(16)
    logits, tr = m.forward_trace(prompt, 0, 1)
    fin = tr[NL]
    assert np.array_equal(logits, _mm(m, "output.weight", _norm(m, "output_norm.weight", fin[-1]))[0])
    for t in range(len(prompt) - 1):
        assert not np.array_equal(logits, _mm(m, "output.weight", _norm(m, "output_norm.weight", fin[t]))[0])
    # the same last-position logits from a step-by-step run (batched == stepwise composition)
    m.reset(16)
    m.forward(prompt[:3], 0, 1)
    m.forward(prompt[3:4], 3, 1)
    step = m.forward(prompt[4:], 4, 1)
    assert np.abs(step - logits).max() < 1e-5
