"""CPU-side checks of the product: the C ABI library loads and exports what include/tpthip.h
declares; host-only logic (KV prefix reuse, the workload generator) behaves."""
import ctypes
import os
import re

import numpy as np
import pytest

import tpthip
from tpthip import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    hdr = open(os.path.join(ROOT, "include", "tpthip.h")).read()
    hdr = re.sub(r"/\*.*?\*/", "", hdr, flags=re.S)
    return sorted(set(re.findall(r"\b(tpt_[a-z0-9_]+)\s*\(", hdr)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(tpthip.LIB_PATH)
    names = declared_symbols()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(tpthip.EXPORTS), set(names) ^ set(tpthip.EXPORTS)


def test_library_is_gfx950_code_object():
    # the offload bundle embedded in the shared object names its target
    blob = open(tpthip.LIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob


def test_version_and_error_plumbing():
    lib = tpthip.lib()
    assert lib.tpt_version() == 1
    # a host-side validation error sets the thread's last error without touching a device
    assert lib.tpt_engine_is_loaded(None) == 0


# ---- KvCache prefix reuse: the reference's own tests (wgpu_kvcache.rs:96-133) re-hosted

def test_empty_cache_returns_zero():
    assert tpthip.common_prefix_len([], [1, 2, 3]) == 0


def test_full_prefix_match():
    assert tpthip.common_prefix_len([1, 2, 3], [1, 2, 3, 4, 5]) == 3


def test_diverges_at_second_token():
    assert tpthip.common_prefix_len([1, 99, 3], [1, 2, 3]) == 1


def test_no_match_at_all():
    assert tpthip.common_prefix_len([5, 6, 7], [1, 2, 3]) == 0


def test_new_tokens_shorter_than_cached():
    assert tpthip.common_prefix_len([1, 2, 3, 4, 5], [1, 2, 3]) == 3


# test_reset_clears_tokens (wgpu_kvcache.rs:126-132) drives the engine's KvCache::reset
# equivalent, tpt_engine_reset_cache, so it needs a device: tests/test_gpu_model.py.


# ---- GGUF validation without a device (tpt_model_inspect: extract_meta + the loader's checks)

@pytest.fixture(scope="module")
def tiny_file(tmp_path_factory):
    p = str(tmp_path_factory.mktemp("gguf") / "tiny.gguf")
    synth.write_llama(p, synth.TINY, seed=3)
    return p


def test_inspect_reads_the_metadata(tiny_file):
    d = tpthip.inspect_gguf(tiny_file)
    assert d["architecture"] == "llama"
    assert (d["n_layers"], d["embed"], d["n_heads"], d["n_kv_heads"], d["head_dim"], d["ffn"],
            d["vocab"], d["context_length"]) == (2, 256, 4, 2, 64, 512, 1024, 512)
    assert abs(d["rope_base"] - 500000.0) < 1 and abs(d["rms_eps"] - 1e-5) < 1e-9
    assert d["type_q"] == tpthip.TYPE_Q4_K and d["type_out"] == tpthip.TYPE_Q6_K
    # weight bytes: every tensor once; a decode step reads every layer tensor, the LM head,
    # the final norm and one embedding row
    from gguf_edit import Gguf
    g = Gguf(tiny_file)
    size = {t["name"]: int(np.prod(t["ne"])) // tpthip.BLOCK[t["type"]] * tpthip.TYPE_SIZE[t["type"]]
            for t in g.tensors}
    assert d["weight_bytes"] == sum(size.values())
    emb_row = 256 // 256 * tpthip.TYPE_SIZE[tpthip.TYPE_Q6_K]
    assert d["decode_bytes_per_token"] == sum(size.values()) - size["token_embd.weight"] + emb_row


def _bad(tiny_file, tmp_path, edit):
    from gguf_edit import Gguf
    g = Gguf(tiny_file)
    edit(g)
    return g.write(str(tmp_path / "bad.gguf"))


def _expect(path, code, text):
    with pytest.raises(tpthip.TptError) as e:
        tpthip.inspect_gguf(path)
    assert e.value.code == code and text in str(e.value), str(e.value)


def test_inspect_rewritten_file_is_valid(tiny_file, tmp_path):
    # the editor round-trips: an unchanged rewrite still validates
    assert tpthip.inspect_gguf(_bad(tiny_file, tmp_path, lambda g: None))["n_layers"] == 2


def test_inspect_rejects_zero_extent(tiny_file, tmp_path):
    # [256, 256, 0]: zero bytes; the kernels would read 256 rows past it
    def edit(g):
        g.tensor("blk.0.attn_q.weight")["ne"] = [256, 256, 0]
    _expect(_bad(tiny_file, tmp_path, edit), tpthip.ERR_FORMAT, "unexpected shape")


def test_inspect_rejects_extra_dimensions(tiny_file, tmp_path):
    def edit(g):
        g.tensor("blk.1.ffn_down.weight")["ne"] = [512, 128, 2]
    _expect(_bad(tiny_file, tmp_path, edit), tpthip.ERR_FORMAT, "unexpected shape")


def test_inspect_rejects_huge_extent(tiny_file, tmp_path):
    def edit(g):
        g.tensor("blk.0.attn_k.weight")["ne"] = [256, 1 << 41]
    _expect(_bad(tiny_file, tmp_path, edit), tpthip.ERR_FORMAT, "extent out of range")


def test_inspect_rejects_overflowing_element_count(tiny_file, tmp_path):
    # each extent below 2^40, the product past 2^62
    def edit(g):
        g.tensor("blk.0.attn_k.weight")["ne"] = [256, (1 << 39) + 1, 1 << 30]
    _expect(_bad(tiny_file, tmp_path, edit), tpthip.ERR_FORMAT, "too many elements")


def test_inspect_rejects_wrapping_offset(tiny_file, tmp_path):
    # data offset + tensor offset wraps past 2^64 onto a small address
    def edit(g):
        g.tensor("output_norm.weight")["offset"] = (1 << 64) - 64
    _expect(_bad(tiny_file, tmp_path, edit), tpthip.ERR_FORMAT, "past end of file")


def test_inspect_rejects_tensor_past_eof(tiny_file, tmp_path):
    def edit(g):
        t = g.tensor("blk.1.ffn_up.weight")
        t["offset"] = len(g.data) - 100
    _expect(_bad(tiny_file, tmp_path, edit), tpthip.ERR_FORMAT, "past end of file")


def test_inspect_rejects_wrong_row_length(tiny_file, tmp_path):
    def edit(g):
        g.tensor("blk.0.ffn_gate.weight")["ne"] = [512, 256]
    _expect(_bad(tiny_file, tmp_path, edit), tpthip.ERR_FORMAT, "unexpected shape")


def test_inspect_rejects_unsupported_matrix_type(tiny_file, tmp_path):
    # ggml type 3 (Q4_1): a block type this engine does not read
    def edit(g):
        g.tensor("blk.0.attn_v.weight")["type"] = 3
    _expect(_bad(tiny_file, tmp_path, edit), tpthip.ERR_UNSUPPORTED, "does not read")


def test_inspect_missing_file_and_bad_magic(tiny_file, tmp_path):
    _expect(str(tmp_path / "none.gguf"), tpthip.ERR_IO, "opening")
    p = str(tmp_path / "magic.gguf")
    open(p, "wb").write(b"GGUX" + open(tiny_file, "rb").read()[4:])
    _expect(p, tpthip.ERR_FORMAT, "bad magic")


# ---- workload generator

def test_synth_is_deterministic_across_thread_counts(tmp_path):
    a, b = str(tmp_path / "a.gguf"), str(tmp_path / "b.gguf")
    synth.write_llama(a, synth.TINY, seed=3, nthreads=1)
    synth.write_llama(b, synth.TINY, seed=3, nthreads=7)
    assert open(a, "rb").read() == open(b, "rb").read()
    c = str(tmp_path / "c.gguf")
    synth.write_llama(c, synth.TINY, seed=4)
    assert open(a, "rb").read() != open(c, "rb").read()


def test_synth_file_reads_back_in_the_oracle(tmp_path):
    import oracle
    p = str(tmp_path / "t.gguf")
    synth.write_llama(p, synth.TINY, seed=1)
    m = oracle.Model(p)
    c = m.cfg
    assert (c["n_layers"], c["embed"], c["n_heads"], c["n_kv_heads"], c["ffn"], c["vocab"]) == \
        (2, 256, 4, 2, 512, 1024)
    assert abs(c["rope_base"] - 500000.0) < 1 and abs(c["eps"] - 1e-5) < 1e-9
    t, n0, n1, raw = m.tensor("blk.0.attn_q.weight")
    assert (t, n0, n1) == (tpthip.TYPE_Q4_K, 256, 256)
    w = oracle.dequant(t, raw, n0 * n1)
    assert 0.015 < w.std() < 0.025 and abs(w.mean()) < 2e-3  # N(0, 0.02) through Q4_K
    t, _, _, raw = m.tensor("token_embd.weight")
    assert t == tpthip.TYPE_Q6_K
    t, _, _, raw = m.tensor("output_norm.weight")
    assert np.all(raw.view(np.float32) == 1.0)


def test_normal_generator_statistics():
    x = synth.normal(5, "stats", 1 << 18)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01
    assert np.array_equal(x[1000:1010], synth.normal(5, "stats", 10, i0=1000))


@pytest.mark.parametrize("qtype", [tpthip.TYPE_Q4_K, tpthip.TYPE_Q6_K, tpthip.TYPE_Q8_0])
def test_quantizer_round_trip(qtype):
    import oracle
    x = synth.normal(2, "rt", 8192, 0.02)
    y = oracle.dequant(qtype, synth.quantize(qtype, x), x.size)
    err = np.linalg.norm(y - x) / np.linalg.norm(x)
    assert err < {tpthip.TYPE_Q4_K: 0.1, tpthip.TYPE_Q6_K: 0.03, tpthip.TYPE_Q8_0: 0.01}[qtype]
