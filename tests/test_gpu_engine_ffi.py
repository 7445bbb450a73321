"""The C ABI driven the way the Rust engine (tpt-spark_amd/rust/engine/hip_engine.rs) drives it,
with raw ctypes calls and no Python wrapper in between:

* load with a progress trampoline whose `user` points at a caller-owned slot that outlives the
  call (the slot holds the callable; here an index into a registry);
* infer from OS threads other than the one that loaded, one call at a time under a lock (the
  Mutex the Rust engine holds across tpt_engine_infer, as EngineHandle's tokio Mutex does,
  src-tauri/src/engine/mod.rs:95);
* cancel by returning non-zero from the token trampoline, after which exactly one done=1 event
  arrives and tpt_engine_infer returns TPT_ERR_CANCELLED (wgpu_engine.rs:297-300);
* reset, reload, unload and the ERR_STATE of an engine with no model.
Greedy results are compared with the oracle (candle's arithmetic) in the f32 cache mode."""
import ctypes as C
import os
import threading

import pytest

import oracle
import tpthip

pytestmark = pytest.mark.gpu

PROMPT = [11, 500, 7, 1023, 42, 99, 3]

_REGISTRY = {}


class Slot(C.Structure):
    _fields_ = [("key", C.c_int64)]


@tpthip.PROGRESS_FN
def progress_tramp(user, done, total):
    key = C.cast(user, C.POINTER(Slot)).contents.key
    _REGISTRY[key](done, total)


@tpthip.TOKEN_FN
def token_tramp(user, token, done):
    key = C.cast(user, C.POINTER(Slot)).contents.key
    return _REGISTRY[key](token, done)


def params(max_tokens, eos=-1):
    p = tpthip._InferParamsC()
    p.max_tokens, p.temperature, p.top_p, p.repeat_penalty = max_tokens, 0.0, 1.0, 1.0
    p.eos_token_id, p.seed = eos, 42
    return p


def infer(lib, e, prompt, p, on_token):
    """One tpt_engine_infer call with the token trampoline; returns (rc, stats)."""
    slot = Slot(id(on_token))
    _REGISTRY[slot.key] = on_token
    ids = (C.c_uint32 * len(prompt))(*prompt)
    st = tpthip.InferStats()
    try:
        rc = lib.tpt_engine_infer(e, C.byref(p), ids, len(prompt), token_tramp, C.byref(slot),
                                  C.byref(st))
    finally:
        del _REGISTRY[slot.key]
    return rc, st


def in_thread(fn):
    out = {}

    def run():
        try:
            out["v"] = fn()
        except BaseException as ex:  # re-raised in the caller
            out["e"] = ex
    t = threading.Thread(target=run)
    t.start()
    t.join()
    if "e" in out:
        raise out["e"]
    return out["v"]


@pytest.fixture(scope="module")
def engine_h(tiny_gguf):
    lib = tpthip.lib()
    e = C.c_void_p()
    assert lib.tpt_engine_create(0, C.byref(e)) == 0
    assert lib.tpt_engine_set_kv_type(e, tpthip.TYPE_F32) == 0
    yield lib, e
    assert lib.tpt_engine_destroy(e) == 0


def test_ffi_load_progress_and_info(engine_h, tiny_gguf):
    lib, e = engine_h
    assert lib.tpt_engine_is_loaded(e) == 0
    seen = []
    slot = Slot(7001)
    _REGISTRY[slot.key] = lambda d, t: seen.append((d, t))
    info = tpthip._ModelInfoC()
    try:
        rc = lib.tpt_engine_load(e, tiny_gguf.encode(), progress_tramp, C.byref(slot), C.byref(info))
    finally:
        del _REGISTRY[slot.key]
    assert rc == 0, lib.tpt_last_error()
    total = seen[-1][1]
    assert seen == [(i + 1, total) for i in range(total)]  # once per tensor, in order
    assert lib.tpt_engine_is_loaded(e) == 1
    assert info.name.decode() == "tiny" and info.size_bytes == os.path.getsize(tiny_gguf)
    assert info.backend.decode().startswith("hip-gfx")
    # a null progress function is accepted (on_progress: None)
    assert lib.tpt_engine_load(e, tiny_gguf.encode(), tpthip.PROGRESS_FN(), None, C.byref(info)) == 0


def test_ffi_infer_from_other_threads(engine_h, tiny_gguf):
    lib, e = engine_h
    om = oracle.Model(tiny_gguf)
    ref, _ = om.greedy(PROMPT, 12)
    om.close()
    lock = threading.Lock()  # the Mutex held across tpt_engine_infer

    def one_turn():
        toks, dones = [], []

        def on_token(tok, done):
            (dones if done else toks).append(tok)
            return 0
        with lock:
            assert lib.tpt_engine_reset_cache(e) == 0
            rc, st = infer(lib, e, PROMPT, params(12), on_token)
        return rc, st, toks, dones

    for _ in range(3):  # three calls, each on a new OS thread
        rc, st, toks, dones = in_thread(one_turn)
        assert rc == 0, lib.tpt_last_error()
        assert toks == ref and len(dones) == 1
        assert st.prompt_tokens == len(PROMPT) and st.generated == 12 and st.cached_prefix == 0


def test_ffi_cancel_delivers_done(engine_h, tiny_gguf):
    lib, e = engine_h
    om = oracle.Model(tiny_gguf)
    ref, _ = om.greedy(PROMPT, 20)
    om.close()
    events = []

    def on_token(tok, done):
        events.append((tok, done))
        if not done and len(events) == 4:
            return 1  # the Rust trampoline's answer to on_token returning Err
        return 0
    assert lib.tpt_engine_reset_cache(e) == 0
    rc, st = in_thread(lambda: infer(lib, e, PROMPT, params(20), on_token))
    assert rc == tpthip.ERR_CANCELLED
    assert [t for t, d in events[:4]] == ref[:4] and all(d == 0 for _, d in events[:4])
    assert events[4:] == [(0, 1)]  # exactly one done event after the cancel
    assert st.generated == 3
    # the cancelled token was not fed: the next turn reuses the prompt + 3 generated tokens
    out = C.c_size_t()
    turn2 = PROMPT + ref[:3] + [5]
    ids = (C.c_uint32 * len(turn2))(*turn2)
    assert lib.tpt_engine_cached_prefix(e, ids, len(turn2), C.byref(out)) == 0
    assert out.value == len(PROMPT) + 3


def test_ffi_cancel_message_on_calling_thread(engine_h):
    lib, e = engine_h

    def body():
        assert lib.tpt_engine_reset_cache(e) == 0
        rc, _ = infer(lib, e, PROMPT, params(5), lambda tok, done: 1)
        return rc, lib.tpt_last_error()
    rc, msg = in_thread(body)
    assert rc == tpthip.ERR_CANCELLED and b"inference cancelled" in msg


def test_ffi_unload_then_state_error(engine_h, tiny_gguf):
    lib, e = engine_h
    assert lib.tpt_engine_unload(e) == 0
    assert lib.tpt_engine_is_loaded(e) == 0
    rc, _ = infer(lib, e, PROMPT, params(4), lambda tok, done: 0)
    assert rc == tpthip.ERR_STATE
    info = tpthip._ModelInfoC()
    assert lib.tpt_engine_model_info(e, C.byref(info)) == tpthip.ERR_STATE
    # and the engine loads again afterwards
    assert lib.tpt_engine_load(e, tiny_gguf.encode(), tpthip.PROGRESS_FN(), None, C.byref(info)) == 0
    assert lib.tpt_engine_is_loaded(e) == 1
