"""ctypes view of the CPU oracle (liboracle.so) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module,
and only as the checker (or as the timed CPU restatement).  The product path never does.
The C sources state which candle 0.8.4 routine each function restates and how each one is
pinned.
"""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K = 0, 1, 2, 8, 12, 13, 14, 15
BLOCK = {F32: 1, F16: 1, Q4_0: 32, Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256, Q8_K: 256}
TYPE_SIZE = {F32: 4, F16: 2, Q4_0: 18, Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_K: 292}


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run `make -C oracle` (or __graft_entry__.build())")
        L = C.CDLL(path)
        P, I64, I32, F = C.c_void_p, C.c_int64, C.c_int, C.c_float
        L.orc_dequant.argtypes = [I32, P, P, I64]
        L.orc_quantize_q8k.argtypes = [P, I64, P]
        L.orc_quantize_q8_0.argtypes = [P, I64, P]
        L.orc_vec_dot.argtypes = [I32, I64, P, P]
        L.orc_vec_dot.restype = F
        L.orc_matmul.argtypes = [I32, I64, I64, I64, P, P, P, I32]
        L.orc_gemv_f64.argtypes = [I32, I64, I64, P, P, P]
        L.orc_rmsnorm.argtypes = [P, P, I64, F, P]
        L.orc_silu.argtypes = [F]
        L.orc_silu.restype = F
        L.orc_rope_tables.argtypes = [I32, F, I32, P, P]
        L.orc_rope_i.argtypes = [P, I32, I32, P, P]
        L.orc_attention.argtypes = [P, P, P, I32, I32, I32, I32, I32, P]
        L.orc_argmax.argtypes = [P, I64]
        L.orc_argmax.restype = C.c_uint32
        L.orc_repeat_penalty.argtypes = [P, I64, P, I64, F]
        L.orc_f32_to_fp16.argtypes = [F]
        L.orc_f32_to_fp16.restype = C.c_uint16
        L.orc_fp16_to_f32.argtypes = [C.c_uint16]
        L.orc_fp16_to_f32.restype = F
        L.orc_model_open.argtypes = [C.c_char_p, C.c_char_p, I32]
        L.orc_model_open.restype = P
        L.orc_model_close.argtypes = [P]
        L.orc_model_get_cfg.argtypes = [P, P]
        L.orc_model_reset.argtypes = [P, I32, I32]
        L.orc_model_forward.argtypes = [P, P, I32, I32, P, I32]
        L.orc_model_last_hidden.argtypes = [P, P]
        L.orc_model_forward_trace.argtypes = [P, P, I32, I32, P, I32, P]
        L.orc_model_set_attn_fma.argtypes = [P, I32]
        L.orc_model_kv.argtypes = [P, I32, P, P]
        L.orc_model_run_layers.argtypes = [P, P, I32, I32, I32, I32, P, I32]
        L.orc_set_dot_block_order.argtypes = [I32]
        L.orc_set_rms_order.argtypes = [I32]
        L.orc_model_prime_cache.argtypes = [P, I32, C.c_uint64]
        L.orc_model_tensor.argtypes = [P, C.c_char_p, P, P, P]
        L.orc_model_tensor.restype = P
        _LIB = L
    return _LIB


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def row_bytes(qtype, k):
    return k // BLOCK[qtype] * TYPE_SIZE[qtype]


def dequant(qtype, raw, n):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(n, np.float32)
    assert lib().orc_dequant(qtype, _p(raw), _p(out), n) == 0
    return out


def quantize_q8k(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.size // 256 * 292, np.uint8)
    assert lib().orc_quantize_q8k(_p(x), x.size, _p(out)) == 0
    return out


def quantize_q8_0(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.size // 32 * 34, np.uint8)
    assert lib().orc_quantize_q8_0(_p(x), x.size, _p(out)) == 0
    return out


def vec_dot(qtype, k, w_row, act_q):
    w_row = np.ascontiguousarray(w_row, np.uint8)
    act_q = np.ascontiguousarray(act_q, np.uint8)
    return float(lib().orc_vec_dot(qtype, k, _p(w_row), _p(act_q)))


def matmul(qtype, x, w, n, nthreads=0):
    """candle k_quants::matmul: x [M,K] f32, w raw blocks [N rows] -> [M,N]"""
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    m, k = x.shape
    w = np.ascontiguousarray(w, np.uint8)
    out = np.empty((m, n), np.float32)
    assert lib().orc_matmul(qtype, m, k, n, _p(x), _p(w), _p(out), nthreads) == 0
    return out


def gemv_f64(qtype, w, x, n):
    x = np.ascontiguousarray(x, np.float64)
    w = np.ascontiguousarray(w, np.uint8)
    y = np.empty(n, np.float64)
    assert lib().orc_gemv_f64(qtype, x.size, n, _p(w), _p(x), _p(y)) == 0
    return y


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    y = np.empty_like(x)
    lib().orc_rmsnorm(_p(x), _p(w), x.size, eps, _p(y))
    return y


def silu(v):
    return float(lib().orc_silu(float(v)))


def rope_tables(rope_dim, base, n_pos):
    c = np.empty((n_pos, rope_dim // 2), np.float32)
    s = np.empty_like(c)
    lib().orc_rope_tables(rope_dim, base, n_pos, _p(c), _p(s))
    return c, s


def rope_i(x, n_heads, hd, cos_row, sin_row):
    x = np.array(x, np.float32, copy=True)
    cos_row = np.ascontiguousarray(cos_row, np.float32)
    sin_row = np.ascontiguousarray(sin_row, np.float32)
    lib().orc_rope_i(_p(x), n_heads, hd, _p(cos_row), _p(sin_row))
    return x


def attention(q, kc, vc, nq, nkv, hd, L):
    """q [nq*hd]; kc/vc [nkv, L_stride, hd] f32 -> o [nq*hd]"""
    q = np.ascontiguousarray(q, np.float32)
    kc = np.ascontiguousarray(kc, np.float32)
    vc = np.ascontiguousarray(vc, np.float32)
    o = np.empty(nq * hd, np.float32)
    lib().orc_attention(_p(q), _p(kc), _p(vc), nq, nkv, hd, L, kc.shape[1], _p(o))
    return o


def set_dot_block_order(on):
    """k-quant dot products in the block-reduced f32 order (a test instrument; off = candle's)."""
    lib().orc_set_dot_block_order(int(on))


def set_rms_order(on):
    """RMSNorm's sum of squares in a 16-run + pairwise-tree order (a test instrument; off =
    candle's sequential sum)."""
    lib().orc_set_rms_order(int(on))


def argmax(logits):
    logits = np.ascontiguousarray(logits, np.float32)
    return int(lib().orc_argmax(_p(logits), logits.size))


def repeat_penalty(logits, seen, penalty):
    logits = np.array(logits, np.float32, copy=True)
    seen = np.ascontiguousarray(seen, np.uint32)
    lib().orc_repeat_penalty(_p(logits), logits.size, _p(seen), seen.size, penalty)
    return logits


def f32_to_fp16_bits(v):
    return int(lib().orc_f32_to_fp16(float(v)))


def fp16_bits_to_f32(h):
    return float(lib().orc_fp16_to_f32(int(h)))


class _Cfg(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layers", "n_heads", "n_kv_heads", "head_dim", "embed",
                                       "ffn", "vocab", "rope_dim", "ctx_len")] + \
               [("eps", C.c_float), ("rope_base", C.c_float)]


class Model:
    """quantized_llama::ModelWeights restated over a GGUF file (mmapped, no copies)."""

    def __init__(self, path):
        err = C.create_string_buffer(256)
        self.h = lib().orc_model_open(path.encode(), err, 256)
        if not self.h:
            raise RuntimeError(err.value.decode())
        c = _Cfg()
        lib().orc_model_get_cfg(self.h, C.byref(c))
        self.cfg = {n: getattr(c, n) for n, _ in _Cfg._fields_}

    def set_attn_fma(self, on):
        """Attention dots as fused multiply-adds (the gemm crate's kernels on an FMA host)."""
        lib().orc_model_set_attn_fma(self.h, int(on))

    def reset(self, max_pos, kv_f16=False):
        assert lib().orc_model_reset(self.h, max_pos, int(kv_f16)) == 0
        self.max_pos = max_pos

    def forward(self, tokens, pos0, nthreads=0):
        toks = np.ascontiguousarray(tokens, np.uint32)
        logits = np.empty(self.cfg["vocab"], np.float32)
        rc = lib().orc_model_forward(self.h, _p(toks), toks.size, pos0, _p(logits), nthreads)
        if rc:
            raise RuntimeError(f"orc_model_forward rc={rc}")
        return logits

    def forward_trace(self, tokens, pos0, nthreads=0):
        """forward() that also returns the residual rows entering each layer and leaving the
        last: trace[l] is layer l's input [n, embed], trace[n_layers] the final rows."""
        toks = np.ascontiguousarray(tokens, np.uint32)
        logits = np.empty(self.cfg["vocab"], np.float32)
        trace = np.empty((self.cfg["n_layers"] + 1, toks.size, self.cfg["embed"]), np.float32)
        rc = lib().orc_model_forward_trace(self.h, _p(toks), toks.size, pos0, _p(logits), nthreads,
                                           _p(trace))
        if rc:
            raise RuntimeError(f"orc_model_forward_trace rc={rc}")
        return logits, trace

    def run_layers(self, x, pos0, l0, l1, nthreads=0):
        """Decoder layers [l0, l1) on residual rows x [n, embed] at positions pos0 ..."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.cfg["embed"])
        out = np.empty_like(x)
        rc = lib().orc_model_run_layers(self.h, _p(x), x.shape[0], pos0, l0, l1, _p(out), nthreads)
        if rc:
            raise RuntimeError(f"orc_model_run_layers rc={rc}")
        return out

    def kv(self, layer):
        """Layer's K and V caches [n_kv_heads, max_pos, head_dim] (f32; fp16-rounded values in
        the fp16 mode)."""
        shape = (self.cfg["n_kv_heads"], self.max_pos, self.cfg["head_dim"])
        k, v = np.empty(shape, np.float32), np.empty(shape, np.float32)
        assert lib().orc_model_kv(self.h, layer, _p(k), _p(v)) == 0
        return k, v

    def prime_cache(self, n_pos, seed=1):
        """Fill K/V of positions [0, n_pos) with synthetic values (benchmark aid)."""
        assert lib().orc_model_prime_cache(self.h, n_pos, seed) == 0

    def last_hidden(self):
        out = np.empty(self.cfg["embed"], np.float32)
        lib().orc_model_last_hidden(self.h, _p(out))
        return out

    def tensor(self, name):
        t, n0, n1 = C.c_int(), C.c_int64(), C.c_int64()
        ptr = lib().orc_model_tensor(self.h, name.encode(), C.byref(t), C.byref(n0), C.byref(n1))
        if not ptr:
            raise KeyError(name)
        nbytes = row_bytes(t.value, n0.value) * n1.value
        buf = (C.c_uint8 * nbytes).from_address(ptr)
        return t.value, n0.value, n1.value, np.frombuffer(buf, np.uint8)

    def close(self):
        if self.h:
            lib().orc_model_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def greedy(self, prompt, n_gen, eos=None, max_pos=None, kv_f16=False, nthreads=0,
               return_logits=()):
        """candle_engine.rs:269-324 with greedy params (commands.rs:518-525): batched
        prefill, then one forward per generated token; returns (tokens, {step: logits}).
        step 0 is the prefill's last-position logits."""
        self.reset(max_pos or (len(prompt) + n_gen + 1), kv_f16)
        saved = {}
        logits = self.forward(prompt, 0, nthreads)
        if 0 in return_logits:
            saved[0] = logits.copy()
        out = []
        nxt = argmax(logits)
        pos = len(prompt)
        while True:
            if eos is not None and nxt == eos:
                break
            if len(out) >= n_gen:
                break
            out.append(nxt)
            logits = self.forward([nxt], pos, nthreads)
            if len(out) in return_logits:
                saved[len(out)] = logits.copy()
            nxt = argmax(logits)
            pos += 1
        return out, saved
