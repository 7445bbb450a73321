"""Python bindings of libtpthip (ctypes over the C ABI in include/tpthip.h).

This is the host-side mirror of the reference's engine surface for tests and benchmarks:
`HipEngine` follows `trait LlmEngine` (src-tauri/src/engine/mod.rs:62-82) with the same
parameter, event and info types (mod.rs:26-92); `Model` and `Context` expose the model-level
and op-level entry points.  Every call goes to the native library; there is no fallback path:
a missing library raises at import of the first call.
"""
import ctypes as C
import os
import weakref
from dataclasses import dataclass, field
from typing import Callable, List, Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))

TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K = 0, 1, 2, 8, 12, 13, 14
BLOCK = {TYPE_F32: 1, TYPE_F16: 1, TYPE_Q4_0: 32, TYPE_Q8_0: 32, TYPE_Q4_K: 256, TYPE_Q5_K: 256,
         TYPE_Q6_K: 256}
TYPE_SIZE = {TYPE_F32: 4, TYPE_F16: 2, TYPE_Q4_0: 18, TYPE_Q8_0: 34, TYPE_Q4_K: 144, TYPE_Q5_K: 176,
             TYPE_Q6_K: 210}
ACT_Q8, ACT_F32, ACT_F16 = 0, 1, 2

ERR_INVALID, ERR_HIP, ERR_IO, ERR_FORMAT, ERR_UNSUPPORTED, ERR_CANCELLED, ERR_STATE, ERR_OOM = \
    -1, -2, -3, -4, -5, -6, -7, -8

LIB_PATH = os.path.join(_HERE, "libtpthip.so")
_lib = None

P, I32, I64, U32, U64, F32, SZ = (C.c_void_p, C.c_int, C.c_int64, C.c_uint32, C.c_uint64,
                                  C.c_float, C.c_size_t)
PROGRESS_FN = C.CFUNCTYPE(None, C.c_void_p, C.c_uint32, C.c_uint32)
TOKEN_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint32, C.c_int)


class ModelDesc(C.Structure):
    _fields_ = [("architecture", C.c_char * 32)] + \
        [(n, C.c_int) for n in ("n_layers", "n_heads", "n_kv_heads", "head_dim", "embed", "ffn",
                                "vocab", "context_length", "max_ctx", "kv_type")] + \
        [("rms_eps", C.c_float), ("rope_base", C.c_float), ("rope_scale", C.c_float),
         ("weight_bytes", C.c_uint64), ("decode_bytes_per_token", C.c_uint64)] + \
        [(n, C.c_int) for n in ("type_q", "type_k", "type_v", "type_o", "type_gate", "type_up",
                                "type_down", "type_embd", "type_out")]


class _ModelInfoC(C.Structure):
    _fields_ = [("name", C.c_char * 256), ("path", C.c_char * 1024), ("size_bytes", C.c_uint64),
                ("backend", C.c_char * 64)]


class _InferParamsC(C.Structure):
    _fields_ = [("max_tokens", C.c_uint32), ("temperature", C.c_float), ("top_p", C.c_float),
                ("repeat_penalty", C.c_float), ("eos_token_id", C.c_int64), ("seed", C.c_uint64)]


class InferStats(C.Structure):
    _fields_ = [("prompt_tokens", C.c_uint32), ("cached_prefix", C.c_uint32),
                ("generated", C.c_uint32), ("prefill_ms", C.c_double), ("decode_ms", C.c_double),
                ("ttft_ms", C.c_double)]


EXPORTS = {
    "tpt_last_error": ([], C.c_char_p),
    "tpt_version": ([], I32),
    "tpt_ctx_create": ([I32, P], I32),
    "tpt_ctx_destroy": ([P], I32),
    "tpt_ctx_synchronize": ([P], I32),
    "tpt_ctx_device_info": ([P, P, C.c_char_p, I32], I32),
    "tpt_malloc": ([P, SZ, P], I32),
    "tpt_free": ([P, P], I32),
    "tpt_memcpy_h2d": ([P, P, P, SZ], I32),
    "tpt_memcpy_d2h": ([P, P, P, SZ], I32),
    "tpt_memset": ([P, P, I32, SZ], I32),
    "tpt_dequant": ([P, I32, P, P, I64], I32),
    "tpt_gemv": ([P, I32, P, P, P, I32, I32, I32], I32),
    "tpt_gemv_rmsnorm": ([P, I32, P, P, P, F32, P, I32, I32], I32),
    "tpt_swiglu": ([P, P, P, P, I32], I32),
    "tpt_rmsnorm": ([P, P, P, P, I32, F32], I32),
    "tpt_rope": ([P, P, I32, I32, I32, P, P], I32),
    "tpt_attn_decode": ([P, P, P, P, I32, P, I32, I32, I32, I32, I32, I32], I32),
    "tpt_attn_decode_noalloc": ([P, P, P, P, I32, P, I32, I32, I32, I32, I32, I32], I32),
    "tpt_argmax": ([P, P, I64, P], I32),
    "tpt_model_load": ([P, C.c_char_p, I32, I32, PROGRESS_FN, P, P], I32),
    "tpt_model_describe": ([P, P], I32),
    "tpt_model_inspect": ([C.c_char_p, P], I32),
    "tpt_model_destroy": ([P], I32),
    "tpt_model_prefill": ([P, P, I32, I32, P, P], I32),
    "tpt_model_decode_step": ([P, U32, I32, P, P], I32),
    "tpt_model_decode_greedy": ([P, U32, I32, I32, I64, P], I32),
    "tpt_model_hidden": ([P, P], I32),
    "tpt_model_run_layers": ([P, P, I32, I32, I32, I32, I32, P], I32),
    "tpt_model_kv_read": ([P, I32, P, P], I32),
    "tpt_model_set_decode_path": ([P, I32], I32),
    "tpt_model_get_decode_path": ([P, P], I32),
    "tpt_engine_create": ([I32, P], I32),
    "tpt_engine_set_kv_type": ([P, I32], I32),
    "tpt_engine_destroy": ([P], I32),
    "tpt_engine_load": ([P, C.c_char_p, PROGRESS_FN, P, P], I32),
    "tpt_engine_unload": ([P], I32),
    "tpt_engine_is_loaded": ([P], I32),
    "tpt_engine_model_info": ([P, P], I32),
    "tpt_engine_infer": ([P, P, P, SZ, TOKEN_FN, P, P], I32),
    "tpt_engine_cached_prefix": ([P, P, SZ, P], I32),
    "tpt_engine_reset_cache": ([P], I32),
    "tpt_common_prefix_len": ([P, SZ, P, SZ], SZ),
    "tpt_bench_gemv": ([P, I32, P, I32, P, P, I32, I32, I32, P], I32),
    "tpt_attn_prefill": ([P, P, P, P, I32, P, I32, I32, I32, I32, I32, I32, I32], I32),
    "tpt_bench_attn_prefill": ([P, P, P, P, I32, P, I32, I32, I32, I32, I32, I32, I32, P], I32),
    "tpt_bench_attn": ([P, P, P, P, I32, I32, P, I32, I32, I32, I32, I32, I32, I32, P], I32),
    "tpt_bench_copy": ([P, P, P, SZ, I32, P], I32),
    "tpt_gemm": ([P, I32, P, P, P, I32, I32, I32, I32], I32),
    "tpt_bench_gemm": ([P, I32, P, P, P, I32, I32, I32, I32, I32, P], I32),
}


def lib():
    """Load libtpthip.so (fails loudly when it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C tpt-spark_amd/csrc` "
                               "or __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        for name, (args, res) in EXPORTS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


class TptError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def check(rc):
    if rc < 0:
        raise TptError(rc, lib().tpt_last_error().decode(errors="replace"))
    return rc


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p)


def common_prefix_len(cached, new):
    """KvCache::common_prefix_len (wgpu_kvcache.rs:63-69); host-only, needs no GPU."""
    a = np.ascontiguousarray(cached, np.uint32)
    b = np.ascontiguousarray(new, np.uint32)
    return int(lib().tpt_common_prefix_len(_ptr(a), a.size, _ptr(b), b.size))


def row_bytes(qtype, k):
    return k // BLOCK[qtype] * TYPE_SIZE[qtype]


class DeviceBuffer:
    """A device allocation owned by a Context."""

    def __init__(self, ctx, nbytes):
        self.ctx, self.nbytes, self.ptr = ctx, int(nbytes), None
        p = C.c_void_p()
        check(lib().tpt_malloc(ctx.h, self.nbytes, C.byref(p)))
        self.ptr = p.value
        ctx._children.add(self)

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes, "upload larger than the buffer"
        check(lib().tpt_memcpy_h2d(self.ctx.h, self.ptr, _ptr(arr), arr.nbytes))
        return self

    def download(self, dtype, count=None):
        dtype = np.dtype(dtype)
        count = self.nbytes // dtype.itemsize if count is None else count
        out = np.empty(count, dtype)
        check(lib().tpt_memcpy_d2h(self.ctx.h, _ptr(out), self.ptr, out.nbytes))
        return out

    def fill(self, value=0):
        check(lib().tpt_memset(self.ctx.h, self.ptr, value, self.nbytes))
        return self

    def free(self):
        if self.ptr and self.ctx.h:
            lib().tpt_free(self.ctx.h, self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Context:
    """One device and one HIP stream (tpt_ctx)."""

    def __init__(self, device=0):
        self.h = None
        self._children = weakref.WeakSet()  # buffers and models, released before the context
        h = C.c_void_p()
        check(lib().tpt_ctx_create(device, C.byref(h)))
        self.h = h.value
        n = C.c_int()
        name = C.create_string_buffer(256)
        check(lib().tpt_ctx_device_info(self.h, C.byref(n), name, 256))
        self.n_cu, self.name = n.value, name.value.decode()

    def close(self):
        if self.h:
            for c in list(self._children):
                c.close() if isinstance(c, Model) else c.free()
            lib().tpt_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def synchronize(self):
        check(lib().tpt_ctx_synchronize(self.h))

    def alloc(self, nbytes):
        return DeviceBuffer(self, nbytes)

    def to_device(self, arr):
        arr = np.ascontiguousarray(arr)
        return DeviceBuffer(self, max(arr.nbytes, 1)).upload(arr)

    # ---- ops (device buffers in, numpy out) ----
    def dequant(self, qtype, wbuf, n):
        y = self.alloc(n * 4)
        check(lib().tpt_dequant(self.h, qtype, wbuf.ptr, y.ptr, n))
        return y.download(np.float32, n)

    def gemv(self, qtype, wbuf, xbuf, K, N, act=ACT_Q8, ybuf=None):
        y = ybuf or self.alloc(N * 4)
        check(lib().tpt_gemv(self.h, qtype, wbuf.ptr, xbuf.ptr, y.ptr, K, N, act))
        return y if ybuf else y.download(np.float32, N)

    def gemv_rmsnorm(self, qtype, wbuf, xbuf, normbuf, eps, K, N):
        y = self.alloc(N * 4)
        check(lib().tpt_gemv_rmsnorm(self.h, qtype, wbuf.ptr, xbuf.ptr, normbuf.ptr, eps, y.ptr, K, N))
        return y.download(np.float32, N)

    def rmsnorm(self, xbuf, wbuf, n, eps):
        y = self.alloc(n * 4)
        check(lib().tpt_rmsnorm(self.h, xbuf.ptr, wbuf.ptr, y.ptr, n, eps))
        return y.download(np.float32, n)

    def swiglu(self, gbuf, ubuf, n):
        y = self.alloc(n * 4)
        check(lib().tpt_swiglu(self.h, gbuf.ptr, ubuf.ptr, y.ptr, n))
        return y.download(np.float32, n)

    def rope(self, xbuf, n_heads, hd, pos, cosbuf, sinbuf):
        check(lib().tpt_rope(self.h, xbuf.ptr, n_heads, hd, pos, cosbuf.ptr, sinbuf.ptr))
        return xbuf.download(np.float32, n_heads * hd)

    def attn_decode(self, qbuf, kbuf, vbuf, nq, nkv, hd, L, L_stride, n_chunks=0,
                    kv_type=TYPE_F16):
        o = self.alloc(nq * hd * 4)
        check(lib().tpt_attn_decode(self.h, qbuf.ptr, kbuf.ptr, vbuf.ptr, kv_type, o.ptr, nq, nkv,
                                    hd, L, L_stride, n_chunks))
        return o.download(np.float32, nq * hd)

    ATTN_AUTO, ATTN_SPLITK, ATTN_MFMA = 0, 1, 2

    def attn_prefill(self, qbuf, kbuf, vbuf, nq, nkv, hd, L0, T, L_stride, form=0,
                     kv_type=TYPE_F16):
        """Causal attention of T query rows (row t at position L0 + t); returns o [T, nq*hd]."""
        o = self.alloc(T * nq * hd * 4)
        check(lib().tpt_attn_prefill(self.h, qbuf.ptr, kbuf.ptr, vbuf.ptr, kv_type, o.ptr, nq, nkv,
                                     hd, L0, T, L_stride, form))
        return o.download(np.float32, T * nq * hd).reshape(T, nq * hd)

    def bench_attn(self, qbuf, kbufs, vbufs, obuf, nq, nkv, hd, L, L_stride, iters, n_chunks=0,
                   kv_type=TYPE_F16):
        """Event-timed back-to-back decode-attention launches, launch i over the caches
        kbufs[i % n] / vbufs[i % n]; returns ms."""
        ks = (C.c_void_p * len(kbufs))(*[b.ptr for b in kbufs])
        vs = (C.c_void_p * len(vbufs))(*[b.ptr for b in vbufs])
        if len(kbufs) != len(vbufs):
            raise ValueError("bench_attn: as many K caches as V caches")
        ms = C.c_float()
        check(lib().tpt_bench_attn(self.h, qbuf.ptr, ks, vs, len(kbufs), kv_type, obuf.ptr, nq, nkv,
                                   hd, L, L_stride, n_chunks, iters, C.byref(ms)))
        return ms.value

    def bench_attn_prefill(self, qbuf, kbuf, vbuf, obuf, nq, nkv, hd, L0, T, L_stride, iters,
                           kv_type=TYPE_F16):
        """Event-timed back-to-back launches of the matrix-core causal attention; returns ms."""
        ms = C.c_float()
        check(lib().tpt_bench_attn_prefill(self.h, qbuf.ptr, kbuf.ptr, vbuf.ptr, kv_type, obuf.ptr,
                                           nq, nkv, hd, L0, T, L_stride, iters, C.byref(ms)))
        return ms.value

    def bench_gemv(self, qtype, wbufs, xbuf, ybuf, K, N, iters):
        """Event-timed back-to-back GEMV launches over rotating weight copies; returns ms."""
        arr = (C.c_void_p * len(wbufs))(*[w.ptr for w in wbufs])
        ms = C.c_float()
        check(lib().tpt_bench_gemv(self.h, qtype, arr, len(wbufs), xbuf.ptr, ybuf.ptr, K, N, iters,
                                   C.byref(ms)))
        return ms.value

    def gemm(self, qtype, wbuf, xbuf, M, K, N, act=ACT_Q8):
        """Prefill GEMM Y[M,N] = X[M,K] . W[N,K]^T (X fp32 rows on the device)."""
        y = self.alloc(M * N * 4)
        check(lib().tpt_gemm(self.h, qtype, wbuf.ptr, xbuf.ptr, y.ptr, M, K, N, act))
        return y.download(np.float32, M * N).reshape(M, N)

    def bench_gemm(self, qtype, wbuf, xbuf, ybuf, M, K, N, iters, act=ACT_Q8):
        """Sum of dispatch-stamped event intervals over iters GEMM launches; returns ms."""
        ms = C.c_float()
        check(lib().tpt_bench_gemm(self.h, qtype, wbuf.ptr, xbuf.ptr, ybuf.ptr, M, K, N, act, iters,
                                   C.byref(ms)))
        return ms.value

    def bench_copy(self, dst, src, nbytes, iters):
        ms = C.c_float()
        check(lib().tpt_bench_copy(self.h, dst.ptr, src.ptr, nbytes, iters, C.byref(ms)))
        return ms.value

    def argmax(self, buf, n):
        out = C.c_uint32()
        check(lib().tpt_argmax(self.h, buf.ptr, n, C.byref(out)))
        return out.value


def inspect_gguf(path):
    """tpt_model_inspect: the validated metadata of a GGUF, host only (no device needed)."""
    d = ModelDesc()
    check(lib().tpt_model_inspect(path.encode(), C.byref(d)))
    out = {n: getattr(d, n) for n, _ in ModelDesc._fields_}
    out["architecture"] = d.architecture.decode()
    return out


class Model:
    """tpt_model: a GGUF resident in HBM with its KV cache (fp16, or f32 like candle's)."""

    def __init__(self, ctx, path, max_ctx=0, on_progress=None, kv_type=TYPE_F16):
        self.ctx, self.h = ctx, None
        self._cb = PROGRESS_FN(lambda u, d, t: on_progress(d, t)) if on_progress else PROGRESS_FN()
        h = C.c_void_p()
        check(lib().tpt_model_load(ctx.h, path.encode(), max_ctx, kv_type, self._cb, None,
                                   C.byref(h)))
        self.h = h.value
        ctx._children.add(self)
        d = ModelDesc()
        check(lib().tpt_model_describe(self.h, C.byref(d)))
        self.desc = {n: getattr(d, n) for n, _ in ModelDesc._fields_}
        self.desc["architecture"] = d.architecture.decode()

    def close(self):
        if self.h and self.ctx.h:
            lib().tpt_model_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def prefill(self, ids, pos0=0, logits=False):
        ids = np.ascontiguousarray(ids, np.uint32)
        nxt = C.c_uint32()
        out = np.empty(self.desc["vocab"], np.float32) if logits else None
        check(lib().tpt_model_prefill(self.h, _ptr(ids), ids.size, pos0, C.byref(nxt),
                                      _ptr(out) if logits else None))
        return (nxt.value, out) if logits else nxt.value

    def decode_step(self, tok, pos, logits=False):
        nxt = C.c_uint32()
        out = np.empty(self.desc["vocab"], np.float32) if logits else None
        check(lib().tpt_model_decode_step(self.h, tok, pos, C.byref(nxt), _ptr(out) if logits else None))
        return (nxt.value, out) if logits else nxt.value

    def decode_greedy(self, first, pos0, n_steps, stop_token=-1):
        out = np.zeros(max(n_steps, 1), np.uint32)
        n = check(lib().tpt_model_decode_greedy(self.h, first, pos0, n_steps, stop_token, _ptr(out)))
        return out[:n].tolist()

    def hidden(self):
        out = np.empty(self.desc["embed"], np.float32)
        check(lib().tpt_model_hidden(self.h, _ptr(out)))
        return out

    PATH_BATCHED, PATH_STEPS = 0, 1
    DECODE_KERNELS, DECODE_PERSISTENT = 0, 1

    @property
    def decode_path(self):
        """DECODE_KERNELS: one launch per fused op, the only decode form (DECODE_PERSISTENT,
        a single-launch step, was removed: setting it raises TPT_ERR_UNSUPPORTED)."""
        v = C.c_int()
        check(lib().tpt_model_get_decode_path(self.h, C.byref(v)))
        return v.value

    @decode_path.setter
    def decode_path(self, path):
        check(lib().tpt_model_set_decode_path(self.h, path))

    def kv(self, layer):
        """Layer's K and V caches as float32 arrays [n_kv_heads, max_ctx, head_dim]."""
        d = self.desc
        shape = (d["n_kv_heads"], d["max_ctx"], d["head_dim"])
        dt = np.float32 if d["kv_type"] == TYPE_F32 else np.float16
        k, v = np.empty(shape, dt), np.empty(shape, dt)
        check(lib().tpt_model_kv_read(self.h, layer, _ptr(k), _ptr(v)))
        return k.astype(np.float32), v.astype(np.float32)

    def run_layers(self, x, pos0, l0, l1, path=0):
        """Decoder layers [l0, l1) on residual rows x [n, embed] at positions pos0 ..; returns
        the output rows.  path 0: batched prefill kernels, 1: decode-step kernels."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.desc["embed"])
        out = np.empty_like(x)
        check(lib().tpt_model_run_layers(self.h, _ptr(x), x.shape[0], pos0, l0, l1, path, _ptr(out)))
        return out


# ---------------------------------------------------------------- LlmEngine mirror

@dataclass
class InferenceParams:
    """InferenceParams (mod.rs:35-59).  The tokenizer is bypassed on this path, so `prompt` is
    the token id list; `eos_token_id` is what find_eos_token (candle_engine.rs:76-83) would
    return for the model's tokenizer (None: no EOS stop).  `system_prompt` is carried for
    interface parity; like both reference engines, infer() does not read it."""
    prompt: List[int] = field(default_factory=list)
    system_prompt: Optional[str] = None
    max_tokens: int = 512
    temperature: float = 0.7
    top_p: float = 0.9
    repeat_penalty: float = 1.1
    eos_token_id: Optional[int] = None
    seed: int = 42


@dataclass
class TokenEvent:
    """TokenEvent (mod.rs:27-32) plus the raw id."""
    token: str
    done: bool
    token_id: int = 0


@dataclass
class ModelInfo:
    """ModelInfo (mod.rs:85-92)."""
    name: str
    path: str
    size_bytes: int
    backend: str


def greedy_params(prompt, max_tokens, eos_token_id=None):
    """run_benchmark's greedy parameter set (commands.rs:518-525)."""
    return InferenceParams(prompt=list(prompt), max_tokens=max_tokens, temperature=0.0, top_p=1.0,
                           repeat_penalty=1.0, eos_token_id=eos_token_id)


class HipEngine:
    """engine-hip behind the LlmEngine interface: load / unload / is_loaded / model_info /
    infer.  `detokenize(id) -> str` fills TokenEvent.token (default: the decimal id)."""

    def __init__(self, device=0, detokenize: Optional[Callable[[int], str]] = None,
                 kv_type=TYPE_F16):
        h = C.c_void_p()
        check(lib().tpt_engine_create(device, C.byref(h)))
        self.h = h.value
        check(lib().tpt_engine_set_kv_type(self.h, kv_type))
        self.detokenize = detokenize or (lambda i: str(i))
        self.last_stats = None

    def close(self):
        if self.h:
            lib().tpt_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def load(self, model_path, on_progress=None) -> ModelInfo:
        cb = PROGRESS_FN(lambda u, d, t: on_progress(d, t)) if on_progress else PROGRESS_FN()
        info = _ModelInfoC()
        check(lib().tpt_engine_load(self.h, model_path.encode(), cb, None, C.byref(info)))
        return self._info(info)

    def unload(self):
        check(lib().tpt_engine_unload(self.h))

    def is_loaded(self) -> bool:
        return bool(lib().tpt_engine_is_loaded(self.h))

    def model_info(self) -> Optional[ModelInfo]:
        if not self.is_loaded():
            return None
        info = _ModelInfoC()
        check(lib().tpt_engine_model_info(self.h, C.byref(info)))
        return self._info(info)

    @staticmethod
    def _info(i):
        return ModelInfo(i.name.decode(), i.path.decode(), int(i.size_bytes), i.backend.decode())

    def cached_prefix_len(self, tokens):
        t = np.ascontiguousarray(tokens, np.uint32)
        out = C.c_size_t()
        check(lib().tpt_engine_cached_prefix(self.h, _ptr(t), t.size, C.byref(out)))
        return out.value

    def reset_cache(self):
        check(lib().tpt_engine_reset_cache(self.h))

    def infer(self, params: InferenceParams, on_token: Callable[[TokenEvent], None]):
        """Runs one generation; on_token raising cancels (the exception propagates after the
        final done event, as an Err from the Rust callback would)."""
        cp = _InferParamsC(params.max_tokens, params.temperature, params.top_p,
                           params.repeat_penalty,
                           -1 if params.eos_token_id is None else params.eos_token_id, params.seed)
        prompt = np.ascontiguousarray(params.prompt, np.uint32)
        raised = []

        def cb(_u, tok, done):
            try:
                on_token(TokenEvent("" if done else self.detokenize(tok), bool(done), int(tok)))
                return 0
            except BaseException as e:  # noqa: BLE001 - handed back to the caller below
                raised.append(e)
                return 1

        fn = TOKEN_FN(cb)
        stats = InferStats()
        rc = lib().tpt_engine_infer(self.h, C.byref(cp), _ptr(prompt), prompt.size, fn, None,
                                    C.byref(stats))
        self.last_stats = stats
        if raised:
            raise raised[0]
        check(rc)
        return stats
