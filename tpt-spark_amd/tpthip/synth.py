"""Seeded synthetic workloads (libtptsynth.so): random-init Llama GGUF files and k-quant
quantization of arrays.  Presets name the model shapes the benchmarks are quoted on."""
import ctypes as C
import os

import numpy as np

from . import TYPE_F32, TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_0, BLOCK, TYPE_SIZE

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libtptsynth.so")
_lib = None


class SynthCfg(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layers", "embed", "n_heads", "n_kv_heads", "ffn", "vocab",
                                       "context_length")] + \
               [("rope_base", C.c_float), ("rms_eps", C.c_float), ("init_std", C.c_float)] + \
               [(n, C.c_int) for n in ("type_matrix", "type_embd", "type_out")] + \
               [("eos_token_id", C.c_uint32), ("type_more_bits", C.c_int)]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build with `make -C tpt-spark_amd/csrc`")
        L = C.CDLL(LIB_PATH)
        L.tpt_synth_quantize.argtypes = [C.c_int, C.c_void_p, C.c_int64, C.c_void_p]
        L.tpt_synth_normal.argtypes = [C.c_uint64, C.c_char_p, C.c_int64, C.c_int64, C.c_float,
                                       C.c_void_p]
        L.tpt_synth_write_llama.argtypes = [C.c_char_p, C.c_void_p, C.c_uint64, C.c_int]
        _lib = L
    return _lib


# Llama-3 shapes (Q4_K_M: token_embd / output Q6_K, other matrices Q4_K, norms F32 = 1.0)
LLAMA_8B = dict(n_layers=32, embed=4096, n_heads=32, n_kv_heads=8, ffn=14336, vocab=128256,
                context_length=8192, rope_base=500000.0, rms_eps=1e-5)
LLAMA_1B = dict(n_layers=16, embed=2048, n_heads=32, n_kv_heads=8, ffn=8192, vocab=128256,
                context_length=8192, rope_base=500000.0, rms_eps=1e-5)
TINY = dict(n_layers=2, embed=256, n_heads=4, n_kv_heads=2, ffn=512, vocab=1024,
            context_length=512, rope_base=500000.0, rms_eps=1e-5)


def write_llama(path, cfg, seed=0, nthreads=0, init_std=0.02, type_matrix=TYPE_Q4_K,
                type_embd=TYPE_Q6_K, type_out=TYPE_Q6_K, type_more_bits=0):
    """type_more_bits (e.g. TYPE_Q6_K): attn_v and ffn_down of the layers llama.cpp's Q4_K_M
    recipe gives more bits get that type, as in a real Q4_K_M file."""
    c = SynthCfg(cfg["n_layers"], cfg["embed"], cfg["n_heads"], cfg["n_kv_heads"], cfg["ffn"],
                 cfg["vocab"], cfg["context_length"], cfg["rope_base"], cfg["rms_eps"], init_std,
                 type_matrix, type_embd, type_out, cfg.get("eos_token_id", 0), type_more_bits)
    rc = lib().tpt_synth_write_llama(path.encode(), C.byref(c), seed, nthreads)
    if rc:
        raise RuntimeError(f"tpt_synth_write_llama({path}) failed: {rc}")
    return path


def quantize(qtype, x):
    x = np.ascontiguousarray(x, np.float32).ravel()
    assert x.size % BLOCK[qtype] == 0
    out = np.zeros(x.size // BLOCK[qtype] * TYPE_SIZE[qtype], np.uint8)
    rc = lib().tpt_synth_quantize(qtype, x.ctypes.data_as(C.c_void_p), x.size,
                                  out.ctypes.data_as(C.c_void_p))
    if rc:
        raise RuntimeError(f"quantize failed: {rc}")
    return out


def normal(seed, name, n, std=1.0, i0=0):
    out = np.empty(n, np.float32)
    lib().tpt_synth_normal(seed, name.encode(), i0, n, std, out.ctypes.data_as(C.c_void_p))
    return out


def random_weights(qtype, n_rows, k, seed, name="w", std=0.02):
    """N(0, std) weights [n_rows, k] quantized to qtype (raw GGUF blocks, rows contiguous)."""
    return quantize(qtype, normal(seed, name, n_rows * k, std))
