"""Op-level parity on the GPU: each HIP kernel through the C ABI against the CPU oracle.

Bars: dequantization bit-exact; GEMV within 1e-3 relative L2 of candle's Q8 integer path (the
integer sums are exact, so the measured gap is f32 block-accumulation order, ~1e-7); decode
attention within 1e-3 relative L2 of the f32 oracle over the same fp16 cache values.
"""
import json
import os
import struct

import numpy as np
import pytest

import oracle
import tpthip
from tpthip import synth, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0, TYPE_Q4_0, TYPE_F16

pytestmark = pytest.mark.gpu

QTYPES = [TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0, TYPE_Q4_0]
GEMV_TYPES = QTYPES + [TYPE_F16]  # F16: candle dequantizes, then an f32 matmul


def rel_l2(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


def random_blocks(qtype, nblocks, seed):
    """Every quant bit pattern, f16 scales spanning subnormal .. large."""
    rng = np.random.default_rng(seed)
    ts = tpthip.TYPE_SIZE[qtype]
    raw = rng.integers(0, 256, nblocks * ts, dtype=np.uint8).reshape(nblocks, ts)
    pool = np.array([0x0001, 0x03FF, 0x0400, 0x1000, 0x2400, 0x3C00, 0x5800, 0x7BFF, 0x8400, 0x9800],
                    np.uint16)
    h = rng.choice(pool, (nblocks, 2)).astype("<u2").view(np.uint8)
    if qtype in (TYPE_Q4_K, TYPE_Q5_K):
        raw[:, 0:4] = h.reshape(nblocks, 4)
    elif qtype == TYPE_Q6_K:
        raw[:, 208:210] = h[:, :2]
    else:
        raw[:, 0:2] = h[:, :2]
    return raw.reshape(-1)


@pytest.mark.parametrize("qtype", QTYPES)
def test_dequant_bit_exact(ctx, qtype):
    nb = 4096
    raw = random_blocks(qtype, nb, 17 + qtype)
    n = nb * tpthip.BLOCK[qtype]
    y = ctx.dequant(qtype, ctx.to_device(raw), n)
    ref = oracle.dequant(qtype, raw, n)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


def test_dequant_known_answer_blocks(ctx):
    gold = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kat_blocks.json")))
    g = gold["q4k"]
    blk = struct.pack("<HH", g["d_bits"], g["dmin_bits"]) + bytes(g["scales"]) + \
        bytes([(i % 16) | ((15 - i % 16) << 4) for i in range(128)])
    y = ctx.dequant(TYPE_Q4_K, ctx.to_device(np.frombuffer(blk, np.uint8)), 256)
    for k, v in g["expect"].items():
        assert y[int(k)] == v


def test_dequant_hand_blocks_q5k_q4_0(ctx):
    """The hand-worked Q5_K and Q4_0 blocks of the oracle's known-answer tests on the GPU
    (embedding rows and tpt_dequant go through this element decode)."""
    qs = bytes([(i % 16) | ((15 - i % 16) << 4) for i in range(128)])
    qh = bytes([0xFF if l % 2 else 0 for l in range(32)])
    q5 = struct.pack("<HH", 0x3C00, 0x3800) + bytes([1, 2, 3, 4, 0, 1, 2, 3, 0x21, 0x43, 0x65, 0x87]) + qh + qs
    y = ctx.dequant(TYPE_Q5_K, ctx.to_device(np.frombuffer(q5, np.uint8)), 256)
    assert [y[k] for k in (0, 1, 33, 34, 69, 167, 222, 255)] == [0.0, 17.0, 59.5, 25.5, 62.0, 70.0, 67.0, 108.0]
    q4 = struct.pack("<H", 0x3800) + bytes([j | ((15 - j) << 4) for j in range(16)])
    y = ctx.dequant(TYPE_Q4_0, ctx.to_device(np.frombuffer(q4, np.uint8)), 32)
    assert list(y[[0, 8, 15, 16, 20, 31]]) == [-4.0, 0.0, 3.5, 3.5, 1.5, -4.0]


def test_dequant_f16_every_finite_value(ctx):
    """Every finite f16 bit pattern (subnormals, both zeros, 65504) widened on the GPU equals
    numpy's float16 -> float32 conversion bit for bit (the embedding row and F16 GEMV decode)."""
    bits = np.arange(65536, dtype=np.uint16)
    bits = bits[(bits & 0x7C00) != 0x7C00]
    y = ctx.dequant(TYPE_F16, ctx.to_device(bits.view(np.uint8)), bits.size)
    np.testing.assert_array_equal(y.view(np.uint32), bits.view(np.float16).astype(np.float32).view(np.uint32))


GEMV_SHAPES = [(4096, 4096), (4096, 1024), (4096, 14336), (14336, 4096)]
SMALL_SHAPES = [(256, 64), (512, 37), (768, 130), (1024, 300), (2048, 1000), (8192, 520)]


def gemv_case(ctx, qtype, K, N, seed):
    w = synth.random_weights(qtype, N, K, seed=seed, name=f"w{K}x{N}")
    x = np.random.default_rng(seed).standard_normal(K).astype(np.float32)
    y = ctx.gemv(qtype, ctx.to_device(w), ctx.to_device(x), K, N)
    return w, x, y


@pytest.mark.parametrize("K,N", GEMV_SHAPES + SMALL_SHAPES)
@pytest.mark.parametrize("qtype", GEMV_TYPES)
def test_gemv_matches_candle_q8_path(ctx, qtype, K, N):
    w, x, y = gemv_case(ctx, qtype, K, N, seed=K * 7 + N)
    ref = oracle.matmul(qtype, x, w, N)[0]
    err = rel_l2(y, ref)
    assert err < 1e-3  # contract
    assert err < 1e-5, f"integer path should be exact up to f32 accumulation, got {err:.2e}"


@pytest.mark.parametrize("K,N", [(4096, 4096), (14336, 4096), (2048, 1000)])
@pytest.mark.parametrize("qtype", GEMV_TYPES)
def test_gemv_fp32_activations(ctx, qtype, K, N):
    w = synth.random_weights(qtype, N, K, seed=5, name="f32w")
    x = np.random.default_rng(6).standard_normal(K).astype(np.float32)
    y = ctx.gemv(qtype, ctx.to_device(w), ctx.to_device(x), K, N, act=tpthip.ACT_F32)
    ref = oracle.gemv_f64(qtype, w, x.astype(np.float64), N)
    assert rel_l2(y, ref) < 1e-5


@pytest.mark.parametrize("qtype", GEMV_TYPES)
def test_gemv_rmsnorm_prologue(ctx, qtype):
    K, N, eps = 4096, 2048, 1e-5
    w = synth.random_weights(qtype, N, K, seed=8, name="nw")
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(K) * 3).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    y = ctx.gemv_rmsnorm(qtype, ctx.to_device(w), ctx.to_device(x), ctx.to_device(nw), eps, K, N)
    ref = oracle.matmul(qtype, oracle.rmsnorm(x, nw, eps), w, N)[0]
    assert rel_l2(y, ref) < 1e-3


def test_gemv_linearity_full_size(ctx):
    """Size-independent property at the 8B down-projection shape: y(a x) = a y(x) for a power of
    two (Q8_K activation quantization is scale-equivariant for powers of two)."""
    K, N = 14336, 4096
    w = synth.random_weights(TYPE_Q4_K, N, K, seed=21, name="lin")
    x = np.random.default_rng(22).standard_normal(K).astype(np.float32)
    wd = ctx.to_device(w)
    y1 = ctx.gemv(TYPE_Q4_K, wd, ctx.to_device(x), K, N)
    y4 = ctx.gemv(TYPE_Q4_K, wd, ctx.to_device(4 * x), K, N)
    np.testing.assert_array_equal(4 * y1, y4)


def test_gemv_rejects_bad_shapes(ctx):
    w = ctx.alloc(1024)
    x = ctx.alloc(1024)
    with pytest.raises(tpthip.TptError) as e:
        ctx.gemv(TYPE_Q4_K, w, x, 100, 4)
    assert e.value.code == tpthip.ERR_INVALID
    with pytest.raises(tpthip.TptError) as e:
        ctx.gemv(tpthip.TYPE_F32, w, x, 256, 4)
    assert e.value.code == tpthip.ERR_UNSUPPORTED
    with pytest.raises(tpthip.TptError) as e:  # F16 activations in LDS: 4 K bytes
        ctx.gemv(TYPE_F16, w, x, 16384, 4)
    assert e.value.code == tpthip.ERR_UNSUPPORTED


def test_gemv_f16_exact_extremes(ctx):
    """F16 rows holding subnormals, +-65504 and zeros against one-hot and power-of-two
    activations: every product and sum is exact, so the GEMV equals the widened weights
    (a wrong run interleave, a swapped half or a bf16 reading changes these values)."""
    K, N = 1024, 64
    rng = np.random.default_rng(4)
    specials = np.array([0x0001, 0x03FF, 0x0400, 0x7BFF, 0xFBFF, 0x8000, 0x0000, 0x3C00, 0xBC01],
                        np.uint16)
    bits = rng.integers(0, 0x7C00, (N, K)).astype(np.uint16) | (rng.integers(0, 2, (N, K)) << 15).astype(np.uint16)
    bits[:, :specials.size] = specials
    wd = ctx.to_device(bits.view(np.uint8).reshape(-1))
    wf = bits.view(np.float16).astype(np.float32)
    for j in list(range(specials.size)) + [255, 256, 511, 777, K - 1]:
        x = np.zeros(K, np.float32)
        x[j] = 2.0 ** -3
        y = ctx.gemv(TYPE_F16, wd, ctx.to_device(x), K, N)
        np.testing.assert_array_equal(y, wf[:, j] * np.float32(2.0 ** -3))


def test_rmsnorm_op(ctx):
    n, eps = 4096, 1e-5
    rng = np.random.default_rng(3)
    x = rng.standard_normal(n).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    y = ctx.rmsnorm(ctx.to_device(x), ctx.to_device(w), n, eps)
    np.testing.assert_allclose(y, oracle.rmsnorm(x, w, eps), rtol=2e-6, atol=1e-7)


def test_rope_op(ctx):
    hd, heads, base = 128, 32, 500000.0
    c, s = oracle.rope_tables(hd, base, 64)
    x = np.random.default_rng(4).standard_normal(heads * hd).astype(np.float32)
    y = ctx.rope(ctx.to_device(x), heads, hd, 37, ctx.to_device(c), ctx.to_device(s))
    np.testing.assert_array_equal(y, oracle.rope_i(x, heads, hd, c[37], s[37]))


def attention_case(ctx, nq, nkv, hd, L, seed, kv_dtype=np.float16):
    """Decode-attention chain: x ~ N(0,1) -> RMSNorm (w = 1, eps 1e-5) -> q (no projection) ->
    RoPE at pos = L-1; cache K/V ~ N(0,1) stored fp16 (or f32), the newest K row RoPE'd at
    L-1; causal."""
    rng = np.random.default_rng(seed)
    base, eps = 500000.0, 1e-5
    cos_t, sin_t = oracle.rope_tables(hd, base, L)
    x = rng.standard_normal(nq * hd).astype(np.float32)
    k = rng.standard_normal((nkv, L, hd)).astype(kv_dtype)
    v = rng.standard_normal((nkv, L, hd)).astype(kv_dtype)
    knew = oracle.rope_i(rng.standard_normal(nkv * hd).astype(np.float32), nkv, hd,
                         cos_t[L - 1], sin_t[L - 1]).reshape(nkv, hd)
    k[:, L - 1] = knew.astype(kv_dtype)
    ones = np.ones(nq * hd, np.float32)
    # GPU: rmsnorm -> rope -> attention
    xd = ctx.to_device(x)
    qn = ctx.alloc(nq * hd * 4)
    from tpthip import lib, check
    check(lib().tpt_rmsnorm(ctx.h, xd.ptr, ctx.to_device(ones).ptr, qn.ptr, nq * hd, eps))
    ctx.rope(qn, nq, hd, L - 1, ctx.to_device(cos_t), ctx.to_device(sin_t))
    kvt = tpthip.TYPE_F32 if kv_dtype == np.float32 else tpthip.TYPE_F16
    o = ctx.attn_decode(qn, ctx.to_device(k), ctx.to_device(v), nq, nkv, hd, L, L, kv_type=kvt)
    # oracle
    q = oracle.rope_i(oracle.rmsnorm(x, ones, eps), nq, hd, cos_t[L - 1], sin_t[L - 1])
    ref = oracle.attention(q, k.astype(np.float32), v.astype(np.float32), nq, nkv, hd, L)
    return o, ref


@pytest.mark.parametrize("L", [512, 4096, 16384, 32768])
def test_attention_gqa_hd128(ctx, L):
    o, ref = attention_case(ctx, 32, 8, 128, L, seed=L)
    assert rel_l2(o, ref) < 1e-3
    assert rel_l2(o, ref) < 1e-5


@pytest.mark.parametrize("L", [1, 2, 17, 512, 4096, 16384, 32768])
def test_attention_mha_hd96(ctx, L):
    o, ref = attention_case(ctx, 32, 32, 96, L, seed=L + 1)
    assert rel_l2(o, ref) < 1e-5


@pytest.mark.parametrize("nq,nkv,hd,L", [(32, 8, 128, 4096), (32, 32, 96, 777), (32, 8, 64, 2048),
                                         (16, 2, 64, 1), (32, 4, 128, 32768)])
def test_attention_f32_cache(ctx, nq, nkv, hd, L):
    """candle's f32 cache layout through the same split-K kernel."""
    o, ref = attention_case(ctx, nq, nkv, hd, L, seed=L + hd, kv_dtype=np.float32)
    assert rel_l2(o, ref) < 1e-5


def test_attention_single_position_is_v(ctx):
    """Closed form: with one cached position softmax is 1, so o = v of the head's kv group."""
    nq, nkv, hd = 32, 8, 128
    rng = np.random.default_rng(3)
    q = rng.standard_normal(nq * hd).astype(np.float32)
    k = rng.standard_normal((nkv, 16, hd)).astype(np.float16)
    v = rng.standard_normal((nkv, 16, hd)).astype(np.float16)
    o = ctx.attn_decode(ctx.to_device(q), ctx.to_device(k), ctx.to_device(v), nq, nkv, hd, 1, 16)
    want = np.repeat(v[:, 0, :].astype(np.float32), nq // nkv, axis=0).reshape(-1)
    np.testing.assert_array_equal(o, want)


def test_attention_uniform_scores_is_mean(ctx):
    """Closed form: identical K rows give uniform softmax weights, so o = mean over V rows."""
    nq, nkv, hd, L = 8, 2, 64, 300
    rng = np.random.default_rng(4)
    q = rng.standard_normal(nq * hd).astype(np.float32)
    k = np.repeat(rng.standard_normal((nkv, 1, hd)).astype(np.float16), 512, axis=1)
    v = rng.standard_normal((nkv, 512, hd)).astype(np.float16)
    o = ctx.attn_decode(ctx.to_device(q), ctx.to_device(k), ctx.to_device(v), nq, nkv, hd, L, 512)
    want = np.repeat(v[:, :L, :].astype(np.float64).mean(axis=1), nq // nkv, axis=0).reshape(-1)
    assert rel_l2(o, want) < 1e-6


@pytest.mark.parametrize("n_chunks", [1, 3, 64, 256])
def test_attention_chunking_invariant(ctx, n_chunks):
    nq, nkv, hd, L = 32, 8, 64, 700
    rng = np.random.default_rng(31)
    q = rng.standard_normal(nq * hd).astype(np.float32)
    k = rng.standard_normal((nkv, 1024, hd)).astype(np.float16)
    v = rng.standard_normal((nkv, 1024, hd)).astype(np.float16)
    o = ctx.attn_decode(ctx.to_device(q), ctx.to_device(k), ctx.to_device(v), nq, nkv, hd, L, 1024,
                        n_chunks)
    ref = oracle.attention(q, k.astype(np.float32), v.astype(np.float32), nq, nkv, hd, L)
    assert rel_l2(o, ref) < 1e-5


# ---------------------------------------------------------------- causal (prompt) attention

def causal_case(ctx, nq, nkv, hd, L0, T, seed, form, qmag=1.0, kv_dtype=np.float16):
    """T query rows at positions L0 .. L0+T-1 over a cache holding positions < L0 + T; the
    cache rows past that hold NaN, which no query may read.  Returns (gpu, oracle): the oracle
    is its single-position attention over the first L0 + t + 1 positions, row by row."""
    rng = np.random.default_rng(seed)
    stride = L0 + T + 40
    k = rng.standard_normal((nkv, stride, hd)).astype(kv_dtype)
    v = rng.standard_normal((nkv, stride, hd)).astype(kv_dtype)
    k[:, L0 + T:] = np.nan
    v[:, L0 + T:] = np.nan
    q = (rng.standard_normal((T, nq * hd)) * qmag).astype(np.float32)
    kvt = tpthip.TYPE_F32 if kv_dtype == np.float32 else tpthip.TYPE_F16
    o = ctx.attn_prefill(ctx.to_device(q), ctx.to_device(k), ctx.to_device(v), nq, nkv, hd, L0, T,
                         stride, form=form, kv_type=kvt)
    kf, vf = k.astype(np.float32), v.astype(np.float32)
    ref = np.stack([oracle.attention(q[t], kf, vf, nq, nkv, hd, L0 + t + 1) for t in range(T)])
    return o, ref


CAUSAL_SHAPES = [
    (32, 8, 128, 0, 256),    # Llama-3 8B heads, a prompt from position 0
    (32, 8, 128, 1000, 77),  # a ragged batch after a cached prefix
    (32, 8, 64, 5, 200),     # 1B heads, first position not on a 32-key block
    (4, 2, 64, 0, 150),      # the tiny test model's heads
    (16, 16, 128, 31, 33),   # MHA, the diagonal across two key blocks
    (16, 2, 64, 0, 1),       # one query
    (64, 8, 128, 3, 45),     # 8 query heads per kv head
]


@pytest.mark.parametrize("form", ["splitk", "mfma"])
@pytest.mark.parametrize("nq,nkv,hd,L0,T", CAUSAL_SHAPES)
def test_causal_attention_matches_oracle(ctx, nq, nkv, hd, L0, T, form):
    """Both causal forms against the oracle: the per-query split-K kernel and the matrix-core
    flash kernel (fp16 pairs for q and p, 2^-20 relative per operand)."""
    f = ctx.ATTN_SPLITK if form == "splitk" else ctx.ATTN_MFMA
    o, ref = causal_case(ctx, nq, nkv, hd, L0, T, seed=T + L0 + hd, form=f)
    assert np.isfinite(o).all()
    assert rel_l2(o, ref) < 1e-5
    # peaked softmax (scores of a few units): the log2-domain running max must track it
    o, ref = causal_case(ctx, nq, nkv, hd, L0, T, seed=T + L0 + hd + 1, form=f, qmag=6.0)
    assert rel_l2(o, ref) < 1e-5


def test_causal_forms_agree_prompt_shape(ctx):
    """The 8B prompt slice of the batched prefill (1024 queries after 1024 cached positions):
    the two causal forms agree to f32 accuracy at full size."""
    nq, nkv, hd, L0, T = 32, 8, 128, 1024, 1024
    rng = np.random.default_rng(77)
    k = ctx.to_device(rng.standard_normal((nkv, L0 + T, hd)).astype(np.float16))
    v = ctx.to_device(rng.standard_normal((nkv, L0 + T, hd)).astype(np.float16))
    q = ctx.to_device((rng.standard_normal((T, nq * hd)) * 2).astype(np.float32))
    a = ctx.attn_prefill(q, k, v, nq, nkv, hd, L0, T, L0 + T, form=ctx.ATTN_SPLITK)
    b = ctx.attn_prefill(q, k, v, nq, nkv, hd, L0, T, L0 + T, form=ctx.ATTN_MFMA)
    assert rel_l2(b, a) < 1e-5


def test_causal_attention_closed_forms(ctx):
    """Query 0 at position 0 sees one key: o = v_0 exactly; identical K rows give uniform
    weights: o = mean of V over the visible positions."""
    nq, nkv, hd = 8, 2, 128
    rng = np.random.default_rng(9)
    q = rng.standard_normal((40, nq * hd)).astype(np.float32)
    k = np.repeat(rng.standard_normal((nkv, 1, hd)).astype(np.float16), 64, axis=1)
    v = rng.standard_normal((nkv, 64, hd)).astype(np.float16)
    o = ctx.attn_prefill(ctx.to_device(q), ctx.to_device(k), ctx.to_device(v), nq, nkv, hd, 0, 40,
                         64, form=ctx.ATTN_MFMA)
    g = nq // nkv
    np.testing.assert_array_equal(o[0], np.repeat(v[:, 0, :].astype(np.float32), g, axis=0).reshape(-1))
    for t in (1, 31, 32, 39):
        want = np.repeat(v[:, :t + 1, :].astype(np.float64).mean(axis=1), g, axis=0).reshape(-1)
        assert rel_l2(o[t], want) < 1e-6, t


def test_causal_mfma_unsupported_shapes(ctx):
    """hd 96 and the f32 cache stay on the split-K form; asking the matrix cores for them fails."""
    for hd, dt in ((96, np.float16), (128, np.float32)):
        q = ctx.to_device(np.zeros((4, 8 * hd), np.float32))
        kv = ctx.to_device(np.zeros((2, 8, hd), dt))
        kvt = tpthip.TYPE_F32 if dt == np.float32 else tpthip.TYPE_F16
        with pytest.raises(tpthip.TptError) as e:
            ctx.attn_prefill(q, kv, kv, 8, 2, hd, 0, 4, 8, form=ctx.ATTN_MFMA, kv_type=kvt)
        assert e.value.code == tpthip.ERR_UNSUPPORTED
        o = ctx.attn_prefill(q, kv, kv, 8, 2, hd, 0, 4, 8, kv_type=kvt)  # auto: split-K
        assert np.all(o == 0)


def test_argmax_semantics(ctx):
    cases = [
        (np.array([1, 3, 3, 2], np.float32), 2),
        (np.array([-0.0, 0.0], np.float32), 1),
        (np.array([np.nan, 1.0], np.float32), 0),
        (np.array([-np.nan, 1.0], np.float32), 1),
    ]
    big = np.random.default_rng(1).standard_normal(128256).astype(np.float32)
    big[[5, 90000, 128000]] = 9.0
    cases.append((big, 128000))
    for v, want in cases:
        assert ctx.argmax(ctx.to_device(v), v.size) == want == oracle.argmax(v)


# ---------------------------------------------------------------- prefill GEMM (MFMA)

def gemm_case(ctx, M, K, N, seed, bf16=False, qtype=TYPE_Q4_K):
    w = synth.random_weights(qtype, N, K, seed=seed, name=f"g{K}x{N}")
    x = np.random.default_rng(seed).standard_normal((M, K)).astype(np.float32)
    if bf16:  # bf16 activations (values exactly representable in bf16)
        x = (x.view(np.uint32) & 0xFFFF0000).view(np.float32)
    return w, x


@pytest.mark.parametrize("M,K,N", [(16, 256, 64), (33, 512, 300), (128, 4096, 4096), (200, 2048, 1000),
                                   (130, 14336, 256), (300, 1024, 700)])
@pytest.mark.parametrize("qtype", GEMV_TYPES)
def test_gemm_q8k_matches_candle(ctx, M, K, N, qtype):
    """TPT_ACT_Q8: candle's prefill arithmetic for the weight type (each X row quantized to
    Q8_K for the k-quants, to Q8_0 for Q8_0 / Q4_0 weights, integer dots; for F16 weights an f32
    product); the integer sums are exact, so only f32 block accumulation order differs."""
    w, x = gemm_case(ctx, M, K, N, seed=M + K + N, qtype=qtype)
    y = ctx.gemm(qtype, ctx.to_device(w), ctx.to_device(x), M, K, N, act=tpthip.ACT_Q8)
    rows = np.arange(M) if M * N <= 200 * 1000 else np.random.default_rng(0).choice(M, 24, replace=False)
    ref = oracle.matmul(qtype, x[rows], w, N)
    for i, r in enumerate(rows):
        assert rel_l2(y[r], ref[i]) < 1e-5, r


@pytest.mark.parametrize("qtype", GEMV_TYPES)
def test_gemm_q8k_equals_gemv_rows(ctx, qtype):
    """Batched prefill rows equal the decode GEMV of the same row (same Q8_K arithmetic)."""
    M, K, N = 40, 4096, 512
    w, x = gemm_case(ctx, M, K, N, seed=77, qtype=qtype)
    wd = ctx.to_device(w)
    y = ctx.gemm(qtype, wd, ctx.to_device(x), M, K, N, act=tpthip.ACT_Q8)
    for r in (0, 17, 39):
        yv = ctx.gemv(qtype, wd, ctx.to_device(x[r].copy()), K, N)
        assert rel_l2(y[r], yv) < 1e-6


def q6k_extreme_blocks(n_blocks, seed):
    """Q6_K blocks whose integers sc * (q - 32) reach the ends of [-4064, 4096] and odd values
    past 2048 (not representable in fp16): scales from {-128, -127, 127, 65, -1, 0}, every
    6-bit q, d = 1."""
    rng = np.random.default_rng(seed)
    b = np.zeros((n_blocks, 210), np.uint8)
    b[:, :192] = rng.integers(0, 256, (n_blocks, 192), dtype=np.uint8)  # ql, qh: all q values
    sc = rng.choice(np.array([-128, -127, 127, 65, -1, 0], np.int8), (n_blocks, 16))
    b[:, 192:208] = sc.view(np.uint8)
    b[:, 208:210] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    return b.reshape(-1)


def test_gemm_q6k_exact_at_integer_extremes(ctx):
    """The split w = 64 w1 + w0 keeps every Q6_K product exact where sc * (q - 32) leaves fp16's
    exact range: rows of +-1 activations (Q8_K values -128 / 127 after quantization) against
    blocks of extreme scales give the oracle's integers to f32 rounding."""
    M, K, N = 48, 1024, 64
    w = q6k_extreme_blocks(N * K // 256, seed=3)
    x = np.random.default_rng(4).choice(np.array([-1.0, 1.0, 0.5], np.float32), (M, K))
    y = ctx.gemm(TYPE_Q6_K, ctx.to_device(w), ctx.to_device(x), M, K, N, act=tpthip.ACT_Q8)
    ref = oracle.matmul(TYPE_Q6_K, x, w, N)
    assert rel_l2(y, ref) < 1e-6
    yv = ctx.gemv(TYPE_Q6_K, ctx.to_device(w), ctx.to_device(x[5].copy()), K, N)
    assert rel_l2(y[5], yv) < 1e-6


def q5k_extreme_blocks(n_blocks, seed):
    """Q5_K blocks (d = 1) with every 5-bit q: half of them with all eight scales and mins 63
    (integers sc * q up to 1953), half with random packed scales."""
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (n_blocks, 176), dtype=np.uint8)  # scales, qh, qs: every value
    b[: n_blocks // 2, 4:16] = 0xFF  # get_scale_min_k4 reads 63 for every sc and m
    b[:, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    b[:, 2:4] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    return b.reshape(-1)


def test_gemm_q5k_exact_at_integer_extremes(ctx):
    """Q5_K's integer sums reach 256 * 128 * 1953 (past 2^24) for +-1 activations against
    scales of 63: the split w = 64 w1 + w0 keeps both chains exact, so the GEMM equals the
    oracle's integer arithmetic to f32 rounding, and the decode GEMV row for row."""
    M, K, N = 48, 1024, 64
    w = q5k_extreme_blocks(N * K // 256, seed=5)
    x = np.random.default_rng(6).choice(np.array([-1.0, 1.0, 0.5], np.float32), (M, K))
    y = ctx.gemm(TYPE_Q5_K, ctx.to_device(w), ctx.to_device(x), M, K, N, act=tpthip.ACT_Q8)
    ref = oracle.matmul(TYPE_Q5_K, x, w, N)
    assert rel_l2(y, ref) < 1e-6
    yv = ctx.gemv(TYPE_Q5_K, ctx.to_device(w), ctx.to_device(x[7].copy()), K, N)
    assert rel_l2(y[7], yv) < 1e-6


def q4k_extreme_blocks(n_blocks, seed):
    """Q4_K blocks (d = 1, dmin = 0.25) with every scale and min 63: a third with all q = 0
    (the integers sc * q - 480 of the 256-row tile at -480), a third with all q = 15 (945), a
    third with random nibbles."""
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (n_blocks, 144), dtype=np.uint8)
    b[:, 4:16] = 0xFF
    b[0::3, 16:] = 0x00
    b[1::3, 16:] = 0xFF
    b[:, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    b[:, 2:4] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    return b.reshape(-1)


# the last three run whole rounds of 256 x 128 tiles and hand the columns of a half round to the
# 128 x 128 kernel (M = 300: shifted-back row tiles in both parts)
WIDE_CASES = [(256, 4096, 4096), (300, 512, 200), (520, 2048, 1000), (2048, 4096, 1024),
              (2048, 4096, 4096), (256, 4096, 256), (512, 256, 24576), (300, 512, 24576),
              (2048, 4096, 6144)]


def gemm_split_count(M, N, K, tile_m):
    """The launcher's split-K count for a grid of tile_m x 128 tiles (k_gemm.hip splits_for)."""
    tiles, nkb = -(-N // 128) * -(-M // tile_m), K // 256
    return 1 if tiles > 128 or nkb < 4 else min(256 // tiles, nkb // 2, 8)


@pytest.mark.parametrize("M,K,N", WIDE_CASES)
@pytest.mark.parametrize("act", [tpthip.ACT_Q8, tpthip.ACT_F16])
def test_gemm_wide_tiles_equal_narrow(ctx, monkeypatch, M, K, N, act):
    """Q4_K over M >= 256 rows runs on 256 x 128 tiles (one exact chain per super-block on
    w - 480, activation tiles by LDS DMA, last tiles shifted back inside the matrix); the
    128 x 128 kernel computes every element with the same integers and f32 steps, so the two
    agree bit for bit when both split K the same way (partial row and column tiles, 4 and 8
    splits, none, a grid split between the two kernels), and to f32 regrouping of the split
    sums otherwise; both modes."""
    w, x = gemm_case(ctx, M, K, N, seed=M + 7 * N + K, qtype=TYPE_Q4_K)
    wd, xd = ctx.to_device(w), ctx.to_device(x)
    monkeypatch.setenv("TPT_HIP_GEMM_TILE", "narrow")
    y0 = ctx.gemm(TYPE_Q4_K, wd, xd, M, K, N, act=act)
    monkeypatch.delenv("TPT_HIP_GEMM_TILE")
    y1 = ctx.gemm(TYPE_Q4_K, wd, xd, M, K, N, act=act)
    if gemm_split_count(M, N, K, 128) == gemm_split_count(M, N, K, 256):
        assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))
    else:
        assert rel_l2(y1, y0) < 1e-6


def test_gemm_wide_exact_at_integer_extremes(ctx, monkeypatch):
    """The 256-row tile's chain sum(q8 * (sc q - 480)) reaches its bound 256 * 128 * 480 < 2^24
    for rows of +1 (Q8_K -128 everywhere) against q = 0 blocks of scale 63; with +-1 and 0.5
    rows and q = 15 or random blocks the GEMM still equals the oracle's integers to f32
    rounding and the 128 x 128 kernel bit for bit."""
    M, K, N = 256, 1024, 128
    w = q4k_extreme_blocks(N * K // 256, seed=8)
    x = np.random.default_rng(9).choice(np.array([-1.0, 1.0, 0.5], np.float32), (M, K))
    x[0::4] = 1.0
    x[1::4] = -1.0
    wd, xd = ctx.to_device(w), ctx.to_device(x)
    monkeypatch.delenv("TPT_HIP_GEMM_TILE", raising=False)
    y = ctx.gemm(TYPE_Q4_K, wd, xd, M, K, N, act=tpthip.ACT_Q8)
    ref = oracle.matmul(TYPE_Q4_K, x, w, N)
    assert rel_l2(y, ref) < 1e-6
    monkeypatch.setenv("TPT_HIP_GEMM_TILE", "narrow")
    y0 = ctx.gemm(TYPE_Q4_K, wd, xd, M, K, N, act=tpthip.ACT_Q8)
    assert np.array_equal(y0.view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("M,N,qtype", [(128, 4096, TYPE_Q4_K), (512, 4096, TYPE_Q4_K), (2048, 4096, TYPE_Q4_K),
                                       (128, 14336, TYPE_Q4_K), (512, 14336, TYPE_Q4_K), (2048, 14336, TYPE_Q4_K),
                                       (512, 4096, TYPE_Q6_K), (512, 4096, TYPE_Q5_K)])
def test_gemm_f16_config3(ctx, M, N, qtype):
    """fp16 MFMA mode at the prefill shapes (K=4096, bf16 activations): within 1e-3 relative L2
    of the fp64 product of the exactly dequantized weights (checked on a row/column sample)."""
    K = 4096
    w, x = gemm_case(ctx, M, K, N, seed=M * 3 + N, bf16=True, qtype=qtype)
    y = ctx.gemm(qtype, ctx.to_device(w), ctx.to_device(x), M, K, N, act=tpthip.ACT_F16)
    nc = min(N, 1024)
    rb = (K // 256) * tpthip.TYPE_SIZE[qtype]
    wdq = oracle.dequant(qtype, w[: nc * rb], nc * K).astype(np.float64).reshape(nc, K)
    rows = np.random.default_rng(1).choice(M, min(M, 64), replace=False)
    ref = x[rows].astype(np.float64) @ wdq.T
    assert rel_l2(y[rows][:, :nc], ref) < 1e-3


def test_gemm_rejects_bad_shapes(ctx):
    w = ctx.alloc(4096)
    x = ctx.alloc(4096)
    with pytest.raises(tpthip.TptError):
        ctx.gemm(TYPE_Q4_K, w, x, 4, 100, 4, act=tpthip.ACT_Q8)  # K not a multiple of 256
    with pytest.raises(tpthip.TptError):
        ctx.gemm(TYPE_Q8_0, w, x, 4, 256, 4, act=tpthip.ACT_F16)  # Q8_0 and Q4_0: Q8_0 activations only
    with pytest.raises(tpthip.TptError):
        ctx.gemm(tpthip.TYPE_F32, w, x, 4, 256, 4, act=tpthip.ACT_Q8)
