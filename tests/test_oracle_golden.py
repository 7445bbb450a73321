"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each check is a known answer worked out by hand, a closed form or an identity, chosen so that
a plausible mistake (wrong nibble order, wrong scale packing, banker's rounding, first-vs-last
tie rule, rotate-half RoPE, a dropped mins term) fails.  The reference ships no golden vectors
for this path (its only tests are KvCache prefix tests, wgpu_kvcache.rs:96-133).
"""
import json
import math
import os
import struct

import numpy as np
import pytest

import oracle

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kat_blocks.json")))


def q4k_block():
    g = GOLD["q4k"]
    qs = bytes([(i % 16) | ((15 - i % 16) << 4) for i in range(128)])
    return struct.pack("<HH", g["d_bits"], g["dmin_bits"]) + bytes(g["scales"]) + qs


def q6k_block():
    g = GOLD["q6k"]
    ql = bytes([(5 * i) & 255 for i in range(128)])
    qh = bytes([(3 * i) & 255 for i in range(64)])
    sc = struct.pack("<16b", *g["scales"])
    return ql + qh + sc + struct.pack("<H", g["d_bits"])


def q8_0_block():
    g = GOLD["q8_0"]
    qs = g["qs"] + [0] * (32 - len(g["qs"]))
    return struct.pack("<H", g["d_bits"]) + struct.pack("<32b", *qs)


def test_q4k_known_answers():
    y = oracle.dequant(oracle.Q4_K, np.frombuffer(q4k_block(), np.uint8), 256)
    for k, v in GOLD["q4k"]["expect"].items():
        assert y[int(k)] == v, (k, y[int(k)], v)


def test_q4k_scale_unpack_matches_hand_packing():
    # every element of sub-block j with q == 0 equals -dmin * m_j; with q == 1 it is sc_j*d - dmin*m_j
    g = GOLD["q4k"]
    y = oracle.dequant(oracle.Q4_K, np.frombuffer(q4k_block(), np.uint8), 256)
    for j in range(8):
        gi, hi = divmod(j, 2)
        first = 64 * gi + 32 * hi  # element whose byte is qs[32*gi] (low nibble 0, high nibble 15)
        q = 0 if hi == 0 else 15
        assert y[first] == g["sc"][j] * q - 0.5 * g["m"][j]


def test_q4k_closed_forms():
    # all qs = 0  ->  y = -dmin * m_j ;  d = 1, dmin = 0, every sc = 1  ->  y = q
    blk = bytearray(q4k_block())
    blk[16:] = bytes(128)
    y = oracle.dequant(oracle.Q4_K, np.frombuffer(bytes(blk), np.uint8), 256)
    m = GOLD["q4k"]["m"]
    assert all(y[32 * j + l] == -0.5 * m[j] for j in range(8) for l in range(32))
    ident = bytearray(struct.pack("<HH", 0x3C00, 0) + bytes([1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]))
    ident += bytes([(i % 16) | ((i // 16 % 16) << 4) for i in range(128)])
    y = oracle.dequant(oracle.Q4_K, np.frombuffer(bytes(ident), np.uint8), 256)
    for g in range(4):
        for l in range(32):
            b = 32 * g + l
            assert y[64 * g + l] == b % 16 and y[64 * g + 32 + l] == b // 16 % 16


def test_q6k_known_answers():
    y = oracle.dequant(oracle.Q6_K, np.frombuffer(q6k_block(), np.uint8), 256)
    for k, v in GOLD["q6k"]["expect"].items():
        assert y[int(k)] == v, (k, y[int(k)], v)


def test_q8_0_known_answers():
    y = oracle.dequant(oracle.Q8_0, np.frombuffer(q8_0_block(), np.uint8), 32)
    assert list(y[:5]) == GOLD["q8_0"]["expect"]
    assert not y[5:].any()


def q5k_block():
    """d = 1, dmin = 0.5; scale bytes giving (sc, m) = (1,0) (2,1) (3,2) (4,3) for sub-blocks 0-3
    (low 6 bits of bytes 0-3 / 4-7) and (1,2) (3,4) (5,6) (7,8) for 4-7 (nibbles of bytes
    8-11); qs[i] = (i % 16) | (15 - i % 16) << 4; qh[l] = 0xFF for odd l, 0 for even l (the
    fifth bit of every sub-block set exactly on odd l)."""
    qs = bytes([(i % 16) | ((15 - i % 16) << 4) for i in range(128)])
    qh = bytes([0xFF if l % 2 else 0 for l in range(32)])
    return struct.pack("<HH", 0x3C00, 0x3800) + bytes([1, 2, 3, 4, 0, 1, 2, 3, 0x21, 0x43, 0x65, 0x87]) + qh + qs


def test_q5k_known_answers():
    """Element e: group j = e // 64, half e % 64 // 32, l = e % 32; q = nibble + 16 * (l odd);
    y = sc * q - 0.5 * m, worked by hand."""
    y = oracle.dequant(oracle.Q5_K, np.frombuffer(q5k_block(), np.uint8), 256)
    expect = {0: 0.0,      # j0 low, l0: nibble 0, bit clear, sc 1, m 0
              1: 17.0,     # j0 low, l1: 1 + 16
              33: 59.5,    # j0 high, l1: 14 + 16 = 30, sc 2: 60 - 0.5 * 1
              34: 25.5,    # j0 high, l2: 13, sc 2: 26 - 0.5
              69: 62.0,    # j1 low, l5: 5 + 16 = 21, sc 3: 63 - 0.5 * 2
              167: 70.0,   # j2 high, l7: qs[71] high nibble 8 + 16 = 24, sc 3: 72 - 0.5 * 4
              222: 67.0,   # j3 low, l30: 14, sc 5: 70 - 0.5 * 6
              255: 108.0}  # j3 high, l31: 0 + 16, sc 7: 112 - 0.5 * 8
    for k, v in expect.items():
        assert y[k] == v, (k, y[k], v)


def test_q4_0_known_answers():
    """d = 0.5, qs[j] = j | (15 - j) << 4: element j < 16 is (j - 8) / 2, element j + 16 is
    (7 - j) / 2."""
    blk = struct.pack("<H", 0x3800) + bytes([j | ((15 - j) << 4) for j in range(16)])
    y = oracle.dequant(oracle.Q4_0, np.frombuffer(blk, np.uint8), 32)
    assert list(y[[0, 8, 15, 16, 20, 31]]) == [-4.0, 0.0, 3.5, 3.5, 1.5, -4.0]


def q8k_parse(raw):
    d = struct.unpack("<f", raw[:4].tobytes())[0]
    return d, raw[4:260].view(np.int8), raw[260:292].view(np.int16)


@pytest.mark.parametrize("case", range(len(GOLD["q8k"])))
def test_q8k_known_answers(case):
    c = GOLD["q8k"][case]
    x = np.zeros(256, np.float32)
    x[:len(c["x_head"])] = c["x_head"]
    d, q, bs = q8k_parse(oracle.quantize_q8k(x))
    assert list(q[:len(c["q_head"])]) == c["q_head"]
    if "d" in c:
        assert d == c["d"]
    else:
        assert abs(d - c["d_approx"]) < 1e-6
    if "bsum0" in c:
        assert bs[0] == c["bsum0"]
    for j in range(16):
        assert bs[j] == int(q[16 * j:16 * j + 16].astype(np.int32).sum())


def test_q8_0_activation_quant():
    x = np.zeros(32, np.float32)
    x[:3] = [0.5, -1.0, 0.25]
    raw = oracle.quantize_q8_0(x)
    d = oracle.fp16_bits_to_f32(struct.unpack("<H", raw[:2].tobytes())[0])
    assert d == oracle.fp16_bits_to_f32(oracle.f32_to_fp16_bits(np.float32(1.0) / np.float32(127.0)))
    assert list(raw[2:5].view(np.int8)) == [64, -127, 32]  # 63.5 rounds away from zero


def test_fp16_roundtrip_edges():
    for bits in (0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0x7C00, 0xFC00, 0x8001):
        assert oracle.f32_to_fp16_bits(oracle.fp16_bits_to_f32(bits)) == bits
    assert oracle.fp16_bits_to_f32(0x0001) == 2.0 ** -24
    assert oracle.f32_to_fp16_bits(2.0 ** -25) == 0  # tie to even
    assert oracle.f32_to_fp16_bits(1.0 + 2.0 ** -11) == 0x3C00  # tie to even
    assert oracle.f32_to_fp16_bits(65520.0) == 0x7C00  # overflow


def _rand_blocks(qtype, nblocks, seed):
    """Random block bytes with sane scale fields (f16 scales in [2^-10, 2^-6])."""
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, nblocks * oracle.TYPE_SIZE[qtype], dtype=np.uint8)
    blk = raw.reshape(nblocks, oracle.TYPE_SIZE[qtype])
    h = rng.integers(0x1000, 0x2400, (nblocks, 2)).astype("<u2").view(np.uint8)
    if qtype in (oracle.Q4_K, oracle.Q5_K):
        blk[:, 0:4] = h.reshape(nblocks, 4)
    elif qtype == oracle.Q6_K:
        blk[:, 208:210] = h[:, :2]
    else:
        blk[:, 0:2] = h[:, :2]
    return raw


@pytest.mark.parametrize("qtype", [oracle.Q4_K, oracle.Q5_K, oracle.Q6_K, oracle.Q8_0, oracle.Q4_0])
def test_vec_dot_identity(qtype):
    """candle's integer vec_dot equals the fp64 dot of the two dequantized operands."""
    k, n = 1024, 24
    w = _rand_blocks(qtype, k // oracle.BLOCK[qtype] * n, 11)
    x = np.random.default_rng(3).standard_normal(k).astype(np.float32)
    q80 = qtype in (oracle.Q8_0, oracle.Q4_0)
    aq = oracle.quantize_q8_0(x) if q80 else oracle.quantize_q8k(x)
    xd = oracle.dequant(oracle.Q8_0 if q80 else oracle.Q8_K, aq, k).astype(np.float64)
    rb = oracle.row_bytes(qtype, k)
    for r in range(n):
        wd = oracle.dequant(qtype, w[r * rb:(r + 1) * rb], k).astype(np.float64)
        ref = float(wd @ xd)
        got = oracle.vec_dot(qtype, k, w[r * rb:(r + 1) * rb], aq)
        # f32 rounding of the block sums only; a dropped or sign-flipped mins term or a wrong
        # nibble order is an O(|ref|) error
        assert abs(got - ref) <= 1e-5 * (abs(ref) + 0.01 * np.abs(wd * xd).sum()), (r, got, ref)
    y = oracle.matmul(qtype, x, w, n)[0]
    assert all(y[r] == oracle.vec_dot(qtype, k, w[r * rb:(r + 1) * rb], aq) for r in range(n))


def test_gemv_f64_linearity():
    k, n = 512, 16
    w = _rand_blocks(oracle.Q4_K, k // 256 * n, 5)
    rng = np.random.default_rng(9)
    a, b = rng.standard_normal(k), rng.standard_normal(k)
    ya, yb = oracle.gemv_f64(oracle.Q4_K, w, a, n), oracle.gemv_f64(oracle.Q4_K, w, b, n)
    np.testing.assert_allclose(oracle.gemv_f64(oracle.Q4_K, w, 2 * a - 3 * b, n), 2 * ya - 3 * yb,
                               rtol=1e-12, atol=1e-12)


def test_f16_matmul_widening_and_fp64():
    """candle's F16 QMatMul (dequantize to f32, f32 matmul): one-hot activations pick single
    weights, so every finite f16 value (subnormals, both zeros, +-65504) must come out as
    numpy's float16 -> float32 widening; random rows stay within f32 rounding of the fp64 dot
    (a byte swap, a bf16 reading or a dropped term is an O(1) error)."""
    bits = np.arange(65536, dtype=np.uint16)
    bits = bits[(bits & 0x7C00) != 0x7C00]
    k = 256
    n = bits.size // k
    w = bits[:n * k].reshape(n, k)
    for j in (0, 1, 100, 255):
        x = np.zeros(k, np.float32)
        x[j] = 1.0
        y = oracle.matmul(oracle.F16, x, w.view(np.uint8).reshape(-1), n)[0]
        np.testing.assert_array_equal(y, w[:, j].view(np.float16).astype(np.float32))
    rng = np.random.default_rng(12)
    k, n = 4096, 48
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
    x = rng.standard_normal(k).astype(np.float32)
    y = oracle.matmul(oracle.F16, x, wf.view(np.uint8).reshape(-1), n)[0]
    prod = wf.astype(np.float64) * x.astype(np.float64)
    assert np.all(np.abs(y - prod.sum(1)) <= 1e-5 * np.abs(prod).sum(1))


def test_rmsnorm_closed_form():
    n, eps = 4096, 1e-5
    y = oracle.rmsnorm(np.full(n, 2.0, np.float32), np.full(n, 3.0, np.float32), eps)
    assert np.allclose(y, 3 * 2 / math.sqrt(4 + eps), rtol=2e-7)


def test_silu_closed_forms():
    assert oracle.silu(0.0) == 0.0
    assert abs(oracle.silu(30.0) - 30.0) < 1e-5
    assert abs(oracle.silu(-1.0) - (-1.0 / (1 + math.e))) < 1e-7


def test_rope_tables_and_pairing():
    hd, base = 64, 500000.0
    c, s = oracle.rope_tables(hd, base, 6)
    assert np.all(c[0] == 1) and np.all(s[0] == 0)  # pos 0 = identity
    for p in range(6):
        for i in range(hd // 2):
            ang = p * (base ** (-2 * i / hd))
            assert abs(c[p, i] - math.cos(ang)) < 2e-6 and abs(s[p, i] - math.sin(ang)) < 2e-6
    x = np.zeros(2 * hd, np.float32)
    x[0] = 1.0
    y = oracle.rope_i(x, 2, hd, c[5], s[5])
    # interleaved pairs: (x0, x1) -> (cos, sin); rotate-half would move sin to index hd/2
    assert abs(y[0] - math.cos(5)) < 2e-6 and abs(y[1] - math.sin(5)) < 2e-6 and y[hd // 2] == 0
    r = np.random.default_rng(1).standard_normal(2 * hd).astype(np.float32)
    yr = oracle.rope_i(r, 2, hd, c[3], s[3])
    np.testing.assert_allclose(np.hypot(yr[0::2], yr[1::2]), np.hypot(r[0::2], r[1::2]), rtol=1e-6)


def test_attention_closed_forms():
    nq, nkv, hd, L = 8, 2, 64, 7
    rng = np.random.default_rng(2)
    kc = rng.standard_normal((nkv, 16, hd)).astype(np.float32)
    vc = rng.standard_normal((nkv, 16, hd)).astype(np.float32)
    q = rng.standard_normal(nq * hd).astype(np.float32)
    o1 = oracle.attention(q, kc, vc, nq, nkv, hd, 1).reshape(nq, hd)
    for h in range(nq):  # a single position: softmax = 1, o = v
        np.testing.assert_allclose(o1[h], vc[h // (nq // nkv), 0], rtol=1e-6)
    o0 = oracle.attention(np.zeros_like(q), kc, vc, nq, nkv, hd, L).reshape(nq, hd)
    for h in range(nq):  # uniform scores: o = mean(V)
        np.testing.assert_allclose(o0[h], vc[h // (nq // nkv), :L].mean(0), rtol=1e-5, atol=1e-6)


def test_argmax_ties_and_total_order():
    assert oracle.argmax(np.array([1, 3, 3, 2], np.float32)) == 2
    assert oracle.argmax(np.array([-0.0, 0.0], np.float32)) == 1
    assert oracle.argmax(np.array([0.0, -0.0], np.float32)) == 0
    assert oracle.argmax(np.array([np.nan, 1.0], np.float32)) == 0
    assert oracle.argmax(np.array([-np.nan, 1.0], np.float32)) == 1


def test_repeat_penalty_applies_per_occurrence():
    lg = np.array([2.0, -2.0, 1.0], np.float32)
    out = oracle.repeat_penalty(lg, [0, 0, 1], 2.0)
    assert list(out) == [0.5, -4.0, 1.0]
    assert list(oracle.repeat_penalty(lg, [0, 1], 1.0)) == list(lg)


def test_rms_order_instrument():
    """The RMSNorm order probe changes only the f32 order of sum(x^2): with it on, m equals the
    16-run + pairwise-tree sum computed here in float64-exact steps rounded as the oracle
    rounds, and every output stays within a few ulps of candle's sequential order."""
    rng = np.random.default_rng(11)
    n = 4096
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    w = np.ones(n, np.float32)
    base = oracle.rmsnorm(x, w, 1e-5)
    oracle.set_rms_order(True)
    try:
        tree = oracle.rmsnorm(x, w, 1e-5)
    finally:
        oracle.set_rms_order(False)
    # the tree order by hand: fmaf runs of 16 (a*b exact in float64, one rounding to f32 per step)
    runs = []
    for j in range(n // 16):
        s = np.float32(0)
        for v in x[16 * j:16 * j + 16]:
            s = np.float32(np.float64(v) * np.float64(v) + np.float64(s))
        runs.append(s)
    p = runs
    while len(p) > 1:
        q = [np.float32(p[2 * i] + p[2 * i + 1]) for i in range(len(p) // 2)]
        if len(p) % 2:
            q.append(p[-1])
        p = q
    m = np.sqrt(np.float32(p[0] / np.float32(n) + np.float32(1e-5)), dtype=np.float32)
    assert np.array_equal(tree, (x / m * w).astype(np.float32))
    ulp = np.spacing(np.abs(base)).astype(np.float64)
    assert np.all(np.abs(tree.astype(np.float64) - base) <= 4 * ulp + 1e-30)
