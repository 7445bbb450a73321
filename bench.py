#!/usr/bin/env python3
"""Benchmark of the bs=1 Q4_K_M Llama decode path on one MI355X.

Workload (the configuration the headline metric is quoted on): a Llama-3 8B-shape random-init
GGUF quantized Q4_K_M (token_embd/output Q6_K, other matrices Q4_K, norms F32), generated from
a fixed seed; end-to-end through the LlmEngine mirror at batch 1 with run_benchmark's greedy
parameters (temperature 0, top_p 1, repeat_penalty 1): a 2048-token seeded random prompt, then
greedy decode.  A "step" is one decode token.  --warmup W decode tokens run in an untimed first
infer; the timed infer decodes --steps K tokens.  value = K / decode seconds, the reference's
tokens_per_sec = tokens_generated / decode_s with decode timed from the first token to the end
(run_benchmark, src-tauri/src/commands.rs:542-564).  Weights and KV are resident in HBM before
the timed region.

roofline: the Q4_K fused dequant-GEMV at 4096 -> 14336 (the gate/up shape), timed with HIP
start/stop events that each dispatch timestamps itself (hipExtLaunchKernelGGL) on the
context's stream, over back-to-back launches that rotate through distinct weight copies
(> 1 GB, more than the 256 MB Infinity Cache).  Algorithmic bytes per launch =
K*N*144/256 + 4K + 4N.  traffic comes from the committed rocprofv3 PMC summary when present.

Further legs reported in `config` (not the headline): decode attention at the long-context
shapes (`attn_decode_f16`, GB/s vs HBM peak over rotating caches), the MFMA prefill GEMM at the
prompt shapes (`prefill_gemm_q4k`, TFLOP/s vs the 2.5 PFLOP/s dense fp16 peak) and the
matrix-core causal prompt attention (`prefill_attn_causal_f16`, algorithmic TFLOP/s, same peak).

Also in `config`: the Q6_K and Q8_0 GEMVs at the same four shapes (`gemv_q6k`, `gemv_q8_0`).

cpu_baseline: the CPU oracle's restatement of candle's CPU decode (Q8_K activation quant,
integer vec_dot, OpenMP over output columns) timed on this host's cores on a bounded sample of
the same model at the GPU run's decode positions (its KV cache primed with as many positions as
the prompt), greedy decode steps for about 20 s; nproc, the CPU model and the thread count are
recorded.
"""
import argparse
import json
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tpt-spark_amd"))

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
METRIC = "decode tok/s (bs=1, 8B-shape Q4_K_M) + Q4_K GEMV achieved HBM GB/s vs peak"
PROMPT_LEN = 2048
SEED = 20261201


def log(*a):
    print(*a, file=sys.stderr, flush=True)


COPY_BYTES = 256 << 20


def copy_calibration(ctx, iters=4):
    """A plain 16-byte vector copy of COPY_BYTES (read) into another buffer (write): the
    reference kernel whose FETCH_SIZE / WRITE_SIZE counters calibrate the GEMV's."""
    src, dst = ctx.alloc(COPY_BYTES), ctx.alloc(COPY_BYTES)
    ctx.bench_copy(dst, src, COPY_BYTES, 1)  # first touch of both buffers
    ms = ctx.bench_copy(dst, src, COPY_BYTES, iters)
    src.free()
    dst.free()
    gbs = 2 * COPY_BYTES / (ms / iters * 1e-3) / 1e9
    log(f"copy {COPY_BYTES >> 20} MiB: {ms / iters * 1e3:.1f} us/launch, {gbs:.0f} GB/s read+write")
    return {"bytes_read": COPY_BYTES, "bytes_written": COPY_BYTES, "us_per_launch": round(ms / iters * 1e3, 2)}


GEMV_SHAPES = [(4096, 14336), (14336, 4096), (4096, 4096), (4096, 1024)]


def gemv_roofline(tp, ctx, iters=256, qtype=None):
    """Event-timed fused dequant-GEMV at the config-2 shapes (K -> N), rotating through >= 1 GB
    of weight copies.  Algorithmic bytes per launch = the quantized weight blocks (Q4_K 144 B,
    Q6_K 210 B per 256 weights, Q8_0 34 B per 32) + fp32 x + fp32 y."""
    from tpthip import synth
    qtype = tp.TYPE_Q4_K if qtype is None else qtype
    name = {tp.TYPE_Q4_K: "q4_k", tp.TYPE_Q6_K: "q6_k", tp.TYPE_Q8_0: "q8_0"}[qtype]
    out = {}
    for K, N in GEMV_SHAPES:
        w = synth.random_weights(qtype, N, K, seed=K + N, name=f"bench{K}x{N}")
        n_copies = max(2, int(np.ceil(1.1e9 / w.nbytes)))
        bufs = [ctx.to_device(w) for _ in range(n_copies)]
        x = ctx.to_device(np.random.default_rng(1).standard_normal(K).astype(np.float32))
        y = ctx.alloc(N * 4)
        ctx.bench_gemv(qtype, bufs, x, y, K, N, n_copies)  # warm-up pass
        ms = ctx.bench_gemv(qtype, bufs, x, y, K, N, iters)
        alg = K * N // tp.BLOCK[qtype] * tp.TYPE_SIZE[qtype] + 4 * K + 4 * N
        us = ms * 1e3 / iters
        gbs = alg / (us * 1e-6) / 1e9
        out[f"{K}x{N}"] = {"bytes": alg, "us_per_launch": round(us, 3), "gbs": round(gbs, 1),
                           "frac": round(gbs / HBM_PEAK_GBS, 4), "copies": n_copies}
        log(f"gemv {name} {K}->{N}: {us:.2f} us/launch, {gbs:.0f} GB/s")
        for b in bufs:
            b.free()
    return out


# decode attention at the long-context shapes: GQA 32/8 hd 128 and MHA 32/32 hd 96, fp16 cache
ATTN_CASES = [(32, 8, 128, 512), (32, 8, 128, 4096), (32, 8, 128, 16384), (32, 8, 128, 32768),
              (32, 32, 96, 512), (32, 32, 96, 4096), (32, 32, 96, 16384), (32, 32, 96, 32768)]


def attn_roofline(tp, ctx, iters=64):
    """Event-timed split-K decode attention (partial + merge launches) at ATTN_CASES, rotating
    through >= 1.1 GB of distinct K/V caches.  Algorithmic bytes per call = K and V rows read
    once (2 * Nkv * L * hd * 2 B) + q and o (2 * Nq * hd * 4 B)."""
    out = {}
    rng = np.random.default_rng(7)
    for nq, nkv, hd, L in ATTN_CASES:
        k = rng.standard_normal((nkv, L, hd), dtype=np.float32).astype(np.float16)
        n_copies = max(2, int(np.ceil(1.1e9 / (2 * k.nbytes))))
        ks = [ctx.to_device(k) for _ in range(n_copies)]
        vs = [ctx.to_device(k) for _ in range(n_copies)]
        q = ctx.to_device(rng.standard_normal(nq * hd, dtype=np.float32))
        o = ctx.alloc(nq * hd * 4)
        ctx.bench_attn(q, ks, vs, o, nq, nkv, hd, L, L, n_copies)  # warm-up pass
        n = max(iters, n_copies)
        ms = ctx.bench_attn(q, ks, vs, o, nq, nkv, hd, L, L, n)
        alg = 2 * nkv * L * hd * 2 + 2 * nq * hd * 4
        us = ms * 1e3 / n
        gbs = alg / (us * 1e-6) / 1e9
        out[f"{nq}/{nkv}x{hd}@{L}"] = {"bytes": alg, "us_per_call": round(us, 3), "gbs": round(gbs, 1),
                                        "frac": round(gbs / HBM_PEAK_GBS, 4), "copies": n_copies}
        log(f"attention {nq}/{nkv} hd {hd} L {L}: {us:.2f} us/call, {gbs:.0f} GB/s")
        for b in ks + vs + [q, o]:
            b.free()
    return out


# causal prompt attention: (Nq, Nkv, hd, L0 cached positions, T queries) at the Llama-3 8B head
# shape -- the 2048-token prompt (one slice), and the second slice of a 4096-token prompt
ATTN_CAUSAL_CASES = [(32, 8, 128, 0, 2048), (32, 8, 128, 2048, 2048)]


def attn_causal_roofline(tp, ctx, iters=20):
    """Event-timed matrix-core causal attention at ATTN_CAUSAL_CASES.  Algorithmic flops per
    launch = 4 * Nq * hd * (visible positions summed over the T queries) -- q.k and p.v, 2 flops
    per multiply-add; the kernel issues twice that on the matrix cores (fp16 hi/lo operand pairs)
    plus the masked halves of the diagonal blocks.  Priced against the dense fp16 MFMA peak."""
    out = {}
    rng = np.random.default_rng(11)
    for nq, nkv, hd, L0, T in ATTN_CAUSAL_CASES:
        L = L0 + T
        k = ctx.to_device(rng.standard_normal((nkv, L, hd), dtype=np.float32).astype(np.float16))
        v = ctx.to_device(rng.standard_normal((nkv, L, hd), dtype=np.float32).astype(np.float16))
        q = ctx.to_device(rng.standard_normal((T, nq * hd), dtype=np.float32))
        o = ctx.alloc(T * nq * hd * 4)
        ctx.bench_attn_prefill(q, k, v, o, nq, nkv, hd, L0, T, L, 2)
        ms = ctx.bench_attn_prefill(q, k, v, o, nq, nkv, hd, L0, T, L, iters)
        us = ms * 1e3 / iters
        flops = 4.0 * nq * hd * (T * L0 + T * (T + 1) / 2)
        tf = flops / (us * 1e-6) / 1e12
        out[f"{nq}/{nkv}x{hd} L0={L0} T={T}"] = {"flops": flops, "us_per_launch": round(us, 2),
                                                 "tflops": round(tf, 1),
                                                 "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4)}
        log(f"causal attention {nq}/{nkv} hd {hd} L0 {L0} T {T}: {us:.1f} us/launch, {tf:.1f} TFLOP/s")
        for b in (k, v, q, o):
            b.free()
    return out


# prefill GEMM shapes: M prompt rows, K = 4096, N = 4096 (Q/O) and 14336 (gate/up)
# prompt shapes at K=4096, then the 8B model's other prefill GEMMs over a 2048-position slice:
# Q|K|V (N=6144), gate|up as one GEMM (N=28672) and down (K=14336)
GEMM_CASES = [(M, 4096, N) for M in (128, 512, 2048) for N in (4096, 14336)] + \
             [(2048, 4096, 6144), (2048, 4096, 28672), (2048, 14336, 4096)]
MFMA_F16_PEAK_TFLOPS = 2500.0


def gemm_roofline(tp, ctx, iters=20):
    """MFMA prefill GEMM Y[M,N] = X[M,K] . W[N,K]^T (W Q4_K) at GEMM_CASES, both activation modes:
    "q8k" (candle's arithmetic, the model's prefill) and "f16".  Each mode runs on fp16 MFMA
    (dense peak 2.5 PFLOP/s); flops per launch = 2 M N K; time = mean of the dispatch-stamped
    event intervals of `iters` launches after one untimed launch."""
    from tpthip import synth
    out = {}
    for M, K, N in GEMM_CASES:
        w = ctx.to_device(synth.random_weights(tp.TYPE_Q4_K, N, K, seed=N + 3, name=f"gemm{N}"))
        x = ctx.to_device(np.random.default_rng(M).standard_normal((M, K), dtype=np.float32))
        y = ctx.alloc(M * N * 4)
        for mode, act in (("q8k", tp.ACT_Q8), ("f16", tp.ACT_F16)):
            ctx.bench_gemm(tp.TYPE_Q4_K, w, x, y, M, K, N, 1, act=act)
            ms = ctx.bench_gemm(tp.TYPE_Q4_K, w, x, y, M, K, N, iters, act=act)
            us = ms * 1e3 / iters
            tf = 2.0 * M * N * K / (us * 1e-6) / 1e12
            out[f"{mode} {M}x{K}x{N}"] = {"us_per_launch": round(us, 2), "tflops": round(tf, 1),
                                          "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4)}
            log(f"gemm {mode} M={M} K={K} N={N}: {us:.1f} us/launch, {tf:.1f} TFLOP/s")
        for b in (w, x, y):
            b.free()
    return out


def host_cpu():
    """nproc, the threads this process may run on, and the CPU model (lscpu's "Model name")."""
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        allowed = len(os.sched_getaffinity(0))
    except AttributeError:
        allowed = os.cpu_count() or 1
    return os.cpu_count() or 1, allowed, model


def cpu_baseline(path, pos0, budget_s=20.0):
    """The oracle (candle's CPU decode restated: Q8_K activations, integer vec_dot, OpenMP over
    output columns) decoding the same model at the GPU run's positions: its f32 KV cache primed
    with pos0 synthetic positions (a real 2048-token CPU prefill would take minutes; the decode
    step's work depends on how many positions it reads, not on their values), then greedy steps
    for about budget_s seconds.  Threads: the CPU share this process is given (the affinity
    mask, capped by OMP_NUM_THREADS when set); nproc and the CPU model are recorded."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    nproc, allowed, model = host_cpu()
    threads = allowed
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
    m = oracle.Model(path)
    m.reset(pos0 + 512)
    m.prime_cache(pos0, SEED)
    rng = np.random.default_rng(SEED)
    tok = int(rng.integers(0, m.cfg["vocab"]))
    pos, n = pos0, 0
    tok = oracle.argmax(m.forward([tok], pos, threads))  # first step untimed (page-in)
    pos += 1
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s and pos < pos0 + 512:
        tok = oracle.argmax(m.forward([tok], pos, threads))
        pos += 1
        n += 1
    dt = time.perf_counter() - t0
    m.close()
    return {"value": round(n / dt, 4), "unit": "tok/s", "cores": threads, "kind": "port",
            "nproc": nproc, "cpu_model": model, "positions": [pos0 + 1, pos - 1],
            "sample": f"8B-shape Q4_K_M (the benchmark's model), f32 KV cache primed with {pos0} "
                      f"synthetic positions, then {n} timed greedy decode steps at positions "
                      f"{pos0 + 1}-{pos - 1} ({dt:.1f} s) on {threads} threads (nproc {nproc})"}


def traffic_from_profiles(shape):
    """HBM bytes per launch of the Q4_K GEMV at `shape` ("KxN"): FETCH_SIZE + WRITE_SIZE from
    the committed rocprofv3 PMC summary, each scaled by the copy-kernel calibration there (a
    line `hbm_bytes_per_launch KxN: <bytes>`); None when the summary is absent."""
    p = os.path.join(ROOT, "profiles", "gemv_q4k_pmc_traffic.md")
    if not os.path.exists(p):
        return None
    key = f"hbm_bytes_per_launch {shape}:"
    for line in open(p):
        line = line.strip().strip("`")
        if line.startswith(key):
            try:
                return int(line[len(key):].strip())
            except ValueError:
                return None
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="timed decode tokens")
    ap.add_argument("--warmup", type=int, default=16, help="untimed decode tokens")
    ap.add_argument("--prompt", type=int, default=PROMPT_LEN)
    ap.add_argument("--model", default="", help="existing GGUF (default: generate the 8B shape)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--leg", choices=["all", "gemv", "gemv-q6k-q80", "attn", "gemm", "causal", "decode"],
                    default="all",
                    help="gemv: only the GEMV roofline leg and the copy calibration (profiling); "
                         "gemv-q6k-q80: only the Q6_K and Q8_0 GEMV legs (profiling); "
                         "attn: only the decode-attention leg; gemm: only the prefill GEMM leg; "
                         "causal: only the prompt-attention leg; decode: only the end-to-end "
                         "prefill + decode run (profiling; no roofline or CPU legs)")
    ap.add_argument("--gemv-iters", type=int, default=256, help="timed launches per GEMV shape")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the path runs on a single MI355X; see DESIGN.md for how it would shard)",
              file=sys.stderr)
        sys.exit(2)

    import tpthip as tp
    from tpthip import synth

    ctx = tp.Context(0)
    log(f"device: {ctx.name}, {ctx.n_cu} CUs")
    if args.leg == "attn":
        print(json.dumps({"attn_decode": attn_roofline(tp, ctx), "copy": copy_calibration(ctx)}))
        return
    if args.leg == "gemm":
        print(json.dumps({"prefill_gemm": gemm_roofline(tp, ctx)}))
        return
    if args.leg == "causal":
        print(json.dumps({"prefill_attn": attn_causal_roofline(tp, ctx)}))
        return
    if args.leg == "gemv-q6k-q80":
        print(json.dumps({"gemv_q6k": gemv_roofline(tp, ctx, iters=64, qtype=tp.TYPE_Q6_K),
                          "gemv_q8_0": gemv_roofline(tp, ctx, iters=64, qtype=tp.TYPE_Q8_0),
                          "copy": copy_calibration(ctx)}))
        return
    decode_only = args.leg == "decode"
    if not decode_only:
        gemv = gemv_roofline(tp, ctx, iters=args.gemv_iters)
        if args.leg == "gemv":
            print(json.dumps({"gemv": gemv, "copy": copy_calibration(ctx)}))
            return
        gemv_q6k = gemv_roofline(tp, ctx, iters=64, qtype=tp.TYPE_Q6_K)
        gemv_q80 = gemv_roofline(tp, ctx, iters=64, qtype=tp.TYPE_Q8_0)
        attn = attn_roofline(tp, ctx)
        gemm = gemm_roofline(tp, ctx)
        causal = attn_causal_roofline(tp, ctx)

    tmpdir = tempfile.mkdtemp(prefix="tpt_bench_", dir=os.environ.get("TPT_BENCH_DIR") or None)
    path = args.model
    if not path:
        path = os.path.join(tmpdir, "llama3-8b-shape-q4_k_m.gguf")
        t0 = time.perf_counter()
        synth.write_llama(path, synth.LLAMA_8B, seed=SEED, nthreads=min(os.cpu_count() or 1, 16))
        log(f"generated {path} ({os.path.getsize(path) / 1e9:.2f} GB) in {time.perf_counter() - t0:.1f} s")
    try:
        eng = tp.HipEngine(0)
        t0 = time.perf_counter()
        info = eng.load(path)
        log(f"loaded {info.name} ({info.size_bytes / 1e9:.2f} GB) backend={info.backend} in "
            f"{time.perf_counter() - t0:.1f} s")
        m = eng  # noqa: F841
        desc_model = tp.Model  # noqa: F841
        rng = np.random.default_rng(SEED)
        prompt = rng.integers(0, 128256, args.prompt).tolist()
        # warm-up infer (graph capture, first-touch), then a cold cache for the timed run
        eng.infer(tp.greedy_params(prompt, args.warmup), lambda ev: None)
        eng.reset_cache()
        n_tok = [0]

        def on_tok(ev):
            if not ev.done:
                n_tok[0] += 1

        st = eng.infer(tp.greedy_params(prompt, args.steps), on_tok)
        assert st.generated == args.steps == n_tok[0], (st.generated, n_tok[0])
        decode_s = st.decode_ms / 1e3
        tok_s = args.steps / decode_s
        prefill_tok_s = len(prompt) / (st.ttft_ms / 1e3)
        # decode ceiling from the model's streamed bytes per token
        probe = tp.Model(ctx, path, max_ctx=64)
        bpt = probe.desc["decode_bytes_per_token"]
        probe.close()
        ceiling = HBM_PEAK_GBS * 1e9 / bpt
        kv_bpt = 32 * 2 * 8 * 128 * 2 * (len(prompt) + args.steps / 2)
        log(f"prefill {len(prompt)} tok in {st.ttft_ms:.0f} ms ({prefill_tok_s:.1f} tok/s); decode "
            f"{args.steps} tok in {st.decode_ms:.1f} ms = {tok_s:.1f} tok/s; ceiling {ceiling:.1f}")
        eng.close()
        cpu = None if (args.no_cpu or decode_only) else cpu_baseline(path, len(prompt))
    finally:
        if not args.model and os.path.exists(path):
            os.remove(path)
        try:
            os.rmdir(tmpdir)
        except OSError:
            pass

    if decode_only:
        print(json.dumps({"decode_tok_s": round(tok_s, 2), "ms_per_step": round(st.decode_ms / args.steps, 4),
                          "prefill_tok_s": round(prefill_tok_s, 2), "decode_ceiling_tok_s": round(ceiling, 1)}))
        return
    g = gemv["4096x14336"]
    line = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(st.decode_ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": "llama-3-8b-shape random-init GGUF Q4_K_M (token_embd/output Q6_K, "
                        "matrices Q4_K), bs=1, 2048-token seeded prompt then greedy decode "
                        "through the LlmEngine mirror",
            "prompt_tokens": len(prompt),
            "prefill_tok_s": round(prefill_tok_s, 2),
            "weight_bytes_per_token": bpt,
            "decode_ceiling_tok_s": round(ceiling, 1),
            "decode_frac_of_ceiling": round(tok_s / ceiling, 4),
            "decode_frac_of_ceiling_with_kv": round(tok_s / (HBM_PEAK_GBS * 1e9 / (bpt + kv_bpt)), 4),
            "arith": "q4_k/q6_k weights x q8_k activations: int8 dot4 -> int32, f32 block scales",
            "gemv_q4k": gemv,
            "gemv_q6k": gemv_q6k,
            "gemv_q8_0": gemv_q80,
            "attn_decode_f16": attn,
            "prefill_gemm_q4k": gemm,
            "prefill_attn_causal_f16": causal,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "gemv_q8_kernel<Q4_K> 4096->14336",
            "achieved": g["gbs"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(g["gbs"] / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profiles("4096x14336"),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
