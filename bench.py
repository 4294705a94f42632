#!/usr/bin/env python3
"""Benchmark of the speculative-decoding verify path on one MI355X.

Workload (default): a 32-layer d4096 MHA (32/32 heads), FFN 11008, vocab
32000 Q4_0 target verifies k = 8 drafts of a 22-layer d2048 GQA (32/4 heads,
head_dim 64, FFN 5632) Q4_0 draft, after a 2048-token prompt of uniform random
ids; sampled acceptance at T = 0.8, top_p = 1.0, seeded uniforms.  Weights are
seeded random-init N(0, 0.02^2) quantised with the reference's Q4_0 writer,
generated directly in HBM.

One step = decoding 256 tokens from the prefilled state (each step restarts
from the same state with uniforms of its own seed, so the figure averages
several acceptance traces of the same workload).  The value is the
emitted-token throughput of the timed steps (accepted drafts + the resampled
or bonus token of every round).

value: tok/s of the timed steps, run clean (no instrumentation).

roofline: the verify dequant-GEMMs of the target (M = k+1 rows), timed with
HIP events that the dispatch records on the target's stream around every 7th
GEMM launch of each class, in a separate instrumented pass of the same
workload after the timed steps; achieved = algorithmic bytes (Q4_0 weight
blocks + fp32 activations in + fp32 results out) / event time, where the time
includes the SwiGLU panel launch that prepares the down projection's input.

config also carries flat scalar figures: per verify GEMM class its average
launch time and HBM fraction (verify_<class>_us / _frac), the mix with and
without the SwiGLU panel, the draft's M = 1 GEMM fraction from the same
instrumented pass, and -- measured on the GPU after the timed work, without
the reference CPU legs of --mode configs -- the 4096x4096 Q4_0 M = 5 GEMM
(c1_gemm_us / _frac) and single verify steps of the 22L d2048 model at 512
positions (c3_verify_step_ms) and of the 28L d3584 V152064 model at 8192
positions (c5_verify_step_ms, with the acceptance kernels' c5_accept_ms).

cpu_baseline: the reference engine's own x86 build (oracle/_ref, built from
its sources by oracle/Makefile) on this host's cores: single-token forwards
of same-shape models at context 2048, combined with the acceptance trace of
the GPU run (the reference verifies one token per forward).

--mode gemm: the verify GEMMs of this workload in isolation.  --mode
configs: the isolated Q4_0/Q8_0 GEMMs at M = 1, 5, 9 (4096x4096, 11008x4096,
4096x11008) and single verify steps of a 22L d2048 model at 512 positions
(k=4, greedy) and of a 28L d3584 V152064 model at 8192 positions (k=8, T=1),
each beside the reference's x86 build.

--mode paths: the MFMA kernel against the dot-product kernel (v_dot2_f32_f16,
no MFMA) on plain panels, at M = k+1 (verify shapes) and M = 1 (draft shapes).

--mode traffic --fetch F.csv --write W.csv: HBM bytes per verify GEMM launch
from two rocprofv3 counter runs of --mode gemm (FETCH_SIZE, WRITE_SIZE).

Usage: python bench.py [--gpus 1] [--steps 5] [--warmup 1] [--mode spec|gemm|configs|paths|traffic]
"""
import argparse
import ctypes as C
import json
import os
import struct
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "tests"))

PEAK_HBM_GBS = 8000.0

TARGET = dict(n_layers=32, n_heads=32, n_kv_heads=32, n_embd=4096, n_ff=11008, n_vocab=32000)
DRAFT = dict(n_layers=22, n_heads=32, n_kv_heads=4, n_embd=2048, n_ff=5632, n_vocab=32000)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def load_product():
    import _native as N
    if not N.product_available():
        sys.exit("bench.py: engine library missing -- run python -c 'import __graft_entry__ as g; g.build()'")
    P = N.product()
    if P.vxh_init() != 0:
        sys.exit("bench.py: GPU init failed: " + P.vxh_last_error().decode())
    return N, P


def synth_model(N, P, shape, n_ctx, seed):
    cfg = N.VxModelConfig()
    for k, v in shape.items():
        setattr(cfg, k, v)
    cfg.n_ctx = n_ctx
    cfg.rope_theta = 10000.0
    spec = N.VxSynthSpec(seed=seed, std=0.02, matrix_type=2, embd_type=2, output_type=2)
    mp = C.POINTER(N.VxModelDev)()
    rc = P.vx_model_create_synthetic(C.byref(cfg), C.byref(spec), C.byref(mp))
    if rc != 0:
        sys.exit("bench.py: model creation failed: " + N.product_error())
    return mp


# ---------------------------------------------------------------------------
# CPU baseline: the reference engine (oracle/_ref) on same-shape GGUF files
# ---------------------------------------------------------------------------
def _gguf_stream(path, shape, rng, emb_type=2):
    """Writes a random Q4_0 Llama GGUF of the given shape, streaming; one
    layer's random blocks are reused by every layer (timing does not depend
    on the values).  emb_type 8: Q8_0 token embedding and output matrix."""
    d, F, V, L = shape["n_embd"], shape["n_ff"], shape["n_vocab"], shape["n_layers"]
    kvd = shape["n_kv_heads"] * (d // shape["n_heads"])

    def blocks(rows, cols, typ=2):
        nb = rows * cols // 32
        bb = 18 if typ == 2 else 34
        b = np.empty((nb, bb), np.uint8)
        b[:, :2] = (np.abs(rng.normal(0, 0.02, nb)).astype(np.float16)).view(np.uint8).reshape(nb, 2)
        b[:, 2:] = rng.integers(0, 256, (nb, bb - 2), dtype=np.uint8)
        if typ == 8:
            b[:, 2:][b[:, 2:] == 128] = 129          # int8 in [-127, 127]
        return b.tobytes()

    layer = {"attn_q": blocks(d, d), "attn_k": blocks(kvd, d), "attn_v": blocks(kvd, d),
             "attn_output": blocks(d, d), "ffn_gate": blocks(F, d), "ffn_up": blocks(F, d),
             "ffn_down": blocks(d, F)}
    dims = {"attn_q": (d, d), "attn_k": (d, kvd), "attn_v": (d, kvd), "attn_output": (d, d),
            "ffn_gate": (d, F), "ffn_up": (d, F), "ffn_down": (F, d)}
    emb = blocks(V, d, emb_type)
    ones = np.ones(d, np.float32).tobytes()
    tensors = [("token_embd.weight", emb_type, (d, V), emb)]
    for l in range(L):
        tensors.append((f"blk.{l}.attn_norm.weight", 0, (d,), ones))
        for nm in ("attn_q", "attn_k", "attn_v", "attn_output"):
            tensors.append((f"blk.{l}.{nm}.weight", 2, dims[nm], layer[nm]))
        tensors.append((f"blk.{l}.ffn_norm.weight", 0, (d,), ones))
        for nm in ("ffn_gate", "ffn_up", "ffn_down"):
            tensors.append((f"blk.{l}.{nm}.weight", 2, dims[nm], layer[nm]))
    tensors.append(("output_norm.weight", 0, (d,), ones))
    tensors.append(("output.weight", emb_type, (d, V), emb))

    def s(x):
        b = x.encode()
        return struct.pack("<Q", len(b)) + b
    kv = [("general.architecture", 8, "llama"), ("llama.block_count", 4, L),
          ("llama.attention.head_count", 4, shape["n_heads"]),
          ("llama.attention.head_count_kv", 4, shape["n_kv_heads"]),
          ("llama.embedding_length", 4, d), ("llama.feedforward_length", 4, F),
          ("llama.rope.freq_base", 6, 10000.0), ("llama.vocab_size", 4, V)]
    head = bytearray(struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(kv)))
    for k, t, v in kv:
        head += s(k) + struct.pack("<I", t)
        head += s(v) if t == 8 else (struct.pack("<f", v) if t == 6 else struct.pack("<I", v))
    off = 0
    offs = []
    for name, t, dm, data in tensors:
        offs.append(off)
        off = (off + len(data) + 31) // 32 * 32
    for (name, t, dm, data), o in zip(tensors, offs):
        head += s(name) + struct.pack("<I", len(dm)) + b"".join(struct.pack("<Q", x) for x in dm)
        head += struct.pack("<IQ", t, o)
    head += b"\0" * ((-len(head)) % 32)
    with open(path, "wb") as f:
        f.write(head)
        for (name, t, dm, data), o in zip(tensors, offs):
            f.write(data)
            f.write(b"\0" * ((-len(data)) % 32))


def _ref_forward_ms(N, R, path, n_tok, ctx, thread_counts):
    """Best of n_tok single-token forwards at context ctx for each thread
    count (tests/benchmark.c:21-50 takes the best of 5); the model is larger
    than the last-level cache, so every forward streams it from DRAM."""
    mp = C.POINTER(N.VxModel)()
    rc = R.vx_model_create(path.encode(), C.byref(mp))
    if rc != 0:
        raise RuntimeError(f"reference vx_model_create failed ({rc})")
    try:
        V = mp.contents.config.n_vocab
        lg = np.zeros(V, np.float32)
        R.vx_model_forward(mp, np.array([1], np.int32), 1, lg)     # allocates the KV cache
        best = {}
        for th in thread_counts:
            R.vx_set_n_threads(th)
            times = []
            for i in range(n_tok):
                mp.contents.cache_len = ctx                     # same context for every sample
                t0 = time.perf_counter()
                R.vx_model_forward(mp, np.array([(7 * i + 3) % V], np.int32), 1, lg)
                times.append(time.perf_counter() - t0)
            best[th] = 1e3 * float(np.min(times))
        return best
    finally:
        R.vx_model_destroy(mp)


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _tmpdir(need):
    import shutil
    for cand in ("/dev/shm", tempfile.gettempdir(), HERE):
        try:
            if os.access(cand, os.W_OK) and shutil.disk_usage(cand).free > need:
                return cand
        except OSError:
            pass
    raise RuntimeError(f"no directory with {need / 1e9:.0f} GB free for the reference's GGUF files")


def cpu_baseline(N, stats_emitted, stats_drafted, ctx, n_trials=5):
    """The reference's x86 build on this host: best of n_trials single-token
    forwards of each model at context ctx, with all threads and with one,
    turned into tok/s for the GPU run's acceptance trace (the reference
    verifies one draft token per forward, src/speculative.c:186-207)."""
    if not N.ref_available("avx2"):
        return None
    R = N.ref("avx2")
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    rng = np.random.default_rng(99)
    tmpdir = _tmpdir(6e9)
    t_start = time.perf_counter()
    counts = sorted({threads, 1}, reverse=True)
    with tempfile.TemporaryDirectory(dir=tmpdir) as td:
        tp, dp = os.path.join(td, "target.gguf"), os.path.join(td, "draft.gguf")
        _gguf_stream(tp, TARGET, rng)
        t_target = _ref_forward_ms(N, R, tp, n_trials, ctx, counts)
        os.remove(tp)
        _gguf_stream(dp, DRAFT, rng)
        t_draft = _ref_forward_ms(N, R, dp, n_trials, ctx, counts)
    R.vx_set_n_threads(threads)

    def tok_s(th):
        return 1e3 * stats_emitted / (stats_drafted * t_draft[th] + stats_emitted * t_target[th])
    cpu = _cpu_model()
    log(f"cpu baseline ({cpu}): target forward {t_target} ms, draft forward {t_draft} ms by thread count "
        f"({time.perf_counter() - t_start:.1f} s)")
    return {
        "value": round(tok_s(threads), 3),
        "unit": "tok/s",
        "cores": threads,
        "kind": "reference",
        "value_1_thread": round(tok_s(1), 3),
        "cpu_model": cpu,
        "sample": (f"reference x86 build (oracle/_ref/libvxref_avx2.so, -Ofast -mavx2 -mfma -fopenmp) on "
                   f"{cpu}: best of {n_trials} single-token forwards of same-shape random Q4_0 GGUFs at "
                   f"context {ctx}, {threads} threads (target {t_target[threads]:.1f} ms, draft "
                   f"{t_draft[threads]:.1f} ms) and 1 thread (target {t_target[1]:.1f} ms, draft "
                   f"{t_draft[1]:.1f} ms); tok/s = emitted / (drafted*t_draft + emitted*t_target) for the "
                   f"GPU run's acceptance trace ({stats_drafted} drafted, {stats_emitted} emitted over the "
                   f"timed steps)"),
    }


def read_traffic():
    """HBM bytes per verify-GEMM launch from the committed rocprof counter
    summary, when present (profiles/verify_gemm_traffic.txt)."""
    p = os.path.join(HERE, "profiles", "verify_gemm_traffic.txt")
    if not os.path.exists(p):
        return None
    for line in open(p):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":")[1])
    return None


# ---------------------------------------------------------------------------
def run_spec(args):
    N, P = load_product()
    name = C.create_string_buffer(256)
    P.vxh_device_name(name, 256)
    log("device:", name.value.decode())
    t0 = time.perf_counter()
    tm = synth_model(N, P, TARGET, 4096, 1001)
    dm = synth_model(N, P, DRAFT, 4096, 2002)
    log(f"models created in HBM: {time.perf_counter() - t0:.1f} s")
    if args.kv_half:
        # the flagged fp16 KV-cache mode of both models (not the headline
        # configuration: the reference keeps its cache in fp32)
        for m in (tm, dm):
            opt = N.VxModelOptions()
            P.vx_model_get_options(m, C.byref(opt))
            opt.kv_half = 1
            if P.vx_model_set_options(m, C.byref(opt)) != 0:
                sys.exit("bench.py: fp16 KV cache refused: " + N.product_error())
    st = P.vx_speculative_create(dm, tm, args.k)
    if not st:
        sys.exit("bench.py: vx_speculative_create failed")
    P.vx_speculative_set_temp(st, 0.8, 1.0)
    P.vx_speculative_set_seed(st, 4242)
    prompt = np.random.default_rng(7).integers(0, TARGET["n_vocab"], args.prompt).astype(np.int32)
    t0 = time.perf_counter()
    if P.vx_speculative_prefill(st, prompt, len(prompt)) != len(prompt):
        sys.exit("bench.py: prefill failed: " + N.product_error())
    P.vxh_device_sync()
    prefill_s = time.perf_counter() - t0
    log(f"prefill of {args.prompt} tokens (both models): {prefill_s:.2f} s")
    out = np.zeros(args.tokens, np.int32)
    for _ in range(args.warmup):
        if P.vx_speculative_decode(st, out, args.tokens) != args.tokens:
            sys.exit("bench.py: decode failed: " + N.product_error())
    # every timed step decodes from the prefilled state with uniforms of its
    # own seed: the acceptance trace of two unrelated random models moves
    # with any rounding change, so the figure averages several traces
    stats = N.VxSpecStats()

    def decode_steps(seeds):
        tot = dict(rounds=0, accepted=0, drafted=0, emitted=0, verify_ms=0.0, draft_ms=0.0)
        elapsed = 0.0
        for seed in seeds:
            P.vx_speculative_set_seed(st, seed)
            t0 = time.perf_counter()
            n = P.vx_speculative_decode(st, out, args.tokens)
            P.vxh_device_sync()
            elapsed += time.perf_counter() - t0
            if n != args.tokens:
                sys.exit("bench.py: decode failed: " + N.product_error())
            P.vx_speculative_get_stats(st, C.byref(stats))
            for key in tot:
                tot[key] += getattr(stats, key)
        return tot, elapsed
    # the headline: a clean pass, no instrumentation
    P.vxh_device_sync()
    tot, elapsed = decode_steps([4243 + i for i in range(args.steps)])
    value = args.steps * args.tokens / elapsed
    # the roofline: a separate pass of the same workload with kernel-execution
    # events around every --prof-every-th verify GEMM of each class (7: a
    # stride that walks through the 32 layers; a launch with events costs
    # ~18 us of host time, so this pass is not the one timed above)
    P.vx_model_set_profiling(tm, args.prof_every)
    P.vx_model_set_profiling(dm, args.prof_every)
    P.vxh_device_sync()
    tot_p, elapsed_p = decode_steps([4243 + i for i in range(args.prof_steps)])
    prof = (N.VxGemmProfile * N.VX_PROF_N)()
    prof_d = (N.VxGemmProfile * N.VX_PROF_N)()
    P.vx_model_get_profile(tm, prof)
    P.vx_model_get_profile(dm, prof_d)
    P.vx_model_set_profiling(tm, 0)
    P.vx_model_set_profiling(dm, 0)
    log(f"instrumented pass: {args.prof_steps * args.tokens / elapsed_p:.1f} tok/s over {args.prof_steps} steps")
    names = ["qkv", "attn_out", "gate_up", "down", "output", "swiglu_panel"]
    gemm = prof[:5]
    ms_gemm = sum(p.ms for p in gemm)
    ms = ms_gemm + prof[5].ms           # the SwiGLU panel feeding down counted in the mix
    byt = sum(p.bytes for p in gemm)
    launches = sum(p.launches for p in gemm)
    achieved = byt / (ms * 1e-3) / 1e9 if ms > 0 else 0.0
    achieved_gemm = byt / (ms_gemm * 1e-3) / 1e9 if ms_gemm > 0 else 0.0
    ms_d = sum(p.ms for p in prof_d[:5])
    draft_gbs = sum(p.bytes for p in prof_d[:5]) / (ms_d * 1e-3) / 1e9 if ms_d > 0 else 0.0
    breakdown = {nm: {"launches": p.launches, "avg_us": round(1e3 * p.ms / max(p.launches, 1), 2),
                      "GB/s": round(p.bytes / (p.ms * 1e-3) / 1e9, 1) if p.ms > 0 else None}
                 for nm, p in zip(names, prof)}
    flat = {}
    for nm, p in zip(names, prof):
        flat[f"verify_{nm}_us"] = round(1e3 * p.ms / max(p.launches, 1), 2)
        if nm != "swiglu_panel":
            flat[f"verify_{nm}_frac"] = round(p.bytes / (p.ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4) if p.ms > 0 else None
    flat["verify_gemm_mix_frac"] = round(achieved / PEAK_HBM_GBS, 4)
    flat["verify_gemm_only_frac"] = round(achieved_gemm / PEAK_HBM_GBS, 4)
    for nm, p in zip(names[:5], prof_d[:5]):
        flat[f"draft_{nm}_us"] = round(1e3 * p.ms / max(p.launches, 1), 2)
        flat[f"draft_{nm}_frac"] = round(p.bytes / (p.ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4) if p.ms > 0 else None
    flat["draft_gemm_frac"] = round(draft_gbs / PEAK_HBM_GBS, 4)
    flat["draft_gemm_avg_us"] = round(1e3 * ms_d / max(sum(p.launches for p in prof_d[:5]), 1), 2)
    log(f"decode: {value:.1f} tok/s; rounds {tot['rounds']}, accepted {tot['accepted']}/{tot['drafted']}; "
        f"verify {tot['verify_ms']:.1f} ms, draft {tot['draft_ms']:.1f} ms over {args.steps} steps")
    log("verify GEMMs:", json.dumps(breakdown))
    cpu = None
    if not args.no_cpu_baseline:
        try:
            cpu = cpu_baseline(N, tot["emitted"], tot["drafted"], args.prompt)
        except Exception as e:   # reported, the GPU figure stands on its own
            log("cpu baseline failed:", repr(e))
    P.vx_speculative_destroy(st)
    P.vx_model_destroy(tm)
    P.vx_model_destroy(dm)
    if not args.no_configs:
        # the other configurations' figures (GPU only, after the timed work)
        L = _bind_gemm(N, P)
        c1 = _configs_gemm(N, P, L, args, None, 0, cases=[("C1", 4096, 4096, 2, 5)])[0]
        c3 = _configs_verify(N, P, L, "C3", C3_SHAPE, 512, 4, 0.0, 2, 10, None, 0)
        c5 = _configs_verify(N, P, L, "C5", C5_SHAPE, 8192, 8, 1.0, 8, 5, None, 0)
        flat.update({"c1_gemm_us": c1["gemm_us"], "c1_gemm_frac": c1["frac"],
                     "c3_verify_step_ms": c3["verify_step_ms"], "c3_accept_ms": c3["accept_ms"],
                     "c5_verify_step_ms": c5["verify_step_ms"], "c5_accept_ms": c5["accept_ms"]})
    line = {
        "metric": "accepted tok/s (7B-shape Q4_0, k=8); verify dequant-GEMM HBM GB/s % of peak",
        "value": round(value, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * elapsed / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded random-init Q4_0 weights, uniform random prompt ids)",
        "config": {
            "workload": (f"speculative decode: 32L d4096 32/32-head FFN11008 V32000 Q4_0 target verifies "
                         f"k={args.k} drafts of a 22L d2048 32/4-head FFN5632 Q4_0 draft; prompt "
                         f"{args.prompt}, {args.tokens} tokens per step, T=0.8 top_p=1.0"),
            "k": args.k, "prompt": args.prompt, "tokens_per_step": args.tokens,
            "kv_cache": "f16 (flagged mode)" if args.kv_half else "f32",
            "acceptance_rate": round(tot["accepted"] / max(tot["drafted"], 1), 4),
            "rounds_per_step": round(tot["rounds"] / args.steps, 1),
            "seeds": f"uniform seeds 4243..{4242 + args.steps}, one per step",
            "verify_ms_per_round": round(tot["verify_ms"] / max(tot["rounds"], 1), 3),
            "draft_ms_per_round": round(tot["draft_ms"] / max(tot["rounds"], 1), 3),
            "prefill_s": round(prefill_s, 3),
            **flat,
            "verify_gemms": breakdown,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": read_traffic(),
            "kernel": (f"verify dequant-GEMMs at M={args.k + 1} (Q4_0: vx_vg_kernel for attn_out, down and "
                       f"the output matrix, vx_gemm_kernel for qkv and gate_up) with the SwiGLU panel launch "
                       f"that feeds down counted in the time; every {args.prof_every}th launch of each class "
                       f"(kernel-execution events), in a separate instrumented pass of {args.prof_steps} "
                       f"steps after the timed ones"),
            "launches": launches,
            "avg_launch_us": round(1e3 * ms / max(launches, 1), 3),
            "bytes_per_launch": round(byt / max(launches, 1)),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


class _Panel(C.Structure):
    _fields_ = [("data", C.c_void_p), ("corr", C.c_void_p), ("rscale", C.c_void_p), ("xs", C.c_void_p),
                ("M", C.c_int), ("K", C.c_int), ("avx2", C.c_int), ("rs_ld", C.c_int)]


class _QMat(C.Structure):
    _fields_ = [("type", C.c_int), ("n_rows", C.c_int), ("n_cols", C.c_int), ("n_pairs", C.c_int),
                ("qs", C.c_void_p), ("d", C.c_void_p), ("cached", C.c_int),
                ("tq", C.c_void_p), ("td", C.c_void_p)]


class _Pro(C.Structure):
    _fields_ = [("kind", C.c_int), ("x", C.c_void_p), ("ldx", C.c_int), ("src", C.c_void_p),
                ("ld_src", C.c_int), ("w", C.c_void_p), ("x_out", C.c_void_p), ("ld_xout", C.c_int),
                ("ss", C.c_void_p), ("ss_in", C.c_void_p), ("ss_K", C.c_int), ("thr", C.c_float),
                ("clear", C.c_void_p), ("n_clear", C.c_size_t), ("part", C.c_void_p), ("n_chunks", C.c_int),
                ("n_heads", C.c_int), ("n_kv_heads", C.c_int), ("head_dim", C.c_int)]


PRO_ROWS, PRO_RESID, PRO_SWIGLU = 1, 2, 3


def _bind_gemm(N, P):
    vp = C.c_void_p
    L = N.bind_vxh(P)
    L.vxh_qmat_alloc.argtypes = [vp, C.c_int, C.c_int, C.c_int]
    L.vxh_synth_blocks.argtypes = [vp, C.c_int, C.c_int, C.c_int, C.c_uint64, C.c_float, vp]
    L.vxh_qmat_set_rows.argtypes = [vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, vp]
    L.vxh_gemm_pro.argtypes = [vp, C.c_int, vp, vp, C.c_int, C.c_int, C.c_float, vp, vp, vp]
    L.vxh_acc_store.argtypes = [vp, C.c_int, C.c_int, C.c_int, vp, C.c_int, vp, C.c_int, vp]
    L.vxh_qmat_free.argtypes = [vp]
    L.vxh_panel_alloc.argtypes = [vp, C.c_int, C.c_int]
    L.vxh_panel_free.argtypes = [vp]
    L.vxh_swiglu_panel_norm.argtypes = [vp, C.c_int, C.c_int, C.c_int, C.c_float, vp, C.c_int, vp, C.c_size_t,
                                        vp, vp]
    L.vxh_gemm_acc.argtypes = [vp, vp, C.c_int, vp, C.c_int, C.c_int, C.c_float, vp, C.c_int, C.c_float,
                               C.c_int, vp]
    L.vxh_event_create.argtypes = [vp]
    L.vxh_event_destroy.argtypes = [vp]
    L.vxh_event_record.argtypes = [vp, vp]
    L.vxh_event_elapsed_ms.argtypes = [vp, vp, vp]
    L.vxh_copy.argtypes = [vp, vp, C.c_size_t, vp]
    return L


def _rotated_mats(N, L, qt, rows, cols, seed0=1000):
    """Enough copies of a seeded random matrix (> 300 MB together) that a
    loop over them streams from HBM, not from the 256 MB Infinity Cache."""
    mat_bytes = rows * cols // 32 * (18 if qt == 2 else 34)
    n_rot = max(2, int(np.ceil(300e6 / mat_bytes)))
    mats = []
    stage = N.DevBuf(L, nbytes=mat_bytes)
    for i in range(n_rot):
        q = _QMat()
        assert L.vxh_qmat_alloc(C.byref(q), qt, rows, cols) == 0, L.vxh_last_error()
        assert L.vxh_synth_blocks(stage.ptr, qt, rows, cols, seed0 + i, 0.02, None) == 0
        assert L.vxh_qmat_set_rows(C.byref(q), stage.ptr, 1, rows, rows, 0, 0, None) == 0
        mats.append(q)
    stage.free()
    return mats, mat_bytes


def _time_loop(L, reps, body):
    """Device time of reps passes of body() between two events on the
    default stream, in ms."""
    e0, e1 = C.c_void_p(), C.c_void_p()
    L.vxh_event_create(C.byref(e0))
    L.vxh_event_create(C.byref(e1))
    L.vxh_device_sync()
    L.vxh_event_record(e0, None)
    for _ in range(reps):
        body()
    L.vxh_event_record(e1, None)
    ms = C.c_float()
    assert L.vxh_event_elapsed_ms(e0, e1, C.byref(ms)) == 0, L.vxh_last_error()
    L.vxh_event_destroy(e0)
    L.vxh_event_destroy(e1)
    return ms.value


def run_gemm(args):
    """Isolated verify GEMM kernels at M = k+1 on the 7B shapes, each with the
    input the verify forward gives it (vxh_gemm_pro: residual add + norm
    weight for QKV and gate/up, attention rows for the output projection, norm
    weight for the logits; down: a plain panel made once by
    vxh_swiglu_panel_norm, then vxh_gemm_acc), weights rotated over > 300 MB so
    the Infinity Cache does not serve them."""
    N, P = load_product()
    import ctypes as CC
    L = _bind_gemm(N, P)
    QMat, Pro = _QMat, _Pro
    M = args.k + 1
    results = []
    # calibration for rocprofv3 byte counters: a device-to-device copy of a
    # known size (FETCH_SIZE and WRITE_SIZE of that copy should read 256 MiB)
    cal_bytes = 256 << 20
    ca, cb = N.DevBuf(L, nbytes=cal_bytes), N.DevBuf(L, nbytes=cal_bytes)
    for _ in range(3):
        assert L.vxh_copy(cb.ptr, ca.ptr, cal_bytes, None) == 0
    L.vxh_device_sync()
    log(json.dumps({"calibration_copy_bytes": cal_bytes, "copies": 3}))
    ca.free()
    cb.free()
    kinds = {(4096, 4096): PRO_ROWS, (12288, 4096): PRO_RESID, (4096, 11008): PRO_SWIGLU,
             (22016, 4096): PRO_RESID, (32000, 4096): PRO_ROWS, (11008, 4096): PRO_RESID}
    rng = np.random.default_rng(1)
    for rows, cols, qt in ((4096, 4096, 2), (12288, 4096, 2), (4096, 11008, 2), (22016, 4096, 2),
                           (32000, 4096, 2), (11008, 4096, 8), (4096, 11008, 8)):
        mats, mat_bytes = _rotated_mats(N, L, qt, rows, cols)
        kind = kinds[(rows, cols)]
        ld_src = (cols + 15) // 16 * 32 if kind == PRO_SWIGLU else cols
        bufs = [N.DevBuf(L, rng.normal(0, 1, (M, cols)).astype(np.float32)),     # x
                N.DevBuf(L, rng.normal(0, 1, (M, ld_src))),                       # src
                N.DevBuf(L, rng.normal(1, 0.1, cols).astype(np.float32)),        # w
                N.DevBuf(L, nbytes=4 * M * cols),                                 # x_out
                N.DevBuf(L, np.zeros(16, np.float64)),                            # ss
                N.DevBuf(L, rng.uniform(100, 1000, 16))]                          # ss_in
        pro = Pro(kind=kind)
        if kind in (PRO_ROWS, PRO_RESID):
            pro.x, pro.ldx, pro.w, pro.ss = bufs[0].ptr, cols, bufs[2].ptr, bufs[4].ptr
        if kind == PRO_RESID:
            pro.src, pro.ld_src, pro.x_out, pro.ld_xout = bufs[1].ptr, cols, bufs[3].ptr, cols
        if kind == PRO_SWIGLU:
            pro.src, pro.ld_src, pro.ss_in, pro.ss_K, pro.thr = bufs[1].ptr, ld_src, bufs[5].ptr, 4096, 0.01
        acc = N.DevBuf(L, np.zeros(M * rows, np.float64))
        panel = None
        if kind == PRO_SWIGLU:
            # the verify forward's down projection: SwiGLU panel once, then a plain-panel GEMM
            panel = _Panel()
            assert L.vxh_panel_alloc(CC.byref(panel), M, cols) == 0, L.vxh_last_error()
            assert L.vxh_swiglu_panel_norm(bufs[1].ptr, ld_src, M, cols, 0.01, bufs[5].ptr, 4096, None, 0,
                                           CC.byref(panel), None) == 0, L.vxh_last_error()

        def launch(q):
            if panel is not None:
                return L.vxh_gemm_acc(CC.byref(q), CC.byref(panel), M, acc.ptr, rows, rows, 1.0, None, 0, 0.0,
                                      0, None)
            return L.vxh_gemm_pro(CC.byref(q), M, CC.byref(pro), acc.ptr, rows, rows, 1.0, None, None, None)
        for q in mats:
            assert launch(q) == 0, L.vxh_last_error()
        reps = args.steps * 10

        def one_pass():
            for q in mats:
                launch(q)
        ms = _time_loop(L, reps, one_pass)
        n = reps * len(mats)
        avg_us = 1e3 * ms / n
        alg = mat_bytes + 4 * M * cols + 4 * M * rows
        gbs = alg / (avg_us * 1e-6) / 1e9
        results.append({"shape": f"{'Q4_0' if qt == 2 else 'Q8_0'} {rows}x{cols} M={M}",
                        "prologue": {PRO_ROWS: "rows", PRO_RESID: "resid", PRO_SWIGLU: "swiglu panel"}[kind],
                        "avg_us": round(avg_us, 2), "GB/s": round(gbs, 1),
                        "frac": round(gbs / PEAK_HBM_GBS, 4)})
        log(json.dumps(results[-1]))
        for b in bufs + [acc]:
            b.free()
        if panel is not None:
            L.vxh_panel_free(CC.byref(panel))
        for q in mats:
            L.vxh_qmat_free(CC.byref(q))
    print(json.dumps({"mode": "gemm", "M": M, "results": results}), flush=True)



def run_paths(args):
    """The MFMA kernel against the dot-product kernel (VXH_PATH_DOT) on the
    same plain panels: the target's verify GEMMs at M = k+1 and the draft's
    decode GEMMs at M = 1, weights rotated over > 300 MB.  Times are device
    time per launch between events (run under rocprofv3 --kernel-trace for
    the kernels' own durations)."""
    N, P = load_product()
    import ctypes as CC
    L = _bind_gemm(N, P)
    L.vxh_prep_panel.argtypes = [CC.c_void_p, CC.c_void_p, CC.c_int, CC.c_int, CC.c_int, CC.c_int,
                                 CC.c_void_p, CC.c_int, CC.c_void_p]
    rng = np.random.default_rng(3)
    cases = [(args.k + 1, r, c) for r, c in ((4096, 4096), (12288, 4096), (4096, 11008), (22016, 4096),
                                             (32000, 4096))]
    cases += [(1, r, c) for r, c in ((2560, 2048), (2048, 2048), (11264, 2048), (2048, 5632), (32000, 2048))]
    results = []
    for M, rows, cols in cases:
        mats, mat_bytes = _rotated_mats(N, L, 2, rows, cols)
        x = N.DevBuf(L, rng.normal(0, 1, (M, cols)).astype(np.float32))
        pan = _Panel()
        assert L.vxh_panel_alloc(CC.byref(pan), M, cols) == 0, L.vxh_last_error()
        assert L.vxh_prep_panel(CC.byref(pan), x.ptr, cols, M, cols, 0, None, 0, None) == 0, L.vxh_last_error()
        acc = N.DevBuf(L, np.zeros(M * rows, np.float64))
        row = {"shape": f"Q4_0 {rows}x{cols} M={M}"}
        for name, path in (("mfma", 1), ("dot", 2)):
            def one_pass():
                for q in mats:
                    L.vxh_gemm_acc(CC.byref(q), CC.byref(pan), M, acc.ptr, rows, rows, 1.0, None, 0, 0.0, path, None)
            assert L.vxh_gemm_acc(CC.byref(mats[0]), CC.byref(pan), M, acc.ptr, rows, rows, 1.0, None, 0, 0.0,
                                  path, None) == 0, L.vxh_last_error()
            reps = args.steps * 10
            ms = _time_loop(L, reps, one_pass)
            us = 1e3 * ms / (reps * len(mats))
            row[name + "_us"] = round(us, 2)
            row[name + "_GB/s"] = round((mat_bytes + 4 * M * cols + 4 * M * rows) / (us * 1e-6) / 1e9, 1)
        row["mfma_speedup"] = round(row["dot_us"] / row["mfma_us"], 2)
        log(json.dumps(row))
        results.append(row)
        x.free()
        acc.free()
        L.vxh_panel_free(CC.byref(pan))
        for q in mats:
            L.vxh_qmat_free(CC.byref(q))
    print(json.dumps({"mode": "paths", "results": results}), flush=True)


# ---------------------------------------------------------------------------
# HBM traffic per verify GEMM from rocprofv3 counters (no GPU needed)
# ---------------------------------------------------------------------------
GEMM_SHAPES = [("Q4_0 4096x4096", 4096, 4096, 18), ("Q4_0 12288x4096", 12288, 4096, 18),
               ("Q4_0 4096x11008", 4096, 11008, 18), ("Q4_0 22016x4096", 22016, 4096, 18),
               ("Q4_0 32000x4096", 32000, 4096, 18), ("Q8_0 11008x4096", 11008, 4096, 34),
               ("Q8_0 4096x11008", 4096, 11008, 34)]
VERIFY_MIX = {"Q4_0 12288x4096": 32, "Q4_0 4096x4096": 32, "Q4_0 22016x4096": 32,
              "Q4_0 4096x11008": 32, "Q4_0 32000x4096": 1}


def run_traffic(args):
    """Post-processes two `rocprofv3 --pmc` runs of `--mode gemm` (one with
    FETCH_SIZE, one with WRITE_SIZE; KiB per dispatch) into HBM bytes per
    launch of each verify GEMM.  Each counter is scaled by what it reads for
    the 256 MiB device-to-device calibration copy that --mode gemm runs
    first; GEMM dispatches are grouped by (kernel, grid size), one group per
    shape in the order --mode gemm runs them.  The verify-step figure is the
    launch-weighted mean over one target forward at M = k+1: 32 layers x
    (QKV, O, gate/up, down) + the output projection."""
    import csv
    from collections import OrderedDict
    M = args.k + 1
    cal_bytes = 256 << 20

    def load(path, counter):
        groups, cal = OrderedDict(), []
        with open(path) as f:
            for d in csv.DictReader(f):
                if d.get("Counter_Name") != counter:
                    continue
                name, v = d["Kernel_Name"], float(d["Counter_Value"]) * 1024.0
                if name.startswith("__amd_rocclr_copyBuffer") and v > cal_bytes / 2:
                    cal.append(v)
                elif name.startswith("void vx_gemm_kernel") or name.startswith("void vx_vg_kernel"):
                    groups.setdefault((name.split("(")[0], d["Grid_Size"]), []).append(v)
        return groups, cal
    fetch, fcal = load(args.fetch, "FETCH_SIZE")
    write, wcal = load(args.write, "WRITE_SIZE")
    ff = cal_bytes / (sum(fcal) / len(fcal))
    wf = cal_bytes / (sum(wcal) / len(wcal))
    print(f"calibration: copy of {cal_bytes} B reads FETCH {sum(fcal) / len(fcal):.0f} B (factor {ff:.4f}), "
          f"WRITE {sum(wcal) / len(wcal):.0f} B (factor {wf:.4f})")
    keys = list(fetch.keys())
    if len(keys) != len(GEMM_SHAPES):
        sys.exit(f"expected {len(GEMM_SHAPES)} GEMM groups, found {len(keys)}: {keys}")
    per, alg = {}, {}
    print(f"{'shape (M=%d)' % M:18s} {'kernel':40s} {'launches':>8s} {'alg MB':>8s} {'fetch MB':>9s} "
          f"{'write MB':>9s} {'traffic/alg':>11s}")
    for (shape, r, c, bpb), key in zip(GEMM_SHAPES, keys):
        fv = sum(fetch[key]) / len(fetch[key]) * ff
        wv = sum(write.get(key, [0.0])) / max(1, len(write.get(key, []))) * wf
        alg[shape] = r * c // 32 * bpb + 4 * M * c + 4 * M * r
        per[shape] = fv + wv
        print(f"{shape:18s} {key[0][5:45]:40s} {len(fetch[key]):8d} {alg[shape] / 1e6:8.2f} {fv / 1e6:9.2f} "
              f"{wv / 1e6:9.2f} {(fv + wv) / alg[shape]:11.3f}")
    n = sum(VERIFY_MIX.values())
    t = sum(per[s] * c for s, c in VERIFY_MIX.items()) / n
    a = sum(alg[s] * c for s, c in VERIFY_MIX.items()) / n
    print(f"verify mix (32 x QKV/O/gate-up/down + output, M={M}): algorithmic {a:.0f} B/launch")
    print(f"traffic_bytes_per_launch: {t:.0f}")

# ---------------------------------------------------------------------------
# the other benchmark configurations: isolated GEMMs and single verify steps
# ---------------------------------------------------------------------------
C3_SHAPE = dict(n_layers=22, n_heads=32, n_kv_heads=4, n_embd=2048, n_ff=5632, n_vocab=32000)
C5_SHAPE = dict(n_layers=28, n_heads=28, n_kv_heads=4, n_embd=3584, n_ff=18944, n_vocab=152064)


def _cpu_gemv_ms(N, R, qt, rows, cols, reps=3):
    """The reference's matrix-vector product for one activation row
    (src/model.c:203-241 on its x86 build): vx_gemv_q4_0_avx2 for Q4_0; for
    Q8_0 the whole matrix is dequantised (vx_dequantize_row_q8_0) and
    vx_gemv_f32_avx2 runs on it, every call.  Median of reps, in ms."""
    rng = np.random.default_rng(rows + cols + qt)
    W = N.rand_q4_0(rng, rows, cols) if qt == 2 else N.rand_q8_0(rng, rows, cols)
    x = np.zeros(cols + 8, np.float32)
    x[:cols] = rng.normal(0, 1, cols)
    y = np.zeros(rows, np.float32)
    tmp = np.zeros(rows * cols, np.float32) if qt == 8 else None
    times = []
    for _ in range(reps + 1):
        t0 = time.perf_counter()
        if qt == 2:
            R.vx_gemv_q4_0_avx2(N._ptr(W), x, y, rows, cols)
        else:
            R.vx_dequantize_row_q8_0(N._ptr(W), tmp, rows * cols)
            R.vx_gemv_f32_avx2(y, tmp, x, rows, cols)
        times.append(time.perf_counter() - t0)
    return 1e3 * float(np.median(times[1:]))


def _configs_gemm(N, P, L, args, R, threads, cases=None):
    """C1 / C2: Y[M][rows] = X[M][cols] . W^T from device-resident fp32 rows,
    W rotated over > 300 MB.  gemm_us: the GEMM kernel alone (vxh_gemm_pro,
    panel built from the fp32 rows in its prologue, fp64 accumulator);
    op_us: GEMM + the store kernel that rounds the accumulator to the fp32
    result and clears it (vxh_acc_store)."""
    cases = cases or [("C1", 4096, 4096, 2, 5)] + [
        ("C2", r, c, t, m) for (r, c) in ((11008, 4096), (4096, 11008)) for t in (2, 8) for m in (1, 5, 9)]
    out = []
    cpu_cache = {}
    rng = np.random.default_rng(5)
    for cfg, rows, cols, qt, M in cases:
        mats, mat_bytes = _rotated_mats(N, L, qt, rows, cols)
        x = N.DevBuf(L, rng.normal(0, 1, (M, cols)).astype(np.float32))
        y = N.DevBuf(L, nbytes=4 * M * rows)
        acc = N.DevBuf(L, np.zeros(M * rows, np.float64))
        pro = _Pro(kind=PRO_ROWS, x=x.ptr, ldx=cols)

        def gemm(q):
            return L.vxh_gemm_pro(C.byref(q), M, C.byref(pro), acc.ptr, rows, rows, 1.0, None, None, None)

        def store():
            return L.vxh_acc_store(acc.ptr, rows, M, rows, y.ptr, rows, None, 0, None)
        for q in mats:
            assert gemm(q) == 0 and store() == 0, L.vxh_last_error()
        reps = max(10, args.steps * 10)

        def p_gemm():
            for q in mats:
                gemm(q)

        def p_op():
            for q in mats:
                gemm(q)
                store()
        n = reps * len(mats)
        g_us = 1e3 * _time_loop(L, reps, p_gemm) / n
        store()
        o_us = 1e3 * _time_loop(L, reps, p_op) / n
        alg = mat_bytes + 4 * M * cols + 4 * M * rows
        gbs = alg / (g_us * 1e-6) / 1e9
        r = {"config": cfg, "shape": f"{'Q4_0' if qt == 2 else 'Q8_0'} {rows}x{cols}", "M": M,
             "gemm_us": round(g_us, 2), "op_us": round(o_us, 2), "GB/s": round(gbs, 1),
             "frac": round(gbs / PEAK_HBM_GBS, 4), "bytes": alg}
        if R is not None:
            key = (qt, rows, cols)
            if key not in cpu_cache:
                cpu_cache[key] = _cpu_gemv_ms(N, R, qt, rows, cols)
            r["cpu_ref_us"] = round(1e3 * M * cpu_cache[key], 1)
            r["gpu_vs_cpu"] = round(1e3 * M * cpu_cache[key] / o_us, 1)
        log(json.dumps(r))
        out.append(r)
        for b in (x, y, acc):
            b.free()
        for q in mats:
            L.vxh_qmat_free(C.byref(q))
    return out


def _configs_verify(N, P, L, name, shape, ctx, k, T, emb_type, reps, R, threads):
    """One verify step of k drafts against ctx prefilled positions: the
    target forward of k+1 tokens through the public entry point
    (vx_model_verify, all k+1 logit rows copied to the host), and the
    acceptance kernels on those logits (vxh_row_stats_mc + vxh_accept_mc; greedy
    at T = 0, else sampled with seeded uniforms against random draft logits
    whose nucleus descriptors vxh_sample wrote).  Medians over reps steps,
    each rolled back to ctx with vx_model_kv_truncate."""
    V = shape["n_vocab"]
    cfg = N.VxModelConfig()
    for kk, v in shape.items():
        setattr(cfg, kk, v)
    cfg.n_ctx = ctx + 16
    cfg.rope_theta = 10000.0
    spec = N.VxSynthSpec(seed=77, std=0.02, matrix_type=2, embd_type=emb_type, output_type=emb_type)
    mp = C.POINTER(N.VxModelDev)()
    t0 = time.perf_counter()
    if P.vx_model_create_synthetic(C.byref(cfg), C.byref(spec), C.byref(mp)) != 0:
        sys.exit("bench.py: model creation failed: " + N.product_error())
    rng = np.random.default_rng(11)
    lg = np.zeros(V, np.float32)
    if P.vx_model_forward(mp, rng.integers(0, V, ctx).astype(np.int32), ctx, lg) != 0:
        sys.exit("bench.py: prefill failed: " + N.product_error())
    log(f"{name}: model + prefill of {ctx} positions {time.perf_counter() - t0:.1f} s")
    logits = np.zeros((k + 1, V), np.float32)
    times = []
    for i in range(reps + 2):
        toks = rng.integers(0, V, k + 1).astype(np.int32)
        t0 = time.perf_counter()
        if P.vx_model_verify(mp, toks, k + 1, logits) != 0:
            sys.exit("bench.py: verify failed: " + N.product_error())
        times.append(time.perf_counter() - t0)
        P.vx_model_kv_truncate(mp, ctx)
    fwd_ms = 1e3 * float(np.median(times[2:]))
    P.vx_model_destroy(mp)
    # acceptance kernels on the last verify's logits
    dL = N.DevBuf(L, logits)
    D = rng.normal(0, 2.0, (k, V)).astype(np.float32)
    dD = N.DevBuf(L, D)
    dstats = N.DevBuf(L, nbytes=4 * 3 * (k + 1))
    dnuc = N.DevBuf(L, nbytes=4 * 8 * k)
    ddr = N.DevBuf(L, toks[1:].copy())
    du = N.DevBuf(L, rng.random(k + 1).astype(np.float32))
    dtok = N.DevBuf(L, nbytes=4)
    dout = N.DevBuf(L, nbytes=4 * (k + 3))
    for j in range(k):
        assert L.vxh_sample(C.c_void_p(dD.ptr.value + 4 * j * V), V, T, 1.0, du.ptr, dtok.ptr,
                            C.c_void_p(dnuc.ptr.value + 32 * j), None) == 0, L.vxh_last_error()

    ws = N.VxhVocabWs()
    assert L.vxh_vocab_ws_alloc(C.byref(ws), k + 1) == 0, L.vxh_last_error()

    def accept():
        L.vxh_row_stats_mc(dL.ptr, V, k + 1, V, T, dstats.ptr, C.byref(ws), None)
        L.vxh_accept_mc(dL.ptr, V, V, dstats.ptr, dD.ptr, V, V, dnuc.ptr, ddr.ptr, k, T, du.ptr, dout.ptr,
                        C.byref(ws), None)
    accept()
    acc_ms = _time_loop(L, 50, accept) / 50
    L.vxh_vocab_ws_free(C.byref(ws))
    res = dout.get(np.int32, k + 3)
    for b in (dL, dD, dstats, dnuc, ddr, du, dtok, dout):
        b.free()
    r = {"config": name,
         "workload": (f"{shape['n_layers']}L d{shape['n_embd']} {shape['n_heads']}/{shape['n_kv_heads']} heads "
                      f"FFN{shape['n_ff']} V{V} Q4_0 (embedding/output {'Q8_0' if emb_type == 8 else 'Q4_0'}), "
                      f"{ctx} prefilled positions (attention cap 4096), k={k}, "
                      f"{'greedy' if T <= 0 else f'sampled T={T}'}"),
         "verify_forward_ms": round(fwd_ms, 3), "accept_ms": round(acc_ms, 4),
         "verify_step_ms": round(fwd_ms + acc_ms, 3),
         "logits_to_host_bytes": 4 * (k + 1) * V, "accepted_last": int(res[1])}
    if R is not None:
        try:
            with tempfile.TemporaryDirectory(dir=_tmpdir(8e9)) as td:
                path = os.path.join(td, "m.gguf")
                t0 = time.perf_counter()
                _gguf_stream(path, shape, np.random.default_rng(98), emb_type)
                t_tok = _ref_forward_ms(N, R, path, 2, ctx, [threads])[threads]
            r["cpu_ref_ms"] = round((k + 1) * t_tok, 1)
            r["cpu_ref_sample"] = (f"reference x86 build, {threads} threads: best of 2 single-token forwards at "
                                   f"cache position {ctx} ({t_tok:.1f} ms; the reference holds 4096 positions "
                                   f"and clamps later ones to the last slot, attending 4096 either way), "
                                   f"times k+1 = {k + 1} (it verifies one token per forward)")
            r["gpu_vs_cpu"] = round((k + 1) * t_tok / (fwd_ms + acc_ms), 1)
            log(f"{name}: reference forward {t_tok:.1f} ms ({time.perf_counter() - t0:.1f} s)")
        except Exception as e:
            log(f"{name}: cpu reference failed: {e!r}")
    log(json.dumps(r))
    return r


def run_configs(args):
    """C1/C2 GEMMs and C3/C5 verify steps on one GPU, with the reference's x86
    build timed beside them; one JSON line (not the headline metric)."""
    N, P = load_product()
    L = _bind_gemm(N, P)
    R, threads = None, 0
    if not args.no_cpu_baseline and N.ref_available("avx2"):
        R = N.ref("avx2")
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        R.vx_set_n_threads(threads)
    gemms = _configs_gemm(N, P, L, args, R, threads)
    c3 = _configs_verify(N, P, L, "C3", C3_SHAPE, 512, 4, 0.0, 2, 20, R, threads)
    c5 = _configs_verify(N, P, L, "C5", C5_SHAPE, 8192, 8, 1.0, 8, 10, R, threads)
    print(json.dumps({"mode": "configs", "cpu_threads": threads, "gemm": gemms, "verify": [c3, c5]}),
          flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--tokens", type=int, default=256)
    ap.add_argument("--prompt", type=int, default=2048)
    ap.add_argument("--k", type=int, default=8)
    ap.add_argument("--mode", choices=["spec", "gemm", "configs", "traffic", "paths"], default="spec")
    ap.add_argument("--fetch", help="traffic mode: counter CSV of the FETCH_SIZE run")
    ap.add_argument("--write", help="traffic mode: counter CSV of the WRITE_SIZE run")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="spec mode: skip the C1 GEMM and C3/C5 verify-step figures")
    ap.add_argument("--kv-half", action="store_true",
                    help="spec mode: both models with the flagged fp16 KV cache (not the headline)")
    ap.add_argument("--prof-steps", type=int, default=2,
                    help="steps of the separate instrumented pass that measures the roofline")
    ap.add_argument("--prof-every", type=int, default=7,
                    help="time every n-th verify GEMM of each class with kernel events")
    args = ap.parse_args()
    if args.prof_steps < 1 or args.prof_every < 1:
        ap.error("--prof-steps and --prof-every must be at least 1 (the roofline comes from that pass)")
    ws = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or ws != 1:
        print(f"bench.py: this engine runs the verify path on ONE GPU; --gpus {args.gpus} "
              f"(WORLD_SIZE {ws}) is not supported -- run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.mode == "traffic":
        run_traffic(args)
    elif args.mode == "paths":
        run_paths(args)
    elif args.mode == "gemm":
        run_gemm(args)
    elif args.mode == "configs":
        run_configs(args)
    else:
        run_spec(args)


if __name__ == "__main__":
    main()
