#!/usr/bin/env python3
"""Benchmark of the speculative-decoding verify path on one MI355X.

Workload (default): a 32-layer d4096 MHA (32/32 heads), FFN 11008, vocab
32000 Q4_0 target verifies k = 8 drafts of a 22-layer d2048 GQA (32/4 heads,
head_dim 64, FFN 5632) Q4_0 draft, after a 2048-token prompt of uniform random
ids; sampled acceptance at T = 0.8, top_p = 1.0, seeded uniforms.  Weights are
seeded random-init N(0, 0.02^2) quantised with the reference's Q4_0 writer,
generated directly in HBM.

One step = decoding 256 tokens from the prefilled state (each step restarts
from the same state, so every step does the same work).  The value is the
emitted-token throughput of the timed steps (accepted drafts + the resampled
or bonus token of every round).

roofline: the verify dequant-GEMMs of the target (M = k+1 rows), timed with
HIP events recorded on the target's stream around every GEMM launch inside
the timed steps; achieved = algorithmic bytes (Q4_0 weight blocks + fp32
activations in + fp32 results out) / event time.

cpu_baseline: the reference engine's own x86 build (oracle/_ref, built from
its sources by oracle/Makefile) on this host's cores: single-token forwards
of same-shape models at context 2048, combined with the acceptance trace of
the GPU run (the reference verifies one token per forward).

Usage: python bench.py [--gpus 1] [--steps 3] [--warmup 1] [--mode spec|gemm]
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
def _gguf_stream(path, shape, rng):
    """Writes a random Q4_0 Llama GGUF of the given shape, streaming; one
    layer's random blocks are reused by every layer (timing does not depend
    on the values)."""
    d, F, V, L = shape["n_embd"], shape["n_ff"], shape["n_vocab"], shape["n_layers"]
    kvd = shape["n_kv_heads"] * (d // shape["n_heads"])

    def blocks(rows, cols):
        nb = rows * cols // 32
        b = np.empty((nb, 18), np.uint8)
        b[:, :2] = (np.abs(rng.normal(0, 0.02, nb)).astype(np.float16)).view(np.uint8).reshape(nb, 2)
        b[:, 2:] = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
        return b.tobytes()

    layer = {"attn_q": blocks(d, d), "attn_k": blocks(kvd, d), "attn_v": blocks(kvd, d),
             "attn_output": blocks(d, d), "ffn_gate": blocks(F, d), "ffn_up": blocks(F, d),
             "ffn_down": blocks(d, F)}
    dims = {"attn_q": (d, d), "attn_k": (d, kvd), "attn_v": (d, kvd), "attn_output": (d, d),
            "ffn_gate": (d, F), "ffn_up": (d, F), "ffn_down": (F, d)}
    emb = blocks(V, d)
    ones = np.ones(d, np.float32).tobytes()
    tensors = [("token_embd.weight", 2, (d, V), emb)]
    for l in range(L):
        tensors.append((f"blk.{l}.attn_norm.weight", 0, (d,), ones))
        for nm in ("attn_q", "attn_k", "attn_v", "attn_output"):
            tensors.append((f"blk.{l}.{nm}.weight", 2, dims[nm], layer[nm]))
        tensors.append((f"blk.{l}.ffn_norm.weight", 0, (d,), ones))
        for nm in ("ffn_gate", "ffn_up", "ffn_down"):
            tensors.append((f"blk.{l}.{nm}.weight", 2, dims[nm], layer[nm]))
    tensors.append(("output_norm.weight", 0, (d,), ones))
    tensors.append(("output.weight", 2, (d, V), emb))

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


def _ref_forward_ms(N, R, path, n_tok, ctx):
    mp = C.POINTER(N.VxModel)()
    rc = R.vx_model_create(path.encode(), C.byref(mp))
    if rc != 0:
        raise RuntimeError(f"reference vx_model_create failed ({rc})")
    try:
        V = mp.contents.config.n_vocab
        lg = np.zeros(V, np.float32)
        R.vx_model_forward(mp, np.array([1], np.int32), 1, lg)     # allocates the KV cache
        mp.contents.cache_len = ctx
        times = []
        for i in range(n_tok):
            t0 = time.perf_counter()
            R.vx_model_forward(mp, np.array([(7 * i + 3) % V], np.int32), 1, lg)
            times.append(time.perf_counter() - t0)
            mp.contents.cache_len = ctx                         # same context for every sample
        return 1e3 * float(np.median(times))
    finally:
        R.vx_model_destroy(mp)


def cpu_baseline(N, stats_emitted, stats_drafted, ctx, n_target=3, n_draft=8):
    if not N.ref_available("avx2"):
        return None
    R = N.ref("avx2")
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    R.vx_set_n_threads(threads)
    rng = np.random.default_rng(99)
    import shutil
    tmpdir = None
    for cand in ("/dev/shm", tempfile.gettempdir(), HERE):
        try:
            if os.access(cand, os.W_OK) and shutil.disk_usage(cand).free > 6e9:
                tmpdir = cand
                break
        except OSError:
            pass
    if tmpdir is None:
        raise RuntimeError("no directory with 6 GB free for the reference's GGUF files")
    t_start = time.perf_counter()
    with tempfile.TemporaryDirectory(dir=tmpdir) as td:
        tp, dp = os.path.join(td, "target.gguf"), os.path.join(td, "draft.gguf")
        _gguf_stream(tp, TARGET, rng)
        t_target = _ref_forward_ms(N, R, tp, n_target, ctx)
        os.remove(tp)
        _gguf_stream(dp, DRAFT, rng)
        t_draft = _ref_forward_ms(N, R, dp, n_draft, ctx)
    cpu_ms = stats_drafted * t_draft + stats_emitted * t_target
    log(f"cpu baseline: target forward {t_target:.1f} ms, draft forward {t_draft:.1f} ms "
        f"({threads} threads, {time.perf_counter() - t_start:.1f} s)")
    return {
        "value": round(1e3 * stats_emitted / cpu_ms, 3),
        "unit": "tok/s",
        "cores": threads,
        "kind": "reference",
        "sample": (f"reference x86 build (oracle/_ref/libvxref_avx2.so, -Ofast -mavx2 -mfma -fopenmp), "
                   f"{threads} threads: median of {n_target} target and {n_draft} draft single-token "
                   f"forwards at context {ctx} on same-shape random Q4_0 GGUFs (target "
                   f"{t_target:.1f} ms, draft {t_draft:.1f} ms); tok/s = emitted / (drafted*t_draft + "
                   f"emitted*t_target) for the GPU run's acceptance trace ({stats_drafted} drafted, "
                   f"{stats_emitted} emitted per step)"),
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
    # kernel-execution events around every --prof-every-th verify GEMM of each
    # class (7: a stride that walks through the 32 layers): a launch with
    # events costs ~18 us of host time, enough to starve the GPU when every
    # verify GEMM carries them (174.7 vs 186.3 tok/s)
    P.vx_model_set_profiling(tm, args.prof_every)
    P.vxh_device_sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        n = P.vx_speculative_decode(st, out, args.tokens)
        if n != args.tokens:
            sys.exit("bench.py: decode failed: " + N.product_error())
    P.vxh_device_sync()
    elapsed = time.perf_counter() - t0
    prof = (N.VxGemmProfile * 5)()
    P.vx_model_get_profile(tm, prof)
    P.vx_model_set_profiling(tm, 0)
    stats = N.VxSpecStats()
    P.vx_speculative_get_stats(st, C.byref(stats))
    value = args.steps * args.tokens / elapsed
    names = ["qkv", "attn_out", "gate_up", "down", "output"]
    ms = sum(p.ms for p in prof)
    byt = sum(p.bytes for p in prof)
    launches = sum(p.launches for p in prof)
    achieved = byt / (ms * 1e-3) / 1e9 if ms > 0 else 0.0
    breakdown = {nm: {"launches": p.launches, "avg_us": round(1e3 * p.ms / max(p.launches, 1), 2),
                      "GB/s": round(p.bytes / (p.ms * 1e-3) / 1e9, 1) if p.ms > 0 else None}
                 for nm, p in zip(names, prof)}
    log(f"decode: {value:.1f} tok/s; rounds {stats.rounds}, accepted {stats.accepted}/{stats.drafted}; "
        f"verify {stats.verify_ms:.1f} ms, draft {stats.draft_ms:.1f} ms per step")
    log("verify GEMMs:", json.dumps(breakdown))
    cpu = None
    if not args.no_cpu_baseline:
        try:
            cpu = cpu_baseline(N, stats.emitted, stats.drafted, args.prompt)
        except Exception as e:   # reported, the GPU figure stands on its own
            log("cpu baseline failed:", repr(e))
    P.vx_speculative_destroy(st)
    P.vx_model_destroy(tm)
    P.vx_model_destroy(dm)
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
            "acceptance_rate": round(stats.accepted / max(stats.drafted, 1), 4),
            "rounds_per_step": stats.rounds,
            "verify_ms_per_round": round(stats.verify_ms / max(stats.rounds, 1), 3),
            "draft_ms_per_round": round(stats.draft_ms / max(stats.rounds, 1), 3),
            "prefill_s": round(prefill_s, 3),
            "verify_gemms": breakdown,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": read_traffic(),
            "kernel": (f"vx_gemm_kernel (Q4_0, M={args.k + 1}), every {args.prof_every}th verify GEMM launch "
                       f"of each class (kernel-execution events)"),
            "launches": launches,
            "avg_launch_us": round(1e3 * ms / max(launches, 1), 3),
            "bytes_per_launch": round(byt / max(launches, 1)),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def run_gemm(args):
    """Isolated verify GEMM kernels at M = k+1 on the 7B shapes, each with the
    panel prologue the verify forward gives it (vxh_gemm_pro: residual add +
    norm weight for QKV and gate/up, attention rows for the output
    projection, SwiGLU for down, norm weight for the logits), weights rotated
    over > 300 MB so the Infinity Cache does not serve them."""
    N, P = load_product()
    import ctypes as CC
    vp = CC.c_void_p
    L = N.bind_vxh(P)
    L.vxh_qmat_alloc.argtypes = [vp, CC.c_int, CC.c_int, CC.c_int]
    L.vxh_synth_blocks.argtypes = [vp, CC.c_int, CC.c_int, CC.c_int, CC.c_uint64, CC.c_float, vp]
    L.vxh_qmat_set_rows.argtypes = [vp, vp, CC.c_int, CC.c_int, CC.c_int, CC.c_int, CC.c_int, vp]
    L.vxh_gemm_pro.argtypes = [vp, CC.c_int, vp, vp, CC.c_int, CC.c_int, CC.c_float, vp, vp, vp]
    L.vxh_qmat_free.argtypes = [vp]
    L.vxh_event_create.argtypes = [vp]
    L.vxh_event_record.argtypes = [vp, vp]
    L.vxh_event_elapsed_ms.argtypes = [vp, vp, vp]

    class QMat(CC.Structure):
        _fields_ = [("type", CC.c_int), ("n_rows", CC.c_int), ("n_cols", CC.c_int), ("n_pairs", CC.c_int),
                    ("qs", vp), ("d", vp)]

    class Pro(CC.Structure):
        _fields_ = [("kind", CC.c_int), ("x", vp), ("ldx", CC.c_int), ("src", vp), ("ld_src", CC.c_int),
                    ("w", vp), ("x_out", vp), ("ld_xout", CC.c_int), ("ss", vp), ("ss_in", vp),
                    ("ss_K", CC.c_int), ("thr", CC.c_float), ("clear", vp), ("n_clear", CC.c_size_t),
                    ("part", vp), ("n_chunks", CC.c_int), ("n_heads", CC.c_int), ("n_kv_heads", CC.c_int),
                    ("head_dim", CC.c_int)]
    PRO_ROWS, PRO_RESID, PRO_SWIGLU = 1, 2, 3

    M = args.k + 1
    results = []
    # calibration for rocprofv3 byte counters: a device-to-device copy of a
    # known size (FETCH_SIZE and WRITE_SIZE of that copy should read 256 MiB)
    cal_bytes = 256 << 20
    ca, cb = N.DevBuf(L, nbytes=cal_bytes), N.DevBuf(L, nbytes=cal_bytes)
    L.vxh_copy.argtypes = [vp, vp, CC.c_size_t, vp]
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
        bpw = 18 if qt == 2 else 34
        mat_bytes = rows * cols // 32 * bpw
        n_rot = max(2, int(np.ceil(300e6 / mat_bytes)))
        mats = []
        stage = N.DevBuf(L, nbytes=mat_bytes)
        for i in range(n_rot):
            q = QMat()
            assert L.vxh_qmat_alloc(CC.byref(q), qt, rows, cols) == 0, L.vxh_last_error()
            assert L.vxh_synth_blocks(stage.ptr, qt, rows, cols, 1000 + i, 0.02, None) == 0
            assert L.vxh_qmat_set_rows(CC.byref(q), stage.ptr, 1, rows, rows, 0, 0, None) == 0
            mats.append(q)
        stage.free()
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
        e0, e1 = vp(), vp()
        L.vxh_event_create(CC.byref(e0))
        L.vxh_event_create(CC.byref(e1))

        def launch(q):
            return L.vxh_gemm_pro(CC.byref(q), M, CC.byref(pro), acc.ptr, rows, rows, 1.0, None, None, None)
        for q in mats:
            assert launch(q) == 0, L.vxh_last_error()
        reps = args.steps * 10
        L.vxh_device_sync()
        L.vxh_event_record(e0, None)
        for r in range(reps):
            for q in mats:
                launch(q)
        L.vxh_event_record(e1, None)
        ms = CC.c_float()
        L.vxh_event_elapsed_ms(e0, e1, CC.byref(ms))
        n = reps * len(mats)
        avg_us = 1e3 * ms.value / n
        alg = mat_bytes + 4 * M * cols + 4 * M * rows
        gbs = alg / (avg_us * 1e-6) / 1e9
        results.append({"shape": f"{'Q4_0' if qt == 2 else 'Q8_0'} {rows}x{cols} M={M}",
                        "prologue": {PRO_ROWS: "rows", PRO_RESID: "resid", PRO_SWIGLU: "swiglu"}[kind],
                        "avg_us": round(avg_us, 2), "GB/s": round(gbs, 1),
                        "frac": round(gbs / PEAK_HBM_GBS, 4)})
        log(json.dumps(results[-1]))
        for b in bufs + [acc]:
            b.free()
        for q in mats:
            L.vxh_qmat_free(CC.byref(q))
    print(json.dumps({"mode": "gemm", "M": M, "results": results}), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--tokens", type=int, default=256)
    ap.add_argument("--prompt", type=int, default=2048)
    ap.add_argument("--k", type=int, default=8)
    ap.add_argument("--mode", choices=["spec", "gemm"], default="spec")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--prof-every", type=int, default=7,
                    help="time every n-th verify GEMM of each class with kernel events")
    args = ap.parse_args()
    ws = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or ws != 1:
        print(f"bench.py: this engine runs the verify path on ONE GPU; --gpus {args.gpus} "
              f"(WORLD_SIZE {ws}) is not supported -- run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.mode == "gemm":
        run_gemm(args)
    else:
        run_spec(args)


if __name__ == "__main__":
    main()
