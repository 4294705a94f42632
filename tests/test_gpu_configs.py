"""Parity at the shapes of the benchmark configurations that are not the bench line.

C1 / C2: the isolated dequant GEMMs (4096x4096 Q4_0 at M=5; 11008x4096 and
4096x11008 in Q4_0 and Q8_0 at M = 1, 5, 9) against the oracle GEMV, with the
fp64 exact product as the fallback reference where the oracle's own fp32
rounding exceeds the bar (the `parity` helper).

C3 / C5: the verify step itself at full size.  The model is created on the
GPU from seeded weights (vx_model_create_synthetic) and the oracle is given
the same weights (read back as GGUF blocks).  The GPU prefills the
configuration's context and its KV cache is checked against the oracle
before any verify row is compared:

* C3 (22 layers, 512 positions): the oracle runs its own prefill of the same
  prompt and every cached K/V row of every layer is compared; the verify
  steps then run from the oracle's own cache.
* C5 (all 28 layers, 8192 positions): at 8-position windows (the start,
  across the 4096 cap edge, the end) the oracle recomputes every row of every
  layer from the GPU rows before the window; the verify step then reads the
  GPU cache so checked.

The logits of every verify row are compared with the oracle's
teacher-forced forwards (1e-4 + 1e-3 |ref|), and the acceptance decisions
(greedy for C3, sampled at T = 1.0 with seeded uniforms for C5) with the
oracle's on the same logits.  Prefills run with the FFN gate-skip off on
both sides (tens of millions of gate decisions, some within rounding of
the threshold); C3's verify step runs at 0 and at the reference's 0.01, where
a row moved by a decision at the threshold must carry a certificate.
"""
import ctypes as C
import itertools

import numpy as np
import pytest

import _native as N
from _native import close, max_violation
from _oracle_model import OracleModel

pytestmark = pytest.mark.gpu
O = N.oracle()


@pytest.fixture(scope="module")
def P():
    if not N.product_available():
        pytest.fail("product library not built")
    L = N.bind_vxh(N.product())
    assert L.vxh_init() == 0, L.vxh_last_error()
    return L


def _oracle_rows(W, typ, X):
    rows, nb = W.shape
    cols = nb * 32
    out = np.zeros((X.shape[0], rows), np.float32)
    if typ == 2:
        for m in range(X.shape[0]):
            O.or_gemv_q4_0(N._ptr(W), np.ascontiguousarray(X[m]), out[m], rows, cols)
        vals = N.q4_values(W)
    else:
        A = np.zeros(rows * cols, np.float32)
        O.or_dequantize_row_q8_0(N._ptr(W), A, rows * cols, 1.0)
        A = A.reshape(rows, cols)
        for m in range(X.shape[0]):
            O.or_gemv_f32(out[m], A, np.ascontiguousarray(X[m]), rows, cols)
        vals = N.q8_values(W)
    return out, X.astype(np.float64) @ vals.T


GEMM_CASES = [("C1", 4096, 4096, 2, 5)] + [
    ("C2", r, c, t, m) for (r, c) in ((11008, 4096), (4096, 11008)) for t in (2, 8) for m in (1, 5, 9)]


@pytest.mark.parametrize("cfg,rows,cols,typ,M", GEMM_CASES)
def test_config_gemm(P, cfg, rows, cols, typ, M):
    print(f"{cfg} gemm {'Q4_0' if typ == 2 else 'Q8_0'} {rows}x{cols} M={M}", flush=True)
    rng = np.random.default_rng(rows + 3 * cols + 7 * typ + M)
    W = N.rand_q4_0(rng, rows, cols) if typ == 2 else N.rand_q8_0(rng, rows, cols)
    X = rng.normal(0, 1, (M, cols)).astype(np.float32)
    Y = np.zeros((M, rows), np.float32)
    if typ == 2:
        rc = P.vx_gemm_q4_0(N._ptr(W), X, cols, Y, M, rows, cols, 0)
    else:
        rc = P.vx_gemm_q8_0(N._ptr(W), X, cols, Y, M, rows, cols)
    assert rc == 0, N.product_error()
    ref, exact = _oracle_rows(W, typ, X)
    ok, nfb = N.parity(Y, ref, exact)
    assert ok, max_violation(Y, ref)
    print(f"elements on the exact-value fallback: {nfb}")


# ---------------------------------------------------------------------------
# full verify steps
# ---------------------------------------------------------------------------
def synth(P, n_layers, d, h, kv, F, V, n_ctx, seed, emb_type=2, out_type=2, cap=4096, thr=0.01):
    cfg = N.VxModelConfig()
    cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.n_embd, cfg.n_ff, cfg.n_vocab = n_layers, h, kv, d, F, V
    cfg.n_ctx = n_ctx
    cfg.rope_theta = 10000.0
    spec = N.VxSynthSpec(seed=seed, std=0.02, matrix_type=2, embd_type=emb_type, output_type=out_type)
    mp = C.POINTER(N.VxModelDev)()
    assert P.vx_model_create_synthetic(C.byref(cfg), C.byref(spec), C.byref(mp)) == 0, N.product_error()
    opt = N.VxModelOptions()
    P.vx_model_get_options(mp, C.byref(opt))
    opt.attn_cap = cap
    opt.ffn_gate_threshold = thr
    assert P.vx_model_set_options(mp, C.byref(opt)) == 0
    return mp


def read_weights(P, mp, n_layers, d, kvd, F, V, emb_type, out_type):
    """GGUF blocks of every matrix of the device model, norms as ones."""
    def blocks(name, rows, cols, typ):
        dt = N.Q4_BLOCK if typ == 2 else N.Q8_BLOCK
        b = np.zeros((rows, cols // 32), dtype=dt)
        assert P.vx_model_read_tensor(mp, name.encode(), N._ptr(b), b.nbytes) == 0, (name, N.product_error())
        return b
    w = {"token_embd.weight": blocks("token_embd.weight", V, d, emb_type),
         "output.weight": blocks("output.weight", V, d, out_type),
         "output_norm.weight": np.ones(d, np.float32)}
    for l in range(n_layers):
        for nm, r, c in (("attn_q", d, d), ("attn_k", kvd, d), ("attn_v", kvd, d), ("attn_output", d, d),
                         ("ffn_gate", F, d), ("ffn_up", F, d), ("ffn_down", d, F)):
            w[f"blk.{l}.{nm}.weight"] = blocks(f"blk.{l}.{nm}.weight", r, c, 2)
        w[f"blk.{l}.attn_norm.weight"] = np.ones(d, np.float32)
        w[f"blk.{l}.ffn_norm.weight"] = np.ones(d, np.float32)
    return w


def prefill(P, mp, toks, V):
    lg = np.zeros(V, np.float32)
    assert P.vx_model_forward(mp, np.ascontiguousarray(toks, np.int32), len(toks), lg) == 0, N.product_error()
    return lg


def oracle_prefilled(P, mp, w, n_layers, d, h, kv, F, V, n_ctx, prompt, cap, what):
    """An oracle model that ran its own prefill of `prompt` (FFN gate-skip
    off, as the GPU prefill must have run), after every row of the GPU's
    cache [0, len(prompt)) in every layer is compared with the oracle's."""
    om = OracleModel(w, n_layers, d, h, kv, F, V, n_ctx=n_ctx, attn_cap=cap, gate_thr=0.0)
    kvd = kv * (d // h)
    assert O.or_forward(om.ptr, np.ascontiguousarray(prompt, np.int32), len(prompt), np.zeros(V, np.float32)) == 0
    kg, vg = read_cache(P, mp, n_layers, len(prompt), kvd)
    check_cache_rows(kg, vg, om, n_layers, n_ctx, kvd, 0, len(prompt), what)
    return om


def read_cache(P, mp, n_layers, n, kvd):
    k = np.zeros((n_layers, n, kvd), np.float32)
    v = np.zeros((n_layers, n, kvd), np.float32)
    for l in range(n_layers):
        assert P.vx_model_read_kv(mp, l, n, k[l], v[l]) == 0, N.product_error()
    return k, v


def check_cache_rows(kg, vg, om, n_layers, n_ctx, kvd, lo, hi, what):
    """GPU cache rows [lo, hi) of every layer against the oracle's."""
    kc = om.k_cache.reshape(n_layers, n_ctx, kvd)
    vc = om.v_cache.reshape(n_layers, n_ctx, kvd)
    worst = 0.0
    for l in range(n_layers):
        for nm, g, r in (("K", kg[l, lo:hi], kc[l, lo:hi]), ("V", vg[l, lo:hi], vc[l, lo:hi])):
            assert close(g, r), (what, nm, "layer", l, max_violation(g, r))
            worst = max(worst, float(np.abs(g.astype(np.float64) - r).max()))
    print(f"{what}: cache rows {lo}..{hi - 1} of {n_layers} layers, max |diff| {worst:.2e}")


@pytest.fixture(scope="module")
def c3(P):
    """C3 model: 22 layers, d 2048, 32/4 heads, FFN 5632, V 32000, Q4_0.  The
    GPU prefills 512 positions (FFN gate-skip off on both sides: with ~6e7
    gate decisions in a 22-layer prefill, hundreds sit within the two sides'
    rounding distance of 0.01), and every cached K/V row of every layer is
    compared with the oracle's own prefill of the same prompt; the verify
    steps then run from the oracle's cache, not the GPU's."""
    L, d, h, kv, F, V, ctx = 22, 2048, 32, 4, 5632, 32000, 512
    kvd = kv * (d // h)
    print("C3 prefill: 22L d2048 32/4 heads FFN 5632 V 32000, 512 positions", flush=True)
    mp = synth(P, L, d, h, kv, F, V, 1024, seed=303, thr=0.0)
    rng = np.random.default_rng(33)
    prompt = rng.integers(0, V, ctx + 1).astype(np.int32)
    prefill(P, mp, prompt[:ctx], V)
    kg, vg = read_cache(P, mp, L, ctx, kvd)
    w = read_weights(P, mp, L, d, kvd, F, V, 2, 2)
    om = OracleModel(w, L, d, h, kv, F, V, n_ctx=1024, attn_cap=4096, gate_thr=0.0)
    assert O.or_forward(om.ptr, prompt[:ctx], ctx, np.zeros(V, np.float32)) == 0
    check_cache_rows(kg, vg, om, L, 1024, kvd, 0, ctx, "C3 prefill")
    yield dict(mp=mp, om=om, prompt=prompt, rng=rng, L=L, V=V, ctx=ctx)
    P.vx_model_destroy(mp)


def set_threshold(P, mp, thr):
    opt = N.VxModelOptions()
    P.vx_model_get_options(mp, C.byref(opt))
    opt.ffn_gate_threshold = thr
    assert P.vx_model_set_options(mp, C.byref(opt)) == 0


@pytest.mark.parametrize("thr", [0.0, 0.01])
def test_c3_verify_step_full_size(P, c3, thr):
    """C3 verify step, k = 4 greedy, on the checked 512-position prefill.  Two
    of the drafts are the model's own greedy continuation so that the
    acceptance path accepts, then rejects.  The verify step runs at the FFN
    gate-skip threshold 0 (strict) and at the reference's 0.01."""
    mp, om, prompt, V, ctx, L, k = c3["mp"], c3["om"], c3["prompt"], c3["V"], c3["ctx"], c3["L"], 4
    print(f"C3 verify step: 22L d2048, 512 prefilled, k=4 greedy, gate threshold {thr}", flush=True)
    rng = np.random.default_rng(34 + int(thr * 100))
    set_threshold(P, mp, thr)
    # greedy continuation of 2 tokens, then roll the cache back
    t0 = int(prompt[ctx])
    g0 = int(np.argmax(prefill(P, mp, [t0], V)))
    g1 = int(np.argmax(prefill(P, mp, [g0], V)))
    P.vx_model_kv_truncate(mp, ctx)
    drafts = [g0, g1] + [int(x) for x in rng.integers(0, V, k - 2)]
    toks = np.array([t0] + drafts, np.int32)
    got = np.zeros((k + 1, V), np.float32)
    assert P.vx_model_verify(mp, toks, k + 1, got) == 0, N.product_error()
    P.vx_model_kv_truncate(mp, ctx)
    om.m.gate_thr = thr
    ref = oracle_verify(om, toks, ctx, k, V)
    diff = np.abs(got.astype(np.float64) - ref)
    print(f"max |diff| {diff.max():.3e}, per row {np.round(diff.max(1), 6)}")
    if not close(got, ref):
        # The FFN gate-skip (src/model.c:582-585) is a step at |silu(g)| = thr:
        # a gate within the two sides' rounding distance of the threshold can
        # fall either way.  Certified only when the first differing row has a
        # gate within the fp32 rounding window of the threshold AND the oracle
        # rerun with exactly that decision inverted matches the GPU on every row.
        assert thr > 0, max_violation(got, ref)
        ref, where = certify_gate_flips(om, toks, ctx, k, V, L, got, ref)
        diff = np.abs(got.astype(np.float64) - ref)
        for j, l, col, dist in where:
            print(f"certified gate at the threshold: token row {j}, layer {l}, column {col} "
                  f"(| |silu(g)| - thr | = {dist:.2e})")
        print(f"max |diff| after {len(where)} inverted decision(s) {diff.max():.3e}")
    check_greedy_rows(got, ref, diff, np.array(drafts, np.int32), k, V)


def set_flips(om, flips):
    om.m.flip = len(flips)
    for f, (j, l, col) in enumerate(flips):
        om.m.flip_tok[f], om.m.flip_layer[f], om.m.flip_col[f] = j, l, col


def certify_gate_flips(om, toks, n_past, k, V, n_layers, got, ref0, max_flips=3):
    """Returns the oracle logits with certified gate decisions inverted and
    their (row, layer, column, distance) list; fails when no set of at most
    max_flips such decisions explains the GPU result.  Rows are explained in
    order: a decision in token row j changes row j and the later rows only, so
    the first row that differs must match once one or two decisions of that
    row -- each a gate within the fp32 rounding window of the threshold -- are
    inverted; then the next differing row, and so on."""
    # window: the fp32 rounding scale of the oracle's own gate, a sequential
    # sum of d products whose partial sums are O(1): 2 sqrt(d) 2^-24
    # (5.4e-6 at d = 2048); the rerun with the decisions inverted certifies
    tol = 2.0 * np.sqrt(om.m.n_embd) * 2.0 ** -24
    flips, where, ref = [], [], ref0
    try:
        while True:
            bad = [j for j in range(k + 1) if not close(got[j], ref[j])]
            if not bad:
                return ref, where
            assert len(flips) < max_flips, ("more gate decisions needed than", max_flips, where, bad)
            j0 = bad[0]
            near = np.zeros((k + 1, n_layers), np.float32)
            idx = np.zeros((k + 1, n_layers), np.int32)
            set_flips(om, flips)
            om.m.gate_near, om.m.gate_near_idx = near.ctypes.data, idx.ctypes.data
            oracle_verify(om, toks, n_past, k, V)
            om.m.gate_near, om.m.gate_near_idx = None, None
            cands = [(int(l), int(idx[j0, l]), float(near[j0, l])) for l in np.argsort(near[j0])
                     if near[j0, l] <= tol]
            assert cands, ("no gate within the rounding window of the threshold in row", j0,
                           float(near[j0].min()), tol)
            found = None
            for combo in [[c] for c in cands] + [list(p) for p in itertools.combinations(cands, 2)]:
                if len(flips) + len(combo) > max_flips:
                    continue
                trial = flips + [(j0, l, col) for l, col, _ in combo]
                set_flips(om, trial)
                r = oracle_verify(om, toks, n_past, k, V)
                if close(got[j0], r[j0]):
                    found = (trial, combo, r)
                    break
            assert found, ("no inverted gate decision of row", j0, "explains the GPU result", cands,
                           max_violation(got[j0], ref[j0]))
            flips, ref = found[0], found[2]
            where += [(j0, l, col, dist) for l, col, dist in found[1]]
    finally:
        set_flips(om, [])


def check_greedy_rows(got, ref, diff, drafts, k, V):
    """Greedy decisions row by row up to the first row whose top-2 gap is within
    twice that row's difference (a near-tie may fall either way there): the
    argmax of every such row and the emitted prefix must agree."""
    srt = np.sort(ref, axis=1)
    gaps = srt[:, -1] - srt[:, -2]
    tie = [j for j in range(k + 1) if gaps[j] <= 2 * diff[j].max()]
    jt = tie[0] if tie else k + 1
    for j in range(jt):
        assert int(np.argmax(got[j])) == int(np.argmax(ref[j])), j
    out_g, out_r = np.zeros(k + 1, np.int32), np.zeros(k + 1, np.int32)
    n_g = O.or_accept_greedy(np.ascontiguousarray(got.ravel()), V, drafts, k, out_g)
    n_r = O.or_accept_greedy(np.ascontiguousarray(ref.ravel()), V, drafts, k, out_r)
    m = min(n_g, n_r, jt)
    assert list(out_g[:m]) == list(out_r[:m])
    if jt > min(n_g, n_r) - 1:   # every decision taken before a near-tie row
        assert n_g == n_r and list(out_g[:n_g]) == list(out_r[:n_r])
    print(f"emitted {n_r} tokens (accepted {n_r - 1}); top-2 gaps {np.round(gaps, 5)}; "
          f"rows compared before a near-tie: {jt}")
    assert n_r >= 2, "the greedy continuation is accepted"


def oracle_verify(om, toks, n_past, k, V):
    """Teacher-forced oracle logits of the verify tokens from cache position n_past."""
    om.cache_len = n_past
    ref = np.zeros((k + 1, V), np.float32)
    assert O.or_forward_all(om.ptr, toks, k + 1, ref) == 0
    return ref


@pytest.fixture(scope="module")
def c5(P):
    """C5 model, all 28 layers: d 3584, 28/4 heads (head_dim 128), FFN 18944,
    V 152064 with Q8_0 embedding/output; its weights read back once."""
    L, d, h, kv, F, V, ctx = 28, 3584, 28, 4, 18944, 152064, 8192
    print("C5 model: 28L d3584 28/4 heads FFN 18944 V 152064", flush=True)
    mp = synth(P, L, d, h, kv, F, V, ctx + 16, seed=505, emb_type=8, out_type=8, cap=4096, thr=0.0)
    w = read_weights(P, mp, L, d, kv * (d // h), F, V, 8, 8)
    om = OracleModel(w, L, d, h, kv, F, V, n_ctx=ctx + 16, attn_cap=4096, gate_thr=0.0)
    yield dict(mp=mp, om=om, L=L, V=V, ctx=ctx, kvd=kv * (d // h))
    P.vx_model_destroy(mp)


@pytest.mark.parametrize("cap", [4096, 0])
def test_c5_verify_step_full_width(P, c5, cap):
    """C5 at all 28 layers: 8192 prefilled positions, read under the
    reference's 4096-position cap (src/model.c:304-305) and without it (every
    position attended); k = 8 sampled at T = 1.0; FFN gate-skip off (with ~5e6
    gate decisions per verify step several sit within rounding of 0.01; the
    skip is certified in the C3 test).

    The GPU prefill's cache is checked before the oracle reads it: at 8-position
    windows (the start, across the 4096 cap edge and the end of the context)
    the oracle recomputes every row of every layer from the GPU rows before the
    window, and the GPU rows must match.  An oracle prefill of all 8192
    positions through 28 layers (~5e13 multiply-adds) is beyond a test; every
    position runs through the same prefill kernels, which the C3 test checks
    row by row over its whole 512-position, 22-layer prefill."""
    mp, om, L, V, ctx, kvd, k = c5["mp"], c5["om"], c5["L"], c5["V"], c5["ctx"], c5["kvd"], 8
    n_ctx = ctx + 16
    print(f"C5 verify step: 28 x (d3584, 28/4 heads, FFN 18944), V 152064 Q8_0, 8192 prefilled, cap {cap}",
          flush=True)
    opt = N.VxModelOptions()
    P.vx_model_get_options(mp, C.byref(opt))
    opt.attn_cap = cap
    assert P.vx_model_set_options(mp, C.byref(opt)) == 0
    P.vx_model_kv_truncate(mp, 0)
    rng = np.random.default_rng(55)
    prompt = rng.integers(0, V, ctx).astype(np.int32)
    prefill(P, mp, prompt, V)
    toks = rng.integers(0, V, k + 1).astype(np.int32)
    got = np.zeros((k + 1, V), np.float32)
    assert P.vx_model_verify(mp, toks, k + 1, got) == 0, N.product_error()
    kg, vg = read_cache(P, mp, L, ctx, kvd)
    P.vx_model_kv_truncate(mp, ctx)
    om.m.attn_cap = cap
    kc = om.k_cache.reshape(L, n_ctx, kvd)
    vc = om.v_cache.reshape(L, n_ctx, kvd)
    kc[:, :ctx], vc[:, :ctx] = kg, vg
    for lo in ([0] if cap else []) + [4092, ctx - 8]:
        om.cache_len = lo
        assert O.or_forward(om.ptr, prompt[lo:lo + 8], 8, np.zeros(V, np.float32)) == 0
        check_cache_rows(kg, vg, om, L, n_ctx, kvd, lo, lo + 8, f"C5 cap {cap} window")
    kc[:, :ctx], vc[:, :ctx] = kg, vg
    ref = oracle_verify(om, toks, ctx, k, V)
    print(f"max |diff| {np.abs(got.astype(np.float64) - ref).max():.3e}")
    assert close(got, ref), max_violation(got, ref)
    # sampled acceptance at T = 1 on the verified logits, against the oracle's
    # decision on the same logits (seeded draft logits and uniforms)
    from test_gpu_accept import run_accept, oracle_accept
    D = rng.normal(0, 2.0, (k, V)).astype(np.float32)
    drafts = toks[1:]
    u = rng.random(k + 1).astype(np.float32)
    n_g, na_g, out_g = run_accept(P, got, D, drafts, 1.0, 1.0, u)
    n_o, na_o, out_o, _ = oracle_accept(got, D, drafts, 1.0, 1.0, u)
    print(f"accepted {na_o} of {k}; emitted {out_o}")
    assert (n_g, na_g, out_g) == (n_o, na_o, out_o)
