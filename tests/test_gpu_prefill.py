"""Large-M prompt prefill (vx_model_forward of a long prompt: chunks of up to
512 rows through vxh_gemm_rows, vxh_rope_kv_rows, vxh_attention and
vxh_swiglu_rows) against the oracle, which runs the prompt one token per
forward like the reference (src/speculative.c:100-107, src/model.c:391-628).

Checked at the fp32 bar (1e-4 + 1e-3 |ref|): the last token's logits, every
cached K/V row of every layer, and the logits of a verify step run on the
prefilled cache.  The same prompt through the batched decode forward
(prefill_min_rows = 0) agrees with the large-M path at the same bar.
"""
import ctypes as C
import itertools

import numpy as np
import pytest

import _native as N
import test_gpu_gemm   # the vxh_qmat mirror
from _gguf import llama_gguf, GGML_Q4_0, GGML_Q8_0
from _native import close, max_violation
from _oracle_model import OracleModel

pytestmark = pytest.mark.gpu
O = N.oracle()


@pytest.fixture(scope="module")
def P():
    if not N.product_available():
        pytest.fail("product library not built")
    L = N.product()
    assert L.vxh_init() == 0, L.vxh_last_error()
    return L


def load(P, path, n_ctx, prefill_min_rows=None, thr=0.0):
    """The FFN gate-skip is off (threshold 0) on both sides by default: with
    ~4e5 gate decisions per prompt one may sit within rounding of 0.01 and
    move a row by ~1e-3.  test_prefill_at_gate_threshold runs the reference's
    0.01 and certifies any such decision."""
    mp = C.POINTER(N.VxModelDev)()
    assert P.vx_model_create(path.encode(), C.byref(mp)) == 0, N.product_error()
    mp.contents.config.n_ctx = n_ctx
    opt = N.VxModelOptions()
    P.vx_model_get_options(mp, C.byref(opt))
    opt.ffn_gate_threshold = thr
    if prefill_min_rows is not None:
        opt.prefill_min_rows = prefill_min_rows
    assert P.vx_model_set_options(mp, C.byref(opt)) == 0
    return mp


CASES = [
    # layers, d, heads, kv, ff, vocab, matrix type, prompt length
    (2, 256, 4, 2, 512, 512, GGML_Q4_0, 512),
    (2, 256, 8, 2, 640, 300, GGML_Q4_0, 600),
    (1, 192, 3, 3, 384, 256, GGML_Q8_0, 300),
    (1, 256, 2, 1, 256, 64, GGML_Q4_0, 300),      # head_dim 128: two chunks per attention wavefront
]


@pytest.mark.parametrize("case", CASES)
def test_prefill_matches_oracle(P, tmp_path, case):
    L, d, h, kv, ff, V, mt, n = case
    print(f"prefill {n} tokens: {L}L d{d} {h}/{kv} heads ff{ff} V{V} {'Q4_0' if mt == GGML_Q4_0 else 'Q8_0'}",
          flush=True)
    rng = np.random.default_rng(sum(case))
    path = str(tmp_path / "m.gguf")
    raw = llama_gguf(path, rng, L, d, h, kv, ff, V, std=0.05, norm_random=True, emb_type=mt, out_type=mt,
                     matrix_type=mt)
    n_ctx = 1024
    prompt = rng.integers(0, V, n).astype(np.int32)
    mp = load(P, path, n_ctx)
    mb = load(P, path, n_ctx, prefill_min_rows=0)
    try:
        got = np.zeros(V, np.float32)
        assert P.vx_model_forward(mp, prompt, n, got) == 0, N.product_error()
        assert mp.contents.cache_len == n
        base = np.zeros(V, np.float32)
        assert P.vx_model_forward(mb, prompt, n, base) == 0, N.product_error()
        hd, kvd = d // h, kv * (d // h)
        kv_gpu = []
        for l in range(L):
            k = np.zeros((n, kvd), np.float32)
            v = np.zeros((n, kvd), np.float32)
            assert P.vx_model_read_kv(mp, l, n, k, v) == 0, N.product_error()
            kv_gpu.append((k, v))
        toks = rng.integers(0, V, 5).astype(np.int32)
        ver = np.zeros((5, V), np.float32)
        assert P.vx_model_verify(mp, toks, 5, ver) == 0, N.product_error()
    finally:
        P.vx_model_destroy(mp)
        P.vx_model_destroy(mb)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=n_ctx, gate_thr=0.0)
    ref = np.zeros(V, np.float32)
    assert O.or_forward(om.ptr, prompt, n, ref) == 0
    print(f"last-token logits: max |diff| {np.abs(got.astype(np.float64) - ref).max():.2e} "
          f"(batched path {np.abs(base.astype(np.float64) - ref).max():.2e})")
    assert close(got, ref), max_violation(got, ref)
    assert close(got, base), max_violation(got, base)
    kc = om.k_cache.reshape(L, n_ctx, kvd)
    vc = om.v_cache.reshape(L, n_ctx, kvd)
    for l, (k, v) in enumerate(kv_gpu):
        assert close(k, kc[l, :n]), ("K", l, max_violation(k, kc[l, :n]))
        assert close(v, vc[l, :n]), ("V", l, max_violation(v, vc[l, :n]))
    vref = np.zeros((5, V), np.float32)
    assert O.or_forward_all(om.ptr, toks, 5, vref) == 0
    print(f"verify after prefill: max |diff| {np.abs(ver.astype(np.float64) - vref).max():.2e}")
    assert close(ver, vref), max_violation(ver, vref)


def _rows_gemm(P, typ, W, X, R=None, scale=1.0):
    """vxh_rows_panel + vxh_gemm_rows on host arrays: Y = R + scale X W^T."""
    vp = C.c_void_p
    L = N.bind_vxh(P)
    L.vxh_qmat_alloc.argtypes = [vp, C.c_int, C.c_int, C.c_int]
    L.vxh_qmat_set_rows.argtypes = [vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, vp]
    L.vxh_qmat_free.argtypes = [vp]
    L.vxh_rows_panel_bytes.restype = C.c_size_t
    L.vxh_rows_panel_bytes.argtypes = [C.c_int, C.c_int]
    L.vxh_rows_panel.argtypes = [vp, C.c_int, C.c_int, C.c_int, vp, vp]
    L.vxh_gemm_rows.argtypes = [vp, vp, C.c_int, vp, C.c_int, C.c_int, vp, C.c_int, C.c_float, vp]
    M, cols = X.shape
    rows = W.shape[0]
    q = test_gpu_gemm._QMat()
    assert L.vxh_qmat_alloc(C.byref(q), typ, rows, cols) == 0, L.vxh_last_error()
    assert L.vxh_qmat_set_rows(C.byref(q), N._ptr(W), 0, rows, rows, 0, 0, None) == 0, L.vxh_last_error()
    dx = N.DevBuf(L, X)
    px = N.DevBuf(L, nbytes=L.vxh_rows_panel_bytes(M, cols))
    dy = N.DevBuf(L, nbytes=4 * M * rows)
    dr = N.DevBuf(L, R) if R is not None else None
    try:
        assert L.vxh_rows_panel(dx.ptr, cols, M, cols, px.ptr, None) == 0, L.vxh_last_error()
        assert L.vxh_gemm_rows(C.byref(q), px.ptr, M, dy.ptr, rows, rows, dr.ptr if dr else None, rows, scale,
                               None) == 0, L.vxh_last_error()
        assert L.vxh_stream_sync(None) == 0
        return dy.get(np.float32, M * rows).reshape(M, rows)
    finally:
        for b in (dx, px, dy, dr):
            if b is not None:
                b.free()
        L.vxh_qmat_free(C.byref(q))


def _oracle_rows(typ, W, X):
    """The oracle's GEMV, one call per row, on 8 threads (ctypes releases
    the GIL), and the fp64 value of the same products."""
    from concurrent.futures import ThreadPoolExecutor
    M, cols = X.shape
    rows = W.shape[0]
    ref = np.zeros((M, rows), np.float32)
    if typ == GGML_Q4_0:
        def one(m):
            O.or_gemv_q4_0(N._ptr(W), np.ascontiguousarray(X[m]), ref[m], rows, cols)
        exact_w = N.q4_values(W)
    else:
        A = np.zeros(rows * cols, np.float32)
        O.or_dequantize_row_q8_0(N._ptr(W), A, rows * cols, 1.0)
        A = A.reshape(rows, cols)

        def one(m):
            O.or_gemv_f32(ref[m], A, np.ascontiguousarray(X[m]), rows, cols)
        exact_w = N.q8_values(W)
    with ThreadPoolExecutor(8) as ex:
        list(ex.map(one, range(M)))
    return ref, X.astype(np.float64) @ exact_w.T



@pytest.mark.parametrize("typ,rows,cols", [(GGML_Q4_0, 11008, 4096), (GGML_Q4_0, 4096, 11008),
                                           (GGML_Q8_0, 11008, 4096), (GGML_Q8_0, 4096, 11008)])
def test_rows_gemm_full_chunk(P, typ, rows, cols):
    """One 512-row prefill chunk through the 7B FFN shapes (gate/up 11008x4096
    and down 4096x11008) against the oracle GEMV of every row."""
    name = "Q4_0" if typ == GGML_Q4_0 else "Q8_0"
    print(f"rows gemm {name} {rows}x{cols} M=512", flush=True)
    rng = np.random.default_rng(rows + cols + typ)
    W = N.rand_q4_0(rng, rows, cols) if typ == GGML_Q4_0 else N.rand_q8_0(rng, rows, cols)
    X = rng.normal(0, 1, (512, cols)).astype(np.float32)
    Y = _rows_gemm(P, typ, W, X)
    ref, exact = _oracle_rows(typ, W, X)
    ok, nfb = N.parity(Y, ref, exact)
    print(f"max |d| {np.abs(Y.astype(np.float64) - ref).max():.2e}; elements on the exact-value fallback: {nfb}; "
          f"max error vs fp64: gpu {np.abs(Y - exact).max():.2e}, oracle {np.abs(ref - exact).max():.2e}")
    assert ok, max_violation(Y, ref)


@pytest.mark.parametrize("typ", [GGML_Q4_0, GGML_Q8_0])
@pytest.mark.parametrize("mag", [1e5, 1e-6, "mixed"])
def test_rows_gemm_row_scales(P, typ, mag):
    """Hidden rows far from unit size: fp16 hi/lo of 1e5 overflows and of
    1e-6 keeps a few bits, so the rows panel scales every row by a power of
    two and the GEMM epilogue scales it back.  Each output row is compared
    relative to its own size (the fp32 bar applied to Y / s, ref / s), and a
    residual R and a 0.5 scale are carried through on the way."""
    rows, cols, M = 1024, 4096, 70
    print(f"rows gemm row scales {mag} {'Q4_0' if typ == GGML_Q4_0 else 'Q8_0'}", flush=True)
    rng = np.random.default_rng(7 + typ)
    W = N.rand_q4_0(rng, rows, cols) if typ == GGML_Q4_0 else N.rand_q8_0(rng, rows, cols)
    if mag == "mixed":
        s = np.where(np.arange(M) % 2 == 0, 1e5, 1e-6)
    else:
        s = np.full(M, mag)
    X = (rng.normal(0, 1, (M, cols)) * s[:, None]).astype(np.float32)
    R = (rng.normal(0, 1, (M, rows)) * s[:, None]).astype(np.float32)
    Y = _rows_gemm(P, typ, W, X, R, 0.5)
    ref, exact = _oracle_rows(typ, W, X)
    ref = (R.astype(np.float64) + 0.5 * ref.astype(np.float64))
    exact = R.astype(np.float64) + 0.5 * exact
    assert np.all(np.isfinite(Y))
    g, o, e = (Y / s[:, None], ref / s[:, None], exact / s[:, None])
    ok, nfb = N.parity(g, o, e)
    print(f"max |d|/s {np.abs(g - o).max():.2e}; elements on the exact-value fallback: {nfb}")
    assert ok, max_violation(g, o)


def _oracle_prefill(om, prompt, L, n_ctx, kvd, flips, near=None, idx=None):
    """The oracle's prompt forward from an empty cache with the given gate
    decisions inverted: (last-token logits, K rows [L][n][kvd], V rows)."""
    n = len(prompt)
    om.cache_len = 0
    om.m.flip = len(flips)
    for f, (j, l, col) in enumerate(flips):
        om.m.flip_tok[f], om.m.flip_layer[f], om.m.flip_col[f] = j, l, col
    if near is not None:
        om.m.gate_near, om.m.gate_near_idx = near.ctypes.data, idx.ctypes.data
    ref = np.zeros(om.n_vocab, np.float32)
    try:
        assert O.or_forward(om.ptr, prompt, n, ref) == 0
    finally:
        om.m.gate_near, om.m.gate_near_idx = None, None
        om.m.flip = 0
    kc = om.k_cache.reshape(L, n_ctx, kvd)[:, :n].copy()
    vc = om.v_cache.reshape(L, n_ctx, kvd)[:, :n].copy()
    return ref, kc, vc


def test_prefill_at_gate_threshold(P, tmp_path):
    """The large-M prefill at the reference's FFN gate-skip threshold 0.01
    (src/model.c:582-585).  The skip is a step at |silu(g)| = 0.01, so a gate
    within the two sides' rounding distance of it may fall either way.  Prompt
    tokens are explained in order: the first token whose cached K/V rows (or,
    for the last token, logits) differ must match once one or two of its own
    gate decisions at layers below the first differing one -- each within the
    fp32 rounding window 2 sqrt(d) 2^-24 of the threshold -- are inverted in
    the oracle; then the next differing token, up to 3 inversions in all.
    With no inversion needed this is the plain fp32 bar."""
    L, d, h, kv, ff, V, mt, n = 2, 256, 4, 2, 512, 512, GGML_Q4_0, 512
    print(f"prefill {n} tokens at gate threshold 0.01: {L}L d{d} ff{ff}", flush=True)
    rng = np.random.default_rng(4242)
    path = str(tmp_path / "m.gguf")
    raw = llama_gguf(path, rng, L, d, h, kv, ff, V, std=0.05, norm_random=True, emb_type=mt, out_type=mt,
                     matrix_type=mt)
    n_ctx, kvd = 1024, kv * (d // h)
    prompt = rng.integers(0, V, n).astype(np.int32)
    mp = load(P, path, n_ctx, thr=0.01)
    try:
        got = np.zeros(V, np.float32)
        assert P.vx_model_forward(mp, prompt, n, got) == 0, N.product_error()
        kg = np.zeros((L, n, kvd), np.float32)
        vg = np.zeros((L, n, kvd), np.float32)
        for l in range(L):
            assert P.vx_model_read_kv(mp, l, n, kg[l], vg[l]) == 0, N.product_error()
    finally:
        P.vx_model_destroy(mp)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=n_ctx, gate_thr=0.01)
    tol = 2.0 * np.sqrt(d) * 2.0 ** -24
    near = np.zeros((n, L), np.float32)
    idx = np.zeros((n, L), np.int32)

    def first_bad(ref, kc, vc):
        for j in range(n):
            for l in range(L):
                if not (close(kg[l, j], kc[l, j]) and close(vg[l, j], vc[l, j])):
                    return j, l
        return (None, None) if close(got, ref) else (n - 1, L)

    flips, where = [], []
    ref, kc, vc = _oracle_prefill(om, prompt, L, n_ctx, kvd, flips, near, idx)
    print(f"closest gate to the threshold: {near.min():.2e} (window {tol:.2e})")
    while True:
        j0, lb = first_bad(ref, kc, vc)
        if j0 is None:
            break
        assert len(flips) < 3, ("more gate decisions needed than 3", where, j0, lb)
        # a decision at layer l changes this token's K/V from layer l + 1 on
        cands = [(l, int(idx[j0, l]), float(near[j0, l])) for l in range(min(lb, L)) if near[j0, l] <= tol]
        assert cands, ("token", j0, "differs at layer", lb, "with no gate within the rounding window",
                       float(near[j0, :lb].min()) if lb else None, tol)
        found = None
        for combo in [[c] for c in cands] + [list(p) for p in itertools.combinations(cands, 2)]:
            if len(flips) + len(combo) > 3:
                continue
            trial = flips + [(j0, l, col) for l, col, _ in combo]
            r, k2, v2 = _oracle_prefill(om, prompt, L, n_ctx, kvd, trial, near, idx)
            j1, _ = first_bad(r, k2, v2)
            if j1 is None or j1 > j0:
                found = (trial, combo, r, k2, v2)
                break
        assert found, ("no inverted gate decision of token", j0, "explains the GPU result", cands)
        flips, (ref, kc, vc) = found[0], found[2:]
        where += [(j0, l, col, dist) for l, col, dist in found[1]]
    for j, l, col, dist in where:
        print(f"certified gate at the threshold: token {j}, layer {l}, column {col} (distance {dist:.2e})")
    print(f"last-token logits: max |diff| {np.abs(got.astype(np.float64) - ref).max():.2e} "
          f"after {len(where)} inverted decision(s)")
    assert close(got, ref), max_violation(got, ref)
    for l in range(L):
        assert close(kg[l], kc[l]) and close(vg[l], vc[l]), l


def test_prefill_after_cache_allocated_again(P, tmp_path):
    """The large-M prefill's attention workspace is sized for the cache's
    n_ctx and the attention cap.  A cache dropped (fp16-KV mode on, then off)
    and allocated again for a larger n_ctx, and a cap changed between
    prefills, must each rebuild it: a prompt past the old n_ctx and one under
    a 64-position cap both match the oracle."""
    L, d, h, kv, ff, V = 2, 256, 4, 2, 512, 300
    print("prefill after the cache is allocated again (n_ctx 256 -> 1024) and after a cap change", flush=True)
    rng = np.random.default_rng(77)
    path = str(tmp_path / "m.gguf")
    raw = llama_gguf(path, rng, L, d, h, kv, ff, V, std=0.05, norm_random=True)
    mp = load(P, path, 256)
    try:
        first = rng.integers(0, V, 200).astype(np.int32)
        lg = np.zeros(V, np.float32)
        assert P.vx_model_forward(mp, first, len(first), lg) == 0, N.product_error()
        opt = N.VxModelOptions()
        P.vx_model_get_options(mp, C.byref(opt))
        opt.kv_half = 1
        assert P.vx_model_set_options(mp, C.byref(opt)) == 0, N.product_error()
        assert mp.contents.cache_len == 0
        mp.contents.config.n_ctx = 1024
        opt.kv_half = 0
        assert P.vx_model_set_options(mp, C.byref(opt)) == 0, N.product_error()
        prompt = rng.integers(0, V, 900).astype(np.int32)
        got = np.zeros(V, np.float32)
        assert P.vx_model_forward(mp, prompt, len(prompt), got) == 0, N.product_error()
        opt.attn_cap = 64
        assert P.vx_model_set_options(mp, C.byref(opt)) == 0, N.product_error()
        P.vx_model_kv_truncate(mp, 0)
        got_cap = np.zeros(V, np.float32)
        assert P.vx_model_forward(mp, prompt[:600], 600, got_cap) == 0, N.product_error()
    finally:
        P.vx_model_destroy(mp)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=1024, gate_thr=0.0)
    ref = np.zeros(V, np.float32)
    assert O.or_forward(om.ptr, prompt, len(prompt), ref) == 0
    assert close(got, ref), max_violation(got, ref)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=1024, gate_thr=0.0, attn_cap=64)
    assert O.or_forward(om.ptr, prompt[:600], 600, ref) == 0
    assert close(got_cap, ref), max_violation(got_cap, ref)
