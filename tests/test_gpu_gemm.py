"""GPU parity of the dequant GEMM / GEMV entry points against the oracle.

Bar: |gpu - oracle| <= 1e-4 + 1e-3*|oracle| elementwise (the floating-point
tolerance of the verify path); dequantisation and repacking are bit-exact.
"""
import ctypes as C

import numpy as np
import pytest

import _native as N
from _native import close, max_violation

pytestmark = pytest.mark.gpu
O = N.oracle()


@pytest.fixture(scope="module")
def P():
    if not N.product_available():
        pytest.fail("product library not built (run __graft_entry__.build())")
    L = N.product()
    assert L.vxh_init() == 0, L.vxh_last_error()
    return L


def oracle_rows(fn, W, X, rows, cols):
    out = np.zeros((X.shape[0], rows), np.float32)
    for m in range(X.shape[0]):
        fn(N._ptr(W), np.ascontiguousarray(X[m]), out[m], rows, cols)
    return out


SHAPES = [(32, 64, 1), (96, 128, 5), (100, 96, 9), (130, 2048, 3), (256, 4096, 16),
          (4096, 4096, 5), (11008, 4096, 9), (4096, 11008, 9), (512, 3584, 7), (64, 5632, 2)]


@pytest.mark.parametrize("rows,cols,M", SHAPES)
def test_gemm_q4_0_exact(P, rows, cols, M):
    print(f"gemm_q4_0 exact rows={rows} cols={cols} M={M}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols + M)
    W = N.rand_q4_0(rng, rows, cols)
    X = rng.normal(0, 1, (M, cols)).astype(np.float32)
    Y = np.zeros((M, rows), np.float32)
    assert P.vx_gemm_q4_0(N._ptr(W), X, cols, Y, M, rows, cols, 0) == 0, N.product_error()
    ref = oracle_rows(O.or_gemv_q4_0, W, X, rows, cols)
    exact = X.astype(np.float64) @ N.q4_values(W).T
    ok, nfb = N.parity(Y, ref, exact)
    assert ok, max_violation(Y, ref)
    print(f"elements on the exact-value fallback: {nfb}")
    assert close(Y, exact, atol=2e-5, rtol=2e-5), max_violation(Y, exact, 2e-5, 2e-5)


@pytest.mark.parametrize("typ", [2, 8])
def test_gemm_every_batch_size(P, typ):
    """Every batch size 1..16 (each has its own kernel instantiation: the
    one-row and few-row GEMMs, the 64-row-tile verify kernel from 5 rows)
    on one Q4_0 / Q8_0 matrix whose row count is not a multiple of 64 and
    whose K spans several slices, against the oracle GEMV at the fp32 bar."""
    rows, cols = 200, 1536
    rng = np.random.default_rng(4242 + typ)
    W = N.rand_q4_0(rng, rows, cols) if typ == 2 else N.rand_q8_0(rng, rows, cols)
    vals = N.q4_values(W) if typ == 2 else N.q8_values(W)
    if typ == 8:
        A = np.zeros(rows * cols, np.float32)
        O.or_dequantize_row_q8_0(N._ptr(W), A, rows * cols, 1.0)
        A = A.reshape(rows, cols)
    for M in range(1, 17):
        print(f"{'Q4_0' if typ == 2 else 'Q8_0'} {rows}x{cols} M={M}", flush=True)
        X = rng.normal(0, 1, (M, cols)).astype(np.float32)
        Y = np.zeros((M, rows), np.float32)
        if typ == 2:
            assert P.vx_gemm_q4_0(N._ptr(W), X, cols, Y, M, rows, cols, 0) == 0, N.product_error()
            ref = oracle_rows(O.or_gemv_q4_0, W, X, rows, cols)
        else:
            assert P.vx_gemm_q8_0(N._ptr(W), X, cols, Y, M, rows, cols) == 0, N.product_error()
            ref = np.zeros((M, rows), np.float32)
            for m in range(M):
                O.or_gemv_f32(ref[m], A, np.ascontiguousarray(X[m]), rows, cols)
        exact = X.astype(np.float64) @ vals.T
        ok, _ = N.parity(Y, ref, exact)
        assert ok, (M, max_violation(Y, ref))


# every exact shape, plus a draft-size matrix at one row (the decode GEMV)
AVX2_SHAPES = SHAPES + [(2048, 5632, 1)]


@pytest.mark.parametrize("rows,cols,M", AVX2_SHAPES)
def test_gemm_q4_0_avx2_lanes(P, rows, cols, M):
    print(f"gemm_q4_0 avx2 rows={rows} cols={cols} M={M}", flush=True)
    rng = np.random.default_rng(rows * 5 + cols + M)
    W = N.rand_q4_0(rng, rows, cols)
    X = rng.normal(0, 1, (M, cols + 4)).astype(np.float32)   # 4-float tails are read
    Y = np.zeros((M, rows), np.float32)
    assert P.vx_gemm_q4_0(N._ptr(W), X, cols + 4, Y, M, rows, cols, 1) == 0, N.product_error()
    ref = oracle_rows(O.or_gemv_q4_0_avx2lanes, W, X, rows, cols)
    assert close(Y, ref), max_violation(Y, ref)


@pytest.mark.parametrize("rows,cols,M", [(64, 128, 1), (300, 2048, 9), (4096, 11008, 5), (1000, 3584, 16)])
def test_gemm_q8_0(P, rows, cols, M):
    print(f"gemm_q8_0 rows={rows} cols={cols} M={M}", flush=True)
    rng = np.random.default_rng(rows + cols * 3 + M)
    W = N.rand_q8_0(rng, rows, cols)
    X = rng.normal(0, 1, (M, cols)).astype(np.float32)
    Y = np.zeros((M, rows), np.float32)
    assert P.vx_gemm_q8_0(N._ptr(W), X, cols, Y, M, rows, cols) == 0, N.product_error()
    A = np.zeros(rows * cols, np.float32)
    O.or_dequantize_row_q8_0(N._ptr(W), A, rows * cols, 1.0)
    A = A.reshape(rows, cols)
    ref = np.zeros((M, rows), np.float32)
    for m in range(M):
        O.or_gemv_f32(ref[m], A, np.ascontiguousarray(X[m]), rows, cols)
    exact = X.astype(np.float64) @ N.q8_values(W).T
    ok, nfb = N.parity(Y, ref, exact)
    assert ok, max_violation(Y, ref)
    print(f"elements on the exact-value fallback: {nfb}")


def test_gemv_entry_points(P):
    rng = np.random.default_rng(31)
    rows, cols = 200, 1024
    W = N.rand_q4_0(rng, rows, cols)
    x = rng.normal(0, 1, cols + 4).astype(np.float32)
    y = np.zeros(rows, np.float32)
    r = np.zeros(rows, np.float32)
    P.vx_gemv_q4_0(N._ptr(W), x, y, rows, cols)
    O.or_gemv_q4_0(N._ptr(W), x, r, rows, cols)
    assert close(y, r)
    gate = rng.normal(0, 0.02, rows).astype(np.float32)
    P.vx_gemv_q4_0_sparse_rows(N._ptr(W), x, y, rows, cols, gate, 0.01)
    O.or_gemv_q4_0_sparse_rows(N._ptr(W), x, r, rows, cols, gate, 0.01)
    assert close(y, r) and np.all(y[np.abs(gate) < 0.01] == 0)
    P.vx_gemv_q4_0_avx2(N._ptr(W), x, y, rows, cols)
    O.or_gemv_q4_0_avx2lanes(N._ptr(W), x, r, rows, cols)
    assert close(y, r)
    P.vx_gemv_q4_0_avx2_sparse_rows(N._ptr(W), x, y, rows, cols, gate, 0.01)
    O.or_gemv_q4_0_avx2lanes_sparse_rows(N._ptr(W), x, r, rows, cols, gate, 0.01)
    assert close(y, r)
    d = C.c_float()
    P.vx_dot_q4_0(N._ptr(W[0]), x, C.byref(d), cols)
    assert close([d.value], [r[0] if False else float(N.q4_values(W[:1])[0] @ x[:cols].astype(np.float64))])


def test_dequantize_rows_bitexact(P):
    rng = np.random.default_rng(32)
    for scale in (1.0, 0.5):
        P.vx_set_synthetic_weight_scale(scale)
        for n in (32, 96, 4096):
            W = N.rand_q4_0(rng, 1, n)
            a = np.zeros(n, np.float32)
            b = np.zeros(n, np.float32)
            P.vx_dequantize_row_q4_0(N._ptr(W), a, n)
            O.or_dequantize_row_q4_0(N._ptr(W), b, n, scale)
            assert np.array_equal(a, b)
            W8 = N.rand_q8_0(rng, 1, n)
            P.vx_dequantize_row_q8_0(N._ptr(W8), a, n)
            O.or_dequantize_row_q8_0(N._ptr(W8), b, n, scale)
            assert np.array_equal(a, b)
    P.vx_set_synthetic_weight_scale(1.0)


def test_gemm_zero_and_one_hot(P):
    # one-hot activations pick one dequantised column exactly; all-8 nibbles give zero
    rng = np.random.default_rng(33)
    rows, cols = 64, 256
    W = N.rand_q4_0(rng, rows, cols)
    X = np.zeros((3, cols), np.float32)
    X[0, 0], X[1, 77], X[2, 255] = 1.0, 1.0, 1.0
    Y = np.zeros((3, rows), np.float32)
    assert P.vx_gemm_q4_0(N._ptr(W), X, cols, Y, 3, rows, cols, 0) == 0
    vals = N.q4_values(W)
    assert np.array_equal(Y[0].astype(np.float64), vals[:, 0])
    assert np.array_equal(Y[1].astype(np.float64), vals[:, 77])
    assert np.array_equal(Y[2].astype(np.float64), vals[:, 255])
    W["qs"][:] = 0x88
    X = rng.normal(0, 1, (2, cols)).astype(np.float32)
    out = np.full((2, rows), 7.0, np.float32)
    assert P.vx_gemm_q4_0(N._ptr(W), X, cols, out, 2, rows, cols, 0) == 0
    assert np.all(out == 0.0), np.abs(out).max()


class _QMat(C.Structure):
    _fields_ = [("type", C.c_int), ("n_rows", C.c_int), ("n_cols", C.c_int), ("n_pairs", C.c_int),
                ("qs", C.c_void_p), ("d", C.c_void_p), ("cached", C.c_int),
                ("tq", C.c_void_p), ("td", C.c_void_p)]


class _Panel(C.Structure):
    _fields_ = [("data", C.c_void_p), ("corr", C.c_void_p), ("rscale", C.c_void_p), ("xs", C.c_void_p),
                ("M", C.c_int), ("K", C.c_int), ("avx2", C.c_int), ("rs_ld", C.c_int)]


@pytest.mark.parametrize("typ,rows,cols,M", [(2, 2560, 2048, 1), (2, 4096, 4096, 9), (2, 4096, 11008, 5),
                                             (8, 2048, 5632, 1), (8, 1024, 4096, 9), (2, 96, 160, 16)])
def test_dot_path_matches_oracle(P, typ, rows, cols, M):
    """VXH_PATH_DOT (v_dot2_f32_f16, no MFMA) on the same panel as the MFMA
    kernel: against the oracle GEMV at the fp32 bar."""
    vp = C.c_void_p
    L = N.bind_vxh(P)
    L.vxh_qmat_alloc.argtypes = [vp, C.c_int, C.c_int, C.c_int]
    L.vxh_qmat_set_rows.argtypes = [vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, vp]
    L.vxh_qmat_free.argtypes = [vp]
    L.vxh_panel_alloc.argtypes = [vp, C.c_int, C.c_int]
    L.vxh_panel_free.argtypes = [vp]
    L.vxh_prep_panel.argtypes = [vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, vp, C.c_int, vp]
    L.vxh_gemm_acc.argtypes = [vp, vp, C.c_int, vp, C.c_int, C.c_int, C.c_float, vp, C.c_int, C.c_float, C.c_int, vp]
    L.vxh_acc_store.argtypes = [vp, C.c_int, C.c_int, C.c_int, vp, C.c_int, vp, C.c_int, vp]
    print(f"dot path {'Q4_0' if typ == 2 else 'Q8_0'} {rows}x{cols} M={M}", flush=True)
    rng = np.random.default_rng(rows + cols + M + typ)
    W = N.rand_q4_0(rng, rows, cols) if typ == 2 else N.rand_q8_0(rng, rows, cols)
    X = rng.normal(0, 1, (M, cols)).astype(np.float32)
    rows_p = (rows + 31) // 32 * 32
    q = _QMat()
    assert L.vxh_qmat_alloc(C.byref(q), typ, rows_p, cols) == 0, L.vxh_last_error()
    assert L.vxh_qmat_set_rows(C.byref(q), N._ptr(W), 0, rows, rows, 0, 0, None) == 0, L.vxh_last_error()
    pan = _Panel()
    assert L.vxh_panel_alloc(C.byref(pan), M, cols) == 0
    dx = N.DevBuf(L, X)
    acc = N.DevBuf(L, np.zeros(M * rows_p, np.float64))
    dy = N.DevBuf(L, nbytes=4 * M * rows)
    try:
        assert L.vxh_prep_panel(C.byref(pan), dx.ptr, cols, M, cols, 0, None, 0, None) == 0
        assert L.vxh_gemm_acc(C.byref(q), C.byref(pan), M, acc.ptr, rows_p, rows, 1.0, None, 0, 0.0, 2, None) == 0, \
            L.vxh_last_error()
        assert L.vxh_acc_store(acc.ptr, rows_p, M, rows, dy.ptr, rows, None, 0, None) == 0
        assert L.vxh_stream_sync(None) == 0
        Y = dy.get(np.float32, M * rows).reshape(M, rows)
    finally:
        for b in (dx, acc, dy):
            b.free()
        L.vxh_panel_free(C.byref(pan))
        L.vxh_qmat_free(C.byref(q))
    ref = np.zeros((M, rows), np.float32)
    if typ == 2:
        for m in range(M):
            O.or_gemv_q4_0(N._ptr(W), np.ascontiguousarray(X[m]), ref[m], rows, cols)
        exact = X.astype(np.float64) @ N.q4_values(W).T
    else:
        A = np.zeros(rows * cols, np.float32)
        O.or_dequantize_row_q8_0(N._ptr(W), A, rows * cols, 1.0)
        for m in range(M):
            O.or_gemv_f32(ref[m], A.reshape(rows, cols), np.ascontiguousarray(X[m]), rows, cols)
        exact = X.astype(np.float64) @ N.q8_values(W).T
    ok, nfb = N.parity(Y, ref, exact)
    print(f"max |d| {np.abs(Y.astype(np.float64) - ref).max():.2e}; elements on the exact-value fallback: {nfb}")
    assert ok, N.max_violation(Y, ref)


@pytest.mark.parametrize("typ,rows,cols,M", [(2, 2048, 5632, 1), (2, 4096, 4096, 9), (8, 1024, 4096, 9)])
def test_cached_and_streamed_weights_agree(P, typ, rows, cols, M):
    """vxh_qmat.cached = 1 (plain weight loads) against the default 0
    (non-temporal loads): the same products, bit for bit."""
    vp = C.c_void_p
    L = N.bind_vxh(P)
    L.vxh_qmat_alloc.argtypes = [vp, C.c_int, C.c_int, C.c_int]
    L.vxh_qmat_set_rows.argtypes = [vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, vp]
    L.vxh_qmat_free.argtypes = [vp]
    L.vxh_panel_alloc.argtypes = [vp, C.c_int, C.c_int]
    L.vxh_panel_free.argtypes = [vp]
    L.vxh_prep_panel.argtypes = [vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, vp, C.c_int, vp]
    L.vxh_gemm_acc.argtypes = [vp, vp, C.c_int, vp, C.c_int, C.c_int, C.c_float, vp, C.c_int, C.c_float, C.c_int, vp]
    print(f"cached vs streamed {'Q4_0' if typ == 2 else 'Q8_0'} {rows}x{cols} M={M}", flush=True)
    rng = np.random.default_rng(rows + cols + M + typ + 5)
    W = N.rand_q4_0(rng, rows, cols) if typ == 2 else N.rand_q8_0(rng, rows, cols)
    X = rng.normal(0, 1, (M, cols)).astype(np.float32)
    q = _QMat()
    assert L.vxh_qmat_alloc(C.byref(q), typ, rows, cols) == 0, L.vxh_last_error()
    assert q.cached == 0
    assert L.vxh_qmat_set_rows(C.byref(q), N._ptr(W), 0, rows, rows, 0, 0, None) == 0, L.vxh_last_error()
    pan = _Panel()
    assert L.vxh_panel_alloc(C.byref(pan), M, cols) == 0
    dx = N.DevBuf(L, X)
    accs = [N.DevBuf(L, np.zeros(M * rows, np.float64)) for _ in range(2)]
    try:
        assert L.vxh_prep_panel(C.byref(pan), dx.ptr, cols, M, cols, 0, None, 0, None) == 0
        for cached, acc in zip((0, 1), accs):
            q.cached = cached
            assert L.vxh_gemm_acc(C.byref(q), C.byref(pan), M, acc.ptr, rows, rows, 1.0, None, 0, 0.0, 0,
                                  None) == 0, L.vxh_last_error()
        assert L.vxh_stream_sync(None) == 0
        got = [a.get(np.float64, M * rows) for a in accs]
    finally:
        for b in [dx] + accs:
            b.free()
        L.vxh_panel_free(C.byref(pan))
        L.vxh_qmat_free(C.byref(q))
    assert np.any(got[0] != 0.0)
    assert np.array_equal(got[0], got[1])
