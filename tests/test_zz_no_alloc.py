"""vxh_gemm_noalloc (static device scratch, no allocation) against vxh_gemm
(workspace argument) on the same inputs, through the C ABI: two calls in a
row, the second smaller, each compared with the workspace entry point and
with the oracle GEMV; and the size limit refused before any launch."""
import ctypes as C

import numpy as np
import pytest

import _native as N

pytestmark = pytest.mark.gpu
O = N.oracle()
vp = C.c_void_p


class Panel(C.Structure):
    _fields_ = [("data", vp), ("corr", vp), ("rscale", vp), ("xs", vp),
                ("M", C.c_int), ("K", C.c_int), ("avx2", C.c_int), ("rs_ld", C.c_int)]


class QMat(C.Structure):
    _fields_ = [("type", C.c_int), ("n_rows", C.c_int), ("n_cols", C.c_int), ("n_pairs", C.c_int),
                ("qs", vp), ("d", vp), ("cached", C.c_int),
                ("tq", vp), ("td", vp)]


class Epi(C.Structure):
    _fields_ = [("kind", C.c_int), ("y", vp), ("ldy", C.c_int), ("r", vp), ("ldr", C.c_int),
                ("thr", C.c_float), ("scale", C.c_float), ("n_out", C.c_int)]


class Workspace(C.Structure):
    _fields_ = [("acc", vp), ("acc_elems", C.c_size_t), ("part", vp), ("part_floats", C.c_size_t)]


EPI_STORE, EPI_RESID = 0, 1


@pytest.fixture(scope="module")
def P():
    if not N.product_available():
        pytest.fail("product library not built")
    L = N.bind_vxh(N.product())
    assert L.vxh_init() == 0, L.vxh_last_error()
    L.vxh_qmat_alloc.argtypes = [vp, C.c_int, C.c_int, C.c_int]
    L.vxh_qmat_set_rows.argtypes = [vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, vp]
    L.vxh_qmat_free.argtypes = [vp]
    L.vxh_panel_alloc.argtypes = [vp, C.c_int, C.c_int]
    L.vxh_panel_free.argtypes = [vp]
    L.vxh_prep_panel.argtypes = [vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, vp, C.c_int, vp]
    L.vxh_workspace_alloc.argtypes = [vp, C.c_size_t, C.c_size_t]
    L.vxh_workspace_free.argtypes = [vp]
    L.vxh_gemm.argtypes = [vp, vp, C.c_int, vp, vp, C.c_int, vp]
    L.vxh_gemm_noalloc.argtypes = [vp, vp, C.c_int, vp, C.c_int, vp]
    L.vxh_gemm_workspace_elems.restype = C.c_size_t
    L.vxh_gemm_workspace_elems.argtypes = [C.c_int, C.c_int]
    return L


def run_case(P, rows, cols, M, kind, seed):
    rng = np.random.default_rng(seed)
    W = N.rand_q4_0(rng, rows, cols)
    X = rng.normal(0, 1, (M, cols)).astype(np.float32)
    R = rng.normal(0, 1, (M, rows)).astype(np.float32)
    q = QMat()
    assert P.vxh_qmat_alloc(C.byref(q), 2, rows, cols) == 0, P.vxh_last_error()
    assert P.vxh_qmat_set_rows(C.byref(q), N._ptr(W), 0, rows, rows, 0, 0, None) == 0, P.vxh_last_error()
    pan = Panel()
    assert P.vxh_panel_alloc(C.byref(pan), M, cols) == 0, P.vxh_last_error()
    dx, dr = N.DevBuf(P, X), N.DevBuf(P, R)
    y_ws = N.DevBuf(P, np.full((M, rows), 7.0, np.float32))
    y_na = N.DevBuf(P, np.full((M, rows), -7.0, np.float32))
    ws = Workspace()
    assert P.vxh_workspace_alloc(C.byref(ws), P.vxh_gemm_workspace_elems(rows, M), 32) == 0
    try:
        assert P.vxh_prep_panel(C.byref(pan), dx.ptr, cols, M, cols, 0, None, 0, None) == 0, P.vxh_last_error()
        outs = []
        for y, noalloc in ((y_ws, False), (y_na, True)):
            e = Epi(kind=kind, y=y.ptr, ldy=rows, r=dr.ptr if kind == EPI_RESID else None, ldr=rows,
                    thr=0.0, scale=1.0, n_out=rows)
            if noalloc:
                rc = P.vxh_gemm_noalloc(C.byref(q), C.byref(pan), M, C.byref(e), 0, None)
            else:
                rc = P.vxh_gemm(C.byref(q), C.byref(pan), M, C.byref(e), C.byref(ws), 0, None)
            assert rc == 0, P.vxh_last_error()
            assert P.vxh_stream_sync(None) == 0
            outs.append(y.get(np.float32, M * rows).reshape(M, rows))
    finally:
        for b in (dx, dr, y_ws, y_na):
            b.free()
        P.vxh_workspace_free(C.byref(ws))
        P.vxh_panel_free(C.byref(pan))
        P.vxh_qmat_free(C.byref(q))
    ref = np.zeros((M, rows), np.float32)
    for m in range(M):
        O.or_gemv_q4_0(N._ptr(W), np.ascontiguousarray(X[m]), ref[m], rows, cols)
    if kind == EPI_RESID:
        ref = ref + R
    return outs[0], outs[1], ref


def test_noalloc_gemm_matches_workspace_gemm_twice(P):
    """Two calls in a row on the shared static scratch, the second smaller."""
    for rows, cols, M, kind, seed in ((4096, 4096, 9, EPI_STORE, 1), (1024, 2048, 3, EPI_RESID, 2)):
        print(f"noalloc gemm {rows}x{cols} M={M} kind={kind}", flush=True)
        y_ws, y_na, ref = run_case(P, rows, cols, M, kind, seed)
        print(f"  identical to vxh_gemm: {np.array_equal(y_ws, y_na)}; max |d| vs oracle "
              f"{np.abs(y_na.astype(np.float64) - ref).max():.2e}")
        assert N.close(y_na, y_ws), N.max_violation(y_na, y_ws)
        assert N.close(y_na, ref), N.max_violation(y_na, ref)


def test_noalloc_gemm_refuses_sizes_beyond_its_scratch(P):
    """M x rows above VXH_NOALLOC_ACC_ELEMS is refused on the host, before
    anything is launched: the output keeps its contents."""
    limit = 1 << 19
    rows, cols, M = 33024, 64, 16
    assert P.vxh_gemm_workspace_elems(rows, M) > limit
    q = QMat()
    assert P.vxh_qmat_alloc(C.byref(q), 2, rows, cols) == 0, P.vxh_last_error()
    pan = Panel()
    assert P.vxh_panel_alloc(C.byref(pan), M, cols) == 0
    y = N.DevBuf(P, np.full((M, rows), 5.0, np.float32))
    try:
        e = Epi(kind=EPI_STORE, y=y.ptr, ldy=rows, r=None, ldr=0, thr=0.0, scale=1.0, n_out=rows)
        rc = P.vxh_gemm_noalloc(C.byref(q), C.byref(pan), M, C.byref(e), 0, None)
        assert rc == -3, rc
        assert b"static scratch" in P.vxh_last_error()
        assert P.vxh_stream_sync(None) == 0
        assert np.all(y.get(np.float32, M * rows) == 5.0)
    finally:
        y.free()
        P.vxh_panel_free(C.byref(pan))
        P.vxh_qmat_free(C.byref(q))
