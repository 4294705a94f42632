"""GPU acceptance sampling (vxh_row_stats / vxh_sample / vxh_accept, and
their many-workgroup forms vxh_row_stats_mc / vxh_sample_keep_mc /
vxh_accept_mc) against the oracle on identical logits and uniforms.

Decisions must be identical.  A difference is accepted only as a certified
tie: the uniform sits within 1e-5 of the acceptance ratio, or the fixed-point
CDF threshold sits within 1e-6 of the mass of a token boundary -- places where
the last-ulp differences of expf between the GPU and the host libm may flip
the outcome.  Every such case is counted and reported.
"""
import ctypes as C

import numpy as np
import pytest

import _native as N

pytestmark = pytest.mark.gpu
O = N.oracle()


@pytest.fixture(scope="module")
def P():
    if not N.product_available():
        pytest.fail("product library not built")
    L = N.bind_vxh(N.product())
    assert L.vxh_init() == 0, L.vxh_last_error()
    return L


_WS = {}


def vocab_ws(P):
    """One many-workgroup workspace for the module (65 rows)."""
    if "ws" not in _WS:
        ws = N.VxhVocabWs()
        assert P.vxh_vocab_ws_alloc(C.byref(ws), 65) == 0, P.vxh_last_error()
        _WS["ws"] = ws
    return _WS["ws"]


def fixed(w):
    w = np.asarray(w, np.float64)
    return np.where(w > 0, np.floor(w * 2.0 ** 32 + 0.5), 0).astype(np.uint64)


def near_boundary(w, u):
    """True when the inverse-CDF threshold of u lies within 1e-6 of the total
    mass of a prefix boundary (a certified tie)."""
    W = fixed(w)
    S = int(W.sum())
    if S == 0:
        return False
    U = int(np.float32(u) * np.float32(16777216.0))
    thr = max(1, (U * S + 16777215) >> 24)
    c = np.cumsum(W.astype(np.float64))
    return bool(np.min(np.abs(c - thr)) <= 1e-6 * S + 2)


def sample_gpu(P, l, T, top_p, u, mc=False):
    V = l.shape[0]
    dl, du = N.DevBuf(P, l), N.DevBuf(P, np.array([u], np.float32))
    dt, dn = N.DevBuf(P, nbytes=4), N.DevBuf(P, nbytes=32)
    if mc:
        assert P.vxh_sample_keep_mc(dl.ptr, V, T, top_p, du.ptr, dt.ptr, dn.ptr, None, C.byref(vocab_ws(P)),
                                    None) == 0, P.vxh_last_error()
    else:
        assert P.vxh_sample(dl.ptr, V, T, top_p, du.ptr, dt.ptr, dn.ptr, None) == 0, P.vxh_last_error()
    tok = int(dt.get(np.int32, 1)[0])
    nuc = dn.get(np.float32, 8)
    for b in (dl, du, dt, dn):
        b.free()
    return tok, nuc


@pytest.mark.parametrize("mc", [False, True])
@pytest.mark.parametrize("V,T,top_p", [(32000, 0.8, 1.0), (32000, 1.0, 0.9), (5000, 0.7, 0.5),
                                       (152064, 1.0, 1.0), (152064, 1.0, 0.95), (1000, 0.0, 1.0),
                                       (70001, 0.9, 1.0),
                                       # sharp and flat distributions; a nucleus of the top token
                                       # (top_p <= 0 and 1e-6) and one past the whole mass (1.5)
                                       (5000, 0.1, 1.0), (5000, 3.0, 0.9), (5000, 0.8, 0.0),
                                       (5000, 0.8, -0.5), (5000, 0.8, 1e-6), (5000, 0.8, 1.5),
                                       # vocabularies of one to three entries
                                       (1, 0.8, 1.0), (2, 0.8, 0.5), (3, 1.0, 1.0)])
def test_sampler_matches_oracle(P, V, T, top_p, mc):
    print(f"sampler V={V} T={T} top_p={top_p} {'many workgroups' if mc else 'one workgroup'}", flush=True)
    rng = np.random.default_rng(V + int(T * 10) + int(top_p * 100))
    ties = boundary = 0
    for trial in range(6):
        l = (rng.normal(0, 2.0, V)).astype(np.float32)
        for u in rng.integers(0, 1 << 24, 4) / float(1 << 24):
            u = float(np.float32(u))
            q = np.zeros(V, np.float32)
            want = O.or_sample_top_p(l, V, T, top_p, u, q.ctypes.data_as(C.c_void_p))
            got, nuc = sample_gpu(P, l, T, top_p, u, mc)
            if got != want:
                w = np.where(q > 0, q, 0)
                assert near_boundary(w, u), (trial, u, got, want)
                ties += 1
            if T > 0 and top_p < 1.0:
                # nucleus membership from the GPU descriptor equals the oracle's
                p = np.zeros(V, np.float32)
                O.or_softmax_temp(l, V, T, p)
                tau, tie = nuc[2], nuc[3:4].view(np.int32)[0]
                member = (p > tau) | ((p == tau) & (np.arange(V) <= tie))
                diff = member != (q > 0)
                # a sequential fp32 sum over V terms (the reference's softmax)
                # carries ~sqrt(V)*6e-8 relative error, which moves the top-p
                # boundary by a few tokens of near-equal probability: every
                # differing token must sit at the boundary value
                if np.any(diff):
                    rel = np.abs(p[diff].astype(np.float64) - tau) / tau
                    assert np.all(rel < 1e-3), (np.count_nonzero(diff), rel.max())
                    boundary += 1
    print(f"certified draw ties: {ties}; draws with boundary-only nucleus differences: {boundary}")
    assert ties <= 2


@pytest.mark.parametrize("V,T,top_p", [(32000, 0.8, 1.0), (1001, 0.0, 1.0), (5000, 0.7, 0.5), (40000, 1.0, 1.0)])
def test_sample_keep_copies_the_row_and_draws_like_sample(P, V, T, top_p):
    """vxh_sample_keep = vxh_sample plus a copy of the row (register sampler:
    the copy is stored as the row is loaded; other cases: a device copy)."""
    print(f"sample_keep V={V} T={T} top_p={top_p}", flush=True)
    rng = np.random.default_rng(V + 7)
    l = rng.normal(0, 2.0, V).astype(np.float32)
    dl, du = N.DevBuf(P, l), N.DevBuf(P, np.array([0.37], np.float32))
    keep = N.DevBuf(P, np.full(V + 4, -7.0, np.float32))
    bufs = [N.DevBuf(P, nbytes=4) for _ in range(2)] + [N.DevBuf(P, nbytes=32) for _ in range(2)]
    assert P.vxh_sample(dl.ptr, V, T, top_p, du.ptr, bufs[0].ptr, bufs[2].ptr, None) == 0, P.vxh_last_error()
    assert P.vxh_sample_keep(dl.ptr, V, T, top_p, du.ptr, bufs[1].ptr, bufs[3].ptr, keep.ptr, None) == 0, \
        P.vxh_last_error()
    assert P.vxh_stream_sync(None) == 0
    got = keep.get(np.float32, V + 4)
    assert np.array_equal(got[:V], l) and np.all(got[V:] == -7.0)
    assert bufs[0].get(np.int32, 1)[0] == bufs[1].get(np.int32, 1)[0]
    assert np.array_equal(bufs[2].get(np.uint32, 8), bufs[3].get(np.uint32, 8))
    for b in [dl, du, keep] + bufs:
        b.free()


def run_accept(P, L, D, drafts, T, top_p, u, mc=False):
    k = D.shape[0]
    V, Vd = L.shape[1], D.shape[1]
    dL, dD = N.DevBuf(P, L), N.DevBuf(P, D)
    dstats = N.DevBuf(P, nbytes=4 * 3 * (k + 1))
    dnuc = N.DevBuf(P, nbytes=4 * 8 * max(k, 1))
    ddr = N.DevBuf(P, np.asarray(drafts, np.int32))
    du1 = N.DevBuf(P, nbytes=4)
    dtok = N.DevBuf(P, nbytes=4)
    dout = N.DevBuf(P, nbytes=4 * (k + 3))
    # nucleus descriptors of the draft rows via the sampler (draws discarded)
    for j in range(k):
        P.vxh_upload(du1.ptr, np.array([0.5], np.float32).ctypes.data_as(C.c_void_p), 4, None)
        row = C.c_void_p(dD.ptr.value + j * Vd * 4)
        nj = C.c_void_p(dnuc.ptr.value + j * 32)
        assert P.vxh_sample(row, Vd, T, top_p, du1.ptr, dtok.ptr, nj, None) == 0
    du = N.DevBuf(P, np.asarray(u, np.float32))
    if mc:
        ws = C.byref(vocab_ws(P))
        assert P.vxh_row_stats_mc(dL.ptr, V, k + 1, V, T, dstats.ptr, ws, None) == 0, P.vxh_last_error()
        assert P.vxh_accept_mc(dL.ptr, V, V, dstats.ptr, dD.ptr, Vd, Vd, dnuc.ptr, ddr.ptr, k, T, du.ptr,
                               dout.ptr, ws, None) == 0, P.vxh_last_error()
    else:
        assert P.vxh_row_stats(dL.ptr, V, k + 1, V, T, dstats.ptr, None) == 0
        assert P.vxh_accept(dL.ptr, V, V, dstats.ptr, dD.ptr, Vd, Vd, dnuc.ptr, ddr.ptr, k, T, du.ptr,
                            dout.ptr, None) == 0, P.vxh_last_error()
    out = dout.get(np.int32, k + 3)
    for b in (dL, dD, dstats, dnuc, ddr, du1, dtok, dout, du):
        b.free()
    return int(out[0]), int(out[1]), list(out[2:2 + out[0]])


def oracle_accept(L, D, drafts, T, top_p, u):
    k, Vd = D.shape
    V = L.shape[1]
    Q = np.zeros((k, Vd), np.float32)
    for j in range(k):
        O.or_sample_top_p(np.ascontiguousarray(D[j]), Vd, T, top_p, 0.5, Q[j].ctypes.data_as(C.c_void_p))
    out = np.zeros(k + 1, np.int32)
    na = C.c_int()
    if T > 0:
        n = O.or_accept_sampled(np.ascontiguousarray(L.ravel()), V, np.ascontiguousarray(Q.ravel()), Vd,
                                np.asarray(drafts, np.int32), k, T, np.asarray(u, np.float32), out,
                                C.byref(na))
    else:
        n = O.or_accept_greedy(np.ascontiguousarray(L.ravel()), V, np.asarray(drafts, np.int32), k, out)
        na.value = n - 1
    return n, na.value, list(out[:n]), Q


@pytest.mark.parametrize("mc", [False, True])
@pytest.mark.parametrize("V,k,T,top_p", [(32000, 8, 0.8, 1.0), (32000, 4, 1.0, 0.95), (2000, 8, 0.8, 1.0),
                                         (32000, 8, 0.0, 1.0), (152064, 8, 1.0, 1.0), (2, 8, 0.8, 1.0),
                                         (3, 4, 1.0, 0.0)])
def test_accept_matches_oracle(P, V, k, T, top_p, mc):
    print(f"accept V={V} k={k} T={T} top_p={top_p} {'many workgroups' if mc else 'one workgroup'}", flush=True)
    rng = np.random.default_rng(V + k)
    ties, n_acc_total, n_cases = 0, 0, 12
    for case in range(n_cases):
        L = rng.normal(0, 1.5, (k + 1, V)).astype(np.float32)
        # drafts close to the target so that some, not all, drafts are accepted
        D = (L[:k] + rng.normal(0, 0.3 + 0.2 * (case % 4), (k, V))).astype(np.float32)
        drafts = []
        for j in range(k):
            if T > 0:
                drafts.append(O.or_sample_top_p(np.ascontiguousarray(D[j]), V, T, top_p,
                                                float(rng.integers(0, 1 << 24) / float(1 << 24)), None))
            else:
                am = int(np.argmax(L[j]))
                drafts.append(am if rng.random() < 0.8 else (am + 1) % V)
        u = (rng.integers(0, 1 << 24, k + 1) / float(1 << 24)).astype(np.float32)
        g = run_accept(P, L, D, drafts, T, top_p, u, mc)
        n, na, toks, Q = oracle_accept(L, D, drafts, T, top_p, u)
        n_acc_total += na
        if (g[0], g[1], g[2]) != (n, na, toks):
            # certify: ratio test tie or CDF-boundary tie at the decision that differs
            j = min(g[1], na)
            p = np.zeros(V, np.float32)
            O.or_softmax_temp(np.ascontiguousarray(L[j]), V, T, p)
            if j < k:
                alpha = min(1.0, p[drafts[j]] / max(Q[j][drafts[j]], 1e-10))
                tie = abs(float(u[j]) - alpha) < 1e-5
                if not tie and g[1] == na:
                    tie = near_boundary(np.maximum(0, p - Q[j]), float(u[k]))
            else:
                tie = near_boundary(p, float(u[k]))
            assert tie, (case, g, (n, na, toks))
            ties += 1
    print(f"accepted {n_acc_total} of {k * n_cases} drafts; certified ties {ties}")
    assert ties <= 1
    if T > 0:
        assert 0 < n_acc_total < k * n_cases


@pytest.mark.parametrize("V", [32000, 152064, 1500])
def test_many_workgroup_kernels_equal_one_workgroup_kernels(P, V):
    """Row statistics (argmax bit-equal; max and sum within fp32 rounding of
    each other), the draw and the decision of the many-workgroup kernels
    against the one-workgroup kernels on the same inputs: the same tokens
    wherever the fixed-point threshold is not within rounding of a token
    boundary; each launch leaves the workspace's counters at zero for the
    next (they run back to back here)."""
    print(f"many vs one workgroup V={V}", flush=True)
    rng = np.random.default_rng(V)
    ws = C.byref(vocab_ws(P))
    R = 9
    Lg = rng.normal(0, 2.0, (R, V)).astype(np.float32)
    Lg[3, 7] = Lg[3].max() + 1.0      # a unique maximum early in a row
    Lg[4, :] = 0.5                    # a flat row: argmax 0
    dL = N.DevBuf(P, Lg)
    s1, s2 = N.DevBuf(P, nbytes=4 * 3 * R), N.DevBuf(P, nbytes=4 * 3 * R)
    for T in (0.8, 0.0):
        assert P.vxh_row_stats(dL.ptr, V, R, V, T, s1.ptr, None) == 0
        assert P.vxh_row_stats_mc(dL.ptr, V, R, V, T, s2.ptr, ws, None) == 0, P.vxh_last_error()
        a, b = s1.get(np.float32, 3 * R).reshape(R, 3), s2.get(np.float32, 3 * R).reshape(R, 3)
        assert np.array_equal(a[:, 2].view(np.int32), b[:, 2].view(np.int32))
        assert np.array_equal(a[:, 0], b[:, 0])
        assert np.allclose(a[:, 1], b[:, 1], rtol=1e-5, atol=0)
    keep = N.DevBuf(P, nbytes=4 * V)
    du, dt, dn = N.DevBuf(P, nbytes=4), N.DevBuf(P, nbytes=4), N.DevBuf(P, nbytes=32)
    same = 0
    for trial in range(20):
        u = np.array([rng.integers(0, 1 << 24) / float(1 << 24)], np.float32)
        P.vxh_upload(du.ptr, u.ctypes.data_as(C.c_void_p), 4, None)
        row = C.c_void_p(dL.ptr.value + 4 * V * (trial % R))
        assert P.vxh_sample_keep(row, V, 0.8, 1.0, du.ptr, dt.ptr, dn.ptr, None, None) == 0
        t1 = int(dt.get(np.int32, 1)[0])
        assert P.vxh_sample_keep_mc(row, V, 0.8, 1.0, du.ptr, dt.ptr, dn.ptr, keep.ptr, ws, None) == 0
        t2 = int(dt.get(np.int32, 1)[0])
        assert np.array_equal(keep.get(np.float32, V), Lg[trial % R])
        if t1 == t2:
            same += 1
        else:
            p = np.exp((Lg[trial % R].astype(np.float64) - Lg[trial % R].max()) / 0.8)
            assert near_boundary(p / p.sum(), float(u[0])), (trial, t1, t2)
    print(f"draws equal: {same} of 20")
    assert same >= 18
    for b in (dL, s1, s2, keep, du, dt, dn):
        b.free()


def test_argmax_of_rows_without_a_maximum_is_index_zero(P):
    """A row with no value above -inf (all NaN, all -inf) has no first max;
    the kernels return index 0 (the reference's scan stays on its first
    element, src/speculative.c:93-98) instead of an index outside the row."""
    V = 3000
    rows = np.stack([np.full(V, np.nan, np.float32), np.full(V, -np.inf, np.float32)])
    dL = N.DevBuf(P, rows)
    dstats = N.DevBuf(P, nbytes=4 * 3 * 2)
    assert P.vxh_row_stats(dL.ptr, V, 2, V, 1.0, dstats.ptr, None) == 0, P.vxh_last_error()
    st = dstats.get(np.float32, 6)
    assert st[2:3].view(np.int32)[0] == 0 and st[5:6].view(np.int32)[0] == 0
    assert P.vxh_row_stats_mc(dL.ptr, V, 2, V, 1.0, dstats.ptr, C.byref(vocab_ws(P)), None) == 0
    st = dstats.get(np.float32, 6)
    assert st[2:3].view(np.int32)[0] == 0 and st[5:6].view(np.int32)[0] == 0
    for T in (0.0, 1.0):
        for r in rows:
            for mc in (False, True):
                tok, _ = sample_gpu(P, r, T, 1.0, 0.5, mc)
                assert 0 <= tok < V
    dL.free()
    dstats.free()
