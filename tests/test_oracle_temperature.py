"""Pins of the oracle's temperature path (CPU only).

The reference scales logits by 1/T before its softmax in sample_top_p
(src/speculative.c:44-53: exp((l - max) / T)).  The oracle restates that in
or_softmax_temp and uses it in or_sample_top_p and or_accept_sampled.  Every
check here compares against a numpy float64 closed form of
softmax(l / T) at T != 1, so that a slip in the temperature (l * T, a missing
max shift, T applied to only one of p and q) fails: the accept ratio, the
nucleus, the residual resample, the bonus draw and the speculative-sampling
theorem (the emitted token is distributed as the target's softmax(l / T)).
"""
import ctypes as C

import numpy as np
import pytest

import _native as N

O = N.oracle()


def softmax_t(l, T):
    """numpy float64 closed form of the reference's sample_top_p softmax."""
    z = (np.asarray(l, np.float64) - np.max(l)) / T
    e = np.exp(z)
    return e / e.sum()


def nucleus(p, top_p):
    """Shortest prefix of tokens by descending p (ties: lower index) with mass
    >= top_p, renormalised; all tokens when top_p >= 1."""
    if top_p >= 1.0:
        return p / p.sum()
    order = np.lexsort((np.arange(len(p)), -p))
    c = np.cumsum(p[order])
    cut = int(np.searchsorted(c, top_p)) + 1
    q = np.zeros_like(p)
    q[order[:cut]] = p[order[:cut]]
    return q / q.sum()


def u_grid(n):
    return (np.arange(n) / float(n)).astype(np.float32)


@pytest.mark.parametrize("T", [0.5, 0.8, 1.7])
def test_softmax_temp_closed_form(T):
    rng = np.random.default_rng(int(T * 10))
    l = rng.normal(0, 3.0, 1000).astype(np.float32)
    p = np.zeros(1000, np.float32)
    O.or_softmax_temp(l, 1000, T, p)
    ref = softmax_t(l, T)
    # fp32 expf and a sequential fp32 sum over 1000 terms
    assert np.allclose(p, ref, rtol=2e-5, atol=1e-12), np.max(np.abs(p - ref) / ref)
    # the temperature matters: the T = 1 distribution is far from it
    assert np.max(np.abs(softmax_t(l, 1.0) - ref)) > 1e-3


@pytest.mark.parametrize("T,top_p", [(0.5, 1.0), (0.8, 1.0), (0.8, 0.9), (0.5, 0.75)])
def test_sample_top_p_temperature_closed_form(T, top_p):
    rng = np.random.default_rng(int(T * 100 + top_p * 10))
    V = 24
    while True:
        l = rng.normal(0, 1.5, V).astype(np.float32)
        p = softmax_t(l, T)
        c = np.cumsum(np.sort(p)[::-1])
        if top_p >= 1.0 or np.min(np.abs(c - top_p)) > 1e-3:
            break   # no token sits at the nucleus boundary
    want = nucleus(p, top_p)
    q = np.zeros(V, np.float32)
    counts = np.zeros(V)
    n = 1 << 13
    for u in u_grid(n):
        t = O.or_sample_top_p(l, V, T, top_p, float(u), q.ctypes.data_as(C.c_void_p))
        counts[t] += 1
    assert np.array_equal(q > 0, want > 0)
    assert np.allclose(q, want, rtol=1e-5, atol=1e-9)
    # the inverse CDF over a uniform grid reproduces q to the grid's resolution
    assert np.allclose(counts / n, want, atol=2.0 / n, rtol=0)


@pytest.mark.parametrize("T", [0.5, 0.8])
def test_accept_ratio_uses_tempered_probabilities(T):
    """accept d_j iff u_j < min(1, p_j(d_j) / q_j(d_j)) with p_j = softmax(L_j/T)
    and q_j = softmax(D_j/T): u just below alpha accepts, just above rejects."""
    rng = np.random.default_rng(31 + int(T * 10))
    V, k = 30, 3
    checked = 0
    for _ in range(200):
        L = rng.normal(0, 1.5, (k + 1, V)).astype(np.float32)
        D = rng.normal(0, 1.5, (k, V)).astype(np.float32)
        Q = np.zeros((k, V), np.float32)
        for j in range(k):
            O.or_softmax_temp(D[j].copy(), V, T, Q[j])
        drafts = rng.integers(0, V, k).astype(np.int32)
        p0 = softmax_t(L[0], T)
        q0 = softmax_t(D[0], T)
        alpha = min(1.0, p0[drafts[0]] / q0[drafts[0]])
        if not 0.05 < alpha < 0.95:
            continue
        out = np.zeros(k + 1, np.int32)
        na = C.c_int()
        for du, accept in ((-2e-3, True), (2e-3, False)):
            u = np.full(k + 1, 0.5, np.float32)
            u[0] = np.float32(alpha + du)
            u[1:k] = 1.0 - 2 ** -24   # later positions reject: one decision per call
            n = O.or_accept_sampled(np.ascontiguousarray(L.ravel()), V, np.ascontiguousarray(Q.ravel()), V,
                                    drafts, k, T, u, out, C.byref(na))
            if accept:
                assert na.value >= 1 and out[0] == drafts[0], (alpha, u[0])
            else:
                assert n == 1 and na.value == 0, (alpha, u[0])
        checked += 1
        if checked == 12:
            break
    assert checked == 12


@pytest.mark.parametrize("T", [0.5, 0.8])
def test_residual_resample_uses_tempered_probabilities(T):
    """On a reject the replacement is the inverse CDF of max(0, p - q) with
    p = softmax(L/T): over a grid of u_k it reproduces that distribution."""
    rng = np.random.default_rng(41 + int(T * 10))
    V, k = 16, 1
    L = rng.normal(0, 1.5, (k + 1, V)).astype(np.float32)
    D = rng.normal(0, 1.5, (k, V)).astype(np.float32)
    Q = np.zeros((k, V), np.float32)
    O.or_softmax_temp(D[0].copy(), V, T, Q[0])
    p, q = softmax_t(L[0], T), softmax_t(D[0], T)
    d0 = int(np.argmax(q - p))          # q > p here: rejected for u near 1
    res = np.maximum(0.0, p - q)
    want = res / res.sum()
    counts = np.zeros(V)
    n = 1 << 12
    out = np.zeros(k + 1, np.int32)
    na = C.c_int()
    for uk in u_grid(n):
        u = np.array([1.0 - 2 ** -24, uk], np.float32)
        assert O.or_accept_sampled(np.ascontiguousarray(L.ravel()), V, Q.ravel().copy(), V,
                                   np.array([d0], np.int32), k, T, u, out, C.byref(na)) == 1
        counts[out[0]] += 1
    assert np.allclose(counts / n, want, atol=2.0 / n + 1e-5, rtol=0)


@pytest.mark.parametrize("T", [0.5, 0.8])
def test_bonus_draw_uses_tempered_probabilities(T):
    """After k accepts the bonus token is drawn from softmax(L_k / T)."""
    rng = np.random.default_rng(51 + int(T * 10))
    V, k = 12, 2
    L = rng.normal(0, 1.5, (k + 1, V)).astype(np.float32)
    Q = np.zeros((k, V), np.float32)
    for j in range(k):
        O.or_softmax_temp(L[j].copy(), V, T, Q[j])    # q == p: every draft accepted
    drafts = np.array([3, 7], np.int32)
    want = softmax_t(L[k], T)
    counts = np.zeros(V)
    n = 1 << 12
    out = np.zeros(k + 1, np.int32)
    na = C.c_int()
    for uk in u_grid(n):
        u = np.array([0.0, 0.0, uk], np.float32)
        assert O.or_accept_sampled(np.ascontiguousarray(L.ravel()), V, np.ascontiguousarray(Q.ravel()), V,
                                   drafts, k, T, u, out, C.byref(na)) == k + 1
        counts[out[k]] += 1
    assert np.allclose(counts / n, want, atol=2.0 / n + 1e-5, rtol=0)


@pytest.mark.parametrize("T,top_p", [(0.8, 0.9), (0.5, 1.0)])
def test_emitted_token_is_target_distributed_at_temperature(T, top_p):
    """Speculative-sampling theorem at T != 1 with a nucleus draft: a draft
    drawn from the nucleus of softmax(D/T), accepted or replaced by the
    residual resample, is distributed as softmax(L/T) (closed form)."""
    rng = np.random.default_rng(12 + int(T * 10))
    V = 6
    L = rng.normal(0, 1, (2, V)).astype(np.float32)
    D = rng.normal(0, 1, V).astype(np.float32)
    q = np.zeros(V, np.float32)
    O.or_sample_top_p(D, V, T, top_p, 0.5, q.ctypes.data_as(C.c_void_p))
    want = softmax_t(L[0], T)
    counts = np.zeros(V)
    out = np.zeros(2, np.int32)
    na = C.c_int()
    n_trials = 40000
    for _ in range(n_trials):
        u = (rng.integers(0, 1 << 24, 3) / float(1 << 24)).astype(np.float32)
        d = O.or_sample_top_p(D, V, T, top_p, float(u[2]), None)
        O.or_accept_sampled(L.ravel().copy(), V, q, V, np.array([d], np.int32), 1, T, u[:2].copy(), out,
                            C.byref(na))
        counts[out[0]] += 1
    assert np.allclose(counts / n_trials, want, atol=0.012, rtol=0)
    # the T = 1 distribution differs from the target by more than the tolerance
    assert np.max(np.abs(softmax_t(L[0], 1.0) - want)) > 0.03


@pytest.mark.parametrize("top_p", [0.0, -0.5, 1e-12])
def test_nucleus_of_a_non_positive_top_p_is_the_first_token(top_p):
    """The reference's cutoff loop (src/speculative.c:67-74) stops at the
    first sorted token once cumsum >= top_p, so top_p <= 0 (or below one
    2^-32 unit) keeps exactly the most probable token, the lowest index
    among equal maxima: every draw returns it and q is one-hot."""
    rng = np.random.default_rng(5)
    V = 40
    l = rng.normal(0, 1.0, V).astype(np.float32)
    l[[7, 23]] = l.max() + 1.0          # two equal maxima: the lower index wins
    q = np.zeros(V, np.float32)
    for u in (0.0, 0.3, 0.999):
        t = O.or_sample_top_p(l, V, 0.8, top_p, u, q.ctypes.data_as(C.c_void_p))
        assert t == 7
        want = np.zeros(V, np.float32)
        want[7] = 1.0
        assert np.array_equal(q, want)
