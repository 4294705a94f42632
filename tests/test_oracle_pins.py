"""Pins for the CPU oracle (oracle/oracle.c), CPU only.

Each oracle function is checked against (a) the reference engine compiled from
its own sources (oracle/_ref, built by oracle/Makefile; skipped where it is
absent) and (b) closed forms / invariants / the reference's own known-answer
tests (tests/test_gguf.c:48,52,56,70,79,85 in the reference), chosen so that
a plausible slip (wrong nibble order, dropped offset, transposed operand, wrong
tail) fails at least one of them.
"""
import ctypes as C

import numpy as np
import pytest

import _native as N
from _native import close

O = N.oracle()
need_ref = pytest.mark.skipif(not N.ref_available("scalar"), reason="reference build absent")
need_avx2 = pytest.mark.skipif(not N.ref_available("avx2"), reason="reference AVX2 build absent")


# ------------------------------------------------------------------ fp16
def test_fp16_to_fp32_exhaustive_vs_numpy():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = np.array([O.or_fp16_to_fp32(int(v)) for v in h], dtype=np.float32)
    want = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))
    assert np.all(np.isinf(got[np.isinf(want)]))


@need_ref
def test_fp16_to_fp32_exhaustive_vs_reference():
    R = N.ref()
    for v in range(0, 65536, 7):
        a, b = O.or_fp16_to_fp32(v), R.vx_fp16_to_fp32(v)
        assert (a == b) or (np.isnan(a) and np.isnan(b)), v


@need_ref
def test_fp32_to_fp16_vs_reference():
    R = N.ref()
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.normal(0, 1, 3000), rng.normal(0, 1e-4, 1000), rng.normal(0, 1e4, 500),
                           [0.0, -0.0, 65504.0, 65520.0, 1e9, -1e9, 6e-5, 6e-8, 1e-10, np.inf, -np.inf]])
    for v in vals.astype(np.float32):
        assert O.or_fp32_to_fp16(float(v)) == R.vx_fp32_to_fp16(float(v)), v


def test_fp32_to_fp16_truncates():
    # 1 + 2^-11 + 2^-12 truncates to 1.0 (round-to-nearest would give 1+2^-10)
    assert O.or_fp32_to_fp16(1.0 + 2 ** -11 + 2 ** -12) == 0x3C00
    assert O.or_fp32_to_fp16(1e-6) == 0  # below the half normal range: flushed


# ------------------------------------------------------------------ blocks
def test_q4_0_block_size_and_roundtrip_kat():
    # reference tests/test_gguf.c:65-79: x = i - 16, block of 18 bytes, max err < 6
    assert N.Q4_BLOCK.itemsize == 18
    x = (np.arange(32) - 16).astype(np.float32)
    blk = np.zeros(1, dtype=N.Q4_BLOCK)
    O.or_quantize_row_q4_0(x, N._ptr(blk), 32)
    y = np.zeros(32, dtype=np.float32)
    O.or_dequantize_row_q4_0(N._ptr(blk), y, 32, 1.0)
    assert np.max(np.abs(x - y)) < 6.0
    # closed form: d = 16/7 in float32; stored d is that value truncated to half;
    # element t -> trunc(x_t * (1/d)) with the unrounded d, clamped, + 8
    d = np.float32(16.0) / np.float32(7.0)
    dbits = d.view(np.uint32)
    assert int(blk["d"][0]) == ((int(dbits >> 23) - 112) << 10) | int((dbits & 0x7FFFFF) >> 13)
    inv = np.float32(1.0) / d
    want = np.clip(np.trunc((x * inv).astype(np.float32)), -8, 7).astype(np.int64) + 8
    got = np.empty(32, np.int64)
    got[0::2] = blk["qs"][0] & 15
    got[1::2] = blk["qs"][0] >> 4
    assert np.array_equal(got, want)


@need_ref
def test_quantize_dequantize_vs_reference():
    R = N.ref()
    rng = np.random.default_rng(2)
    for n in (32, 64, 4096):
        x = rng.normal(0, 0.02, n).astype(np.float32)
        a = np.zeros(n // 32, dtype=N.Q4_BLOCK)
        b = np.zeros(n // 32, dtype=N.Q4_BLOCK)
        O.or_quantize_row_q4_0(x, N._ptr(a), n)
        R.vx_quantize_row_q4_0(x, N._ptr(b), n)
        assert a.tobytes() == b.tobytes()
        y1 = np.zeros(n, dtype=np.float32)
        y2 = np.zeros(n, dtype=np.float32)
        for scale in (1.0, 0.37):
            R.vx_set_synthetic_weight_scale(scale)
            O.or_dequantize_row_q4_0(N._ptr(a), y1, n, scale)
            R.vx_dequantize_row_q4_0(N._ptr(a), y2, n)
            assert np.array_equal(y1, y2)
            q8 = N.rand_q8_0(rng, 1, n)
            O.or_dequantize_row_q8_0(N._ptr(q8), y1, n, scale)
            R.vx_dequantize_row_q8_0(N._ptr(q8), y2, n)
            assert np.array_equal(y1, y2)
        R.vx_set_synthetic_weight_scale(1.0)


def test_q4_0_adjacent_pair_nibble_order():
    # element 2j is the LOW nibble of qs[j], element 2j+1 the HIGH nibble
    blk = np.zeros(1, dtype=N.Q4_BLOCK)
    blk["d"] = np.float16(1.0).view(np.uint16)
    blk["qs"][0][:] = 0x88
    blk["qs"][0][3] = 0xB9  # elements 6 -> 9-8 = 1, 7 -> 11-8 = 3
    y = np.zeros(32, dtype=np.float32)
    O.or_dequantize_row_q4_0(N._ptr(blk), y, 32, 1.0)
    want = np.zeros(32)
    want[6], want[7] = 1, 3
    assert np.array_equal(y, want)


# ------------------------------------------------------------------ GEMV exact
@pytest.mark.parametrize("rows,cols", [(1, 32), (7, 64), (33, 256), (64, 4096)])
def test_gemv_q4_0_exact_closed_form(rows, cols):
    rng = np.random.default_rng(rows * 1000 + cols)
    W = N.rand_q4_0(rng, rows, cols)
    x = rng.normal(0, 1, cols).astype(np.float32)
    y = np.zeros(rows, dtype=np.float32)
    O.or_gemv_q4_0(N._ptr(W), x, y, rows, cols)
    ref = N.q4_values(W) @ x.astype(np.float64)
    assert close(y, ref, atol=1e-5, rtol=1e-5)


def test_gemv_q4_0_invariants():
    rng = np.random.default_rng(3)
    rows, cols = 16, 128
    W = N.rand_q4_0(rng, rows, cols)
    y = np.zeros(rows, dtype=np.float32)
    # one-hot x picks column t: d_b * (s_t - 8)
    vals = N.q4_values(W)
    for t in (0, 1, 2, 31, 32, 127):
        x = np.zeros(cols, dtype=np.float32)
        x[t] = 1.0
        O.or_gemv_q4_0(N._ptr(W), x, y, rows, cols)
        assert np.array_equal(y.astype(np.float64), vals[:, t])
    # all nibbles 8 -> zero output
    W8 = W.copy()
    W8["qs"][:] = 0x88
    x = rng.normal(0, 1, cols).astype(np.float32)
    O.or_gemv_q4_0(N._ptr(W8), x, y, rows, cols)
    assert np.all(y == 0)


@need_ref
def test_gemv_q4_0_and_f32_vs_reference_bitexact():
    R = N.ref()
    rng = np.random.default_rng(4)
    rows, cols = 96, 512
    W = N.rand_q4_0(rng, rows, cols)
    x = rng.normal(0, 1, cols).astype(np.float32)
    a = np.zeros(rows, dtype=np.float32)
    b = np.zeros(rows, dtype=np.float32)
    O.or_gemv_q4_0(N._ptr(W), x, a, rows, cols)
    R.vx_gemv_q4_0(N._ptr(W), x, b, rows, cols)
    assert np.array_equal(a, b)
    gate = rng.normal(0, 0.02, rows).astype(np.float32)
    O.or_gemv_q4_0_sparse_rows(N._ptr(W), x, a, rows, cols, gate, 0.01)
    R.vx_gemv_q4_0_sparse_rows(N._ptr(W), x, b, rows, cols, gate, 0.01)
    assert np.array_equal(a, b)
    assert np.all(a[np.abs(gate) < 0.01] == 0) and np.any(a != 0)
    A = rng.normal(0, 1, (rows, cols + 3)).astype(np.float32)
    x3 = rng.normal(0, 1, cols + 3).astype(np.float32)
    O.or_gemv_f32(a, A, x3, rows, cols + 3)
    R.vx_gemv_f32(b, A, x3, rows, cols + 3)
    assert np.array_equal(a, b)


# ------------------------------------------------------------------ GEMV AVX2 lanes
def _avx2_lane_closed_form(W, x_ext):
    """Closed form of the AVX2 lane pattern in float64: per block
    d * [sum_t w_t s_t x_t - 8 (sum_{0..31} x_t + sum_{4..35} x_t)],
    w_t = 2 when t % 8 >= 4."""
    rows, nb = W.shape
    d = W["d"].view(np.float16).astype(np.float64)
    qs = W["qs"]
    s = np.empty((rows, nb, 32), dtype=np.float64)
    s[..., 0::2] = qs & 15
    s[..., 1::2] = qs >> 4
    w = np.where(np.arange(32) % 8 >= 4, 2.0, 1.0)
    out = np.zeros(rows)
    xe = x_ext.astype(np.float64)
    for b in range(nb):
        xb = xe[32 * b: 32 * b + 36]
        off = xb[:32].sum() + xb[4:36].sum()
        out += d[:, b] * ((s[:, b, :] * w * xb[:32]).sum(axis=1) - 8.0 * off)
    return out


@pytest.mark.parametrize("rows,cols", [(5, 32), (16, 256), (40, 4096)])
def test_gemv_avx2lanes_closed_form(rows, cols):
    rng = np.random.default_rng(rows + cols)
    W = N.rand_q4_0(rng, rows, cols)
    x = rng.normal(0, 1, cols + 4).astype(np.float32)
    y = np.zeros(rows, dtype=np.float32)
    O.or_gemv_q4_0_avx2lanes(N._ptr(W), x, y, rows, cols)
    assert close(y, _avx2_lane_closed_form(W, x), atol=1e-5, rtol=1e-5)
    # and it is NOT the exact Q4_0 product
    ex = N.q4_values(W) @ x[:cols].astype(np.float64)
    assert not close(y, ex)


def test_gemv_avx2lanes_one_hot_pattern():
    # one-hot x at position t (0..35) of a one-block row: reveals the double
    # weight of t%8>=4, the -8d offsets and the 4-float tail read.
    blk = np.zeros((1, 1), dtype=N.Q4_BLOCK)
    blk["d"] = np.float16(0.5).view(np.uint16)
    rng = np.random.default_rng(5)
    blk["qs"][0, 0] = rng.integers(0, 256, 16, dtype=np.uint8)
    s = np.empty(32)
    s[0::2] = blk["qs"][0, 0] & 15
    s[1::2] = blk["qs"][0, 0] >> 4
    y = np.zeros(1, dtype=np.float32)
    for t in range(36):
        x = np.zeros(36, dtype=np.float32)
        x[t] = 1.0
        O.or_gemv_q4_0_avx2lanes(N._ptr(blk), x, y, 1, 32)
        if t < 32:
            wt = 2.0 if t % 8 >= 4 else 1.0
            cnt = 1 + (1 if t >= 4 else 0)  # in sum_{0..31} and in sum_{4..35}
            want = 0.5 * (wt * s[t] - 8.0 * cnt)
        else:
            want = 0.5 * (-8.0)  # tail element only in sum_{4..35}
        assert y[0] == np.float32(want), t


@need_avx2
def test_gemv_avx2lanes_vs_reference_avx2_build():
    R = N.ref("avx2")
    rng = np.random.default_rng(6)
    for rows, cols in ((64, 256), (256, 4096)):
        W = N.rand_q4_0(rng, rows, cols)
        x = rng.normal(0, 1, cols + 4).astype(np.float32)
        a = np.zeros(rows, dtype=np.float32)
        b = np.zeros(rows, dtype=np.float32)
        O.or_gemv_q4_0_avx2lanes(N._ptr(W), x, a, rows, cols)
        R.vx_gemv_q4_0_avx2(N._ptr(W), x, b, rows, cols)
        assert close(a, b, atol=1e-5, rtol=1e-5), N.max_violation(a, b, 1e-5, 1e-5)
        gate = rng.normal(0, 0.02, rows).astype(np.float32)
        O.or_gemv_q4_0_avx2lanes_sparse_rows(N._ptr(W), x, a, rows, cols, gate, 0.01)
        R.vx_gemv_q4_0_avx2_sparse_rows(N._ptr(W), x, b, rows, cols, gate, 0.01)
        assert close(a, b, atol=1e-5, rtol=1e-5)
        A = rng.normal(0, 1, (rows, cols + 5)).astype(np.float32)
        x5 = rng.normal(0, 1, cols + 5).astype(np.float32)
        O.or_gemv_f32_avx2lanes(a, A, x5, rows, cols + 5)
        R.vx_gemv_f32_avx2(b, A, x5, rows, cols + 5)
        assert close(a, b, atol=1e-5, rtol=1e-5)


# ------------------------------------------------------------------ elementwise
def test_elementwise_kats():
    # reference tests/test_gguf.c:44-56
    o = np.zeros(4, dtype=np.float32)
    O.or_rms_norm(o, np.array([1, 2, 3, 4], np.float32), np.ones(4, np.float32), 4)
    assert abs(o[0] - 0.365) < 0.02
    assert abs(o[0] - 1.0 / np.sqrt(7.5 + 1e-5)) < 1e-6
    s = np.array([2.0, 1.0, 0.5], np.float32)
    O.or_softmax(s, 3)
    assert abs(s.sum() - 1.0) < 1e-5
    e = np.exp(np.array([2.0, 1.0, 0.5]) - 2.0)
    assert close(s, e / e.sum(), atol=1e-7, rtol=1e-6)
    v = np.array([-1.0, 0.0, 1.0], np.float32)
    O.or_silu(v, 3)
    assert abs(v[1]) < 1e-5 and abs(v[2] - 1 / (1 + np.exp(-1))) < 1e-6


@need_ref
def test_elementwise_vs_reference_bitexact():
    R = N.ref()
    rng = np.random.default_rng(7)
    x = rng.normal(0, 3, 2048).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 2048).astype(np.float32)
    a = np.zeros_like(x)
    b = np.zeros_like(x)
    O.or_rms_norm(a, x, w, 2048)
    R.vx_rms_norm(b, x, w, 2048)
    assert np.array_equal(a, b)
    a, b = x.copy(), x.copy()
    O.or_softmax(a, 2048)
    R.vx_softmax(b, 2048)
    assert np.array_equal(a, b)
    a, b = x.copy(), x.copy()
    O.or_silu(a, 2048)
    R.vx_silu(b, 2048)
    assert np.array_equal(a, b)


@need_ref
@pytest.mark.parametrize("pos", [0, 1, 17, 2047, 8191])
def test_rope_vs_reference_bitexact(pos):
    R = N.ref()
    rng = np.random.default_rng(pos)
    nh, nkv, hd = 8, 2, 64
    q = rng.normal(0, 1, nh * hd + 8).astype(np.float32)
    k = rng.normal(0, 1, nkv * hd + 8).astype(np.float32)
    q1, k1, q2, k2 = q.copy(), k.copy(), q.copy(), k.copy()
    O.or_rope(q1, k1, pos, nh, nkv, hd, 0, 10000.0)
    R.vx_rope(q2, k2, pos, nh, nkv, hd, 0, 10000.0)
    assert np.array_equal(q1, q2) and np.array_equal(k1, k2)


def test_rope_invariants():
    rng = np.random.default_rng(8)
    nh, hd = 4, 128
    q = rng.normal(0, 1, nh * hd).astype(np.float32)
    k = rng.normal(0, 1, nh * hd).astype(np.float32)
    q0, k0 = q.copy(), k.copy()
    O.or_rope(q0, k0, 0, nh, nh, hd, 0, 10000.0)
    assert np.array_equal(q0, q)  # pos 0 is the identity
    q1, k1 = q.copy(), k.copy()
    O.or_rope(q1, k1, 123, nh, nh, hd, 0, 10000.0)
    n0 = (q.reshape(-1, 2) ** 2).sum(1)
    n1 = (q1.reshape(-1, 2) ** 2).sum(1)
    assert close(n1, n0, atol=1e-5, rtol=1e-5)  # each pair keeps its norm
    # pair i is rotated by 123 * theta^(-2i/hd): compare with float64 rotation
    i = np.arange(hd // 2)
    ang = 123 * (10000.0 ** (-2.0 * i / hd))
    qq = q.reshape(nh, hd // 2, 2).astype(np.float64)
    want = np.stack([qq[..., 0] * np.cos(ang) - qq[..., 1] * np.sin(ang),
                     qq[..., 0] * np.sin(ang) + qq[..., 1] * np.cos(ang)], -1).reshape(-1)
    assert close(q1, want, atol=2e-4, rtol=1e-3)
    # relative-position property: <R(a)q, R(b)k> depends on a-b only
    qa, ka = q[:hd].copy(), k[:hd].copy()
    qb, kb = q[:hd].copy(), k[:hd].copy()
    O.or_rope(qa, ka, 10, 1, 1, hd, 0, 10000.0)
    O.or_rope(qb, kb, 30, 1, 1, hd, 0, 10000.0)
    qc, kc = q[:hd].copy(), k[:hd].copy()
    O.or_rope(qc, kc, 50, 1, 1, hd, 0, 10000.0)
    assert abs(float(qc @ kb) - float(qb @ ka)) < 1e-3


# ------------------------------------------------------------------ acceptance
def test_inverse_cdf_fixed_closed_form():
    w = np.array([0.1, 0.0, 0.2, 0.7], np.float32)
    # thresholds: cumulative 0.1, 0.1, 0.3, 1.0
    assert O.or_inverse_cdf_fixed(w, 4, 0.0) == 0
    assert O.or_inverse_cdf_fixed(w, 4, 0.05) == 0
    assert O.or_inverse_cdf_fixed(w, 4, 0.2) == 2
    assert O.or_inverse_cdf_fixed(w, 4, 0.5) == 3
    assert O.or_inverse_cdf_fixed(w, 4, 1.0 - 2 ** -24) == 3
    assert O.or_inverse_cdf_fixed(np.zeros(4, np.float32), 4, 0.5) == -1


def test_inverse_cdf_matches_brute_force_distribution():
    rng = np.random.default_rng(9)
    w = rng.uniform(0, 1, 24).astype(np.float32)
    counts = np.zeros(24)
    n = 1 << 14
    for k in range(n):
        u = np.float32(k / n)
        counts[O.or_inverse_cdf_fixed(w, 24, float(u))] += 1
    assert close(counts / n, w / w.sum(), atol=2.0 / n, rtol=0)


def test_accept_greedy_matches_target_greedy_decode():
    rng = np.random.default_rng(10)
    V, k = 50, 6
    L = rng.normal(0, 1, (k + 1, V)).astype(np.float32)
    am = L.argmax(1)
    out = np.zeros(k + 1, np.int32)
    # all drafts equal the target argmax -> k accepted + bonus argmax(L_k)
    n = O.or_accept_greedy(L.ravel(), V, am[:k].astype(np.int32).copy(), k, out)
    assert n == k + 1 and np.array_equal(out, am)
    d = am[:k].astype(np.int32).copy()
    d[3] = (d[3] + 1) % V
    n = O.or_accept_greedy(L.ravel(), V, d, k, out)
    assert n == 4 and np.array_equal(out[:4], am[:4])


def test_accept_sampled_properties():
    rng = np.random.default_rng(11)
    V, k, T = 40, 4, 0.8
    L = rng.normal(0, 2, (k + 1, V)).astype(np.float32)
    # draft distribution equal to the target's: every draft is accepted
    Q = np.zeros((k, V), np.float32)
    for j in range(k):
        O.or_softmax_temp(L[j].copy(), V, T, Q[j])
    drafts = rng.integers(0, V, k).astype(np.int32)
    u = np.full(k + 1, 1.0 - 2 ** -24, np.float32)
    out = np.zeros(k + 1, np.int32)
    na = C.c_int()
    n = O.or_accept_sampled(L.ravel(), V, Q.ravel(), V, drafts, k, T, u, out, C.byref(na))
    assert n == k + 1 and na.value == k and np.array_equal(out[:k], drafts)
    # q(d) > p(d) with u just above p/q -> reject; the resample comes from max(0, p-q)
    p0 = np.zeros(V, np.float32)
    O.or_softmax_temp(L[0].copy(), V, T, p0)
    Qr = np.roll(Q, 7, axis=1).copy()
    dj = int(np.argmax(Qr[0] - p0))
    drafts[0] = dj
    alpha = p0[dj] / Qr[0, dj]
    u[0] = np.float32(min(alpha + 1e-3, 0.999))
    n = O.or_accept_sampled(L.ravel(), V, Qr.ravel(), V, drafts, k, T, u, out, C.byref(na))
    assert n == 1 and na.value == 0
    res = np.maximum(0, p0 - Qr[0])
    assert res[out[0]] > 0


def test_accept_sampled_output_is_target_distributed():
    # statistical check of the speculative-sampling theorem on a tiny vocab:
    # accepted draft or residual resample at position 0 ~ p_0
    rng = np.random.default_rng(12)
    V, T = 6, 1.0
    L = rng.normal(0, 1, (2, V)).astype(np.float32)
    D = rng.normal(0, 1, V).astype(np.float32)
    p = np.zeros(V, np.float32)
    O.or_softmax_temp(L[0].copy(), V, T, p)
    q = np.zeros(V, np.float32)
    O.or_softmax_temp(D.copy(), V, T, q)
    counts = np.zeros(V)
    out = np.zeros(2, np.int32)
    na = C.c_int()
    n_trials = 40000
    for _ in range(n_trials):
        u = (rng.integers(0, 1 << 24, 3) / float(1 << 24)).astype(np.float32)
        d = int(O.or_inverse_cdf_fixed(q, V, float(u[2])))
        O.or_accept_sampled(L.ravel(), V, q, V, np.array([d], np.int32), 1, T, u[:2].copy(), out,
                            C.byref(na))
        counts[out[0]] += 1
    assert close(counts / n_trials, p, atol=0.012, rtol=0)


def test_sample_top_p_nucleus():
    l = np.log(np.array([0.05, 0.4, 0.3, 0.15, 0.1], np.float32))
    q = np.zeros(5, np.float32)
    seen = set()
    for k in range(64):
        u = k / 64.0
        t = O.or_sample_top_p(l, 5, 1.0, 0.7, u, q.ctypes.data_as(C.c_void_p))
        seen.add(t)
    # nucleus {1, 2} (0.4 + 0.3 >= 0.7): renormalised 4/7, 3/7
    assert seen == {1, 2}
    assert close(q, [0, 0.4 / 0.7, 0.3 / 0.7, 0, 0], atol=1e-6, rtol=1e-5)
    assert O.or_sample_top_p(l, 5, 0.0, 0.7, 0.3, None) == 1  # T<=0: argmax
