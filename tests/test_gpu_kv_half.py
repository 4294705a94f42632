"""The flagged fp16 KV-cache mode (vx_model_options.kv_half) against the
oracle with the same rounding (or_model.kv_half: each stored K/V row rounded
to the nearest binary16, ties to even): a verify batch after a GPU prefill,
teacher-forced, at head_dim 64 (draft-shaped, the attention-in-attn_o path
for one row) and 128 (target-shaped), to the same tolerance as the fp32
cache.  The cache read back holds only binary16 values, and the mode is
refused where a forward would take a kernel without it."""
import ctypes as C

import numpy as np
import pytest

import _native as N
from _native import close, max_violation
from _oracle_model import OracleModel
from test_gpu_configs import prefill, read_weights, synth

pytestmark = pytest.mark.gpu
O = N.oracle()


@pytest.fixture(scope="module")
def P():
    if not N.product_available():
        pytest.fail("product library not built")
    L = N.bind_vxh(N.product())
    assert L.vxh_init() == 0, L.vxh_last_error()
    return L


def set_kv_half(P, mp, on, **over):
    opt = N.VxModelOptions()
    P.vx_model_get_options(mp, C.byref(opt))
    opt.kv_half = on
    for k, v in over.items():
        setattr(opt, k, v)
    return P.vx_model_set_options(mp, C.byref(opt))


@pytest.mark.parametrize("d,h,kv,L,n_ctx,n_past", [
    (256, 4, 2, 2, 256, 100), (512, 4, 2, 2, 256, 100),
    # a layer's cache beyond 16 MB is read with non-temporal loads (the
    # streamed instantiations of the fp16-cache kernels): head_dim 128, 64
    (2048, 16, 16, 1, 2304, 2100), (2048, 32, 32, 1, 2304, 2100)])
def test_kv_half_verify_matches_oracle(P, d, h, kv, L, n_ctx, n_past):
    F, V, k = 512, 512, 4
    hd = d // h
    kvd = kv * hd
    print(f"kv_half verify: d{d} {h}/{kv} heads (head_dim {hd}), {n_past} prefilled, k={k}", flush=True)
    mp = synth(P, L, d, h, kv, F, V, n_ctx, seed=77 + d, thr=0.0)
    try:
        assert set_kv_half(P, mp, 1) == 0, N.product_error()
        rng = np.random.default_rng(d)
        toks = rng.integers(0, V, n_past + k + 1).astype(np.int32)
        prefill(P, mp, toks[:n_past], V)
        # one-row forward (attention combined inside attn_o), then roll back
        one = prefill(P, mp, toks[n_past:n_past + 1], V)
        P.vx_model_kv_truncate(mp, n_past)
        got = np.zeros((k + 1, V), np.float32)
        assert P.vx_model_verify(mp, toks[n_past:], k + 1, got) == 0, N.product_error()
        P.vx_model_kv_truncate(mp, n_past)
        w = read_weights(P, mp, L, d, kvd, F, V, 2, 2)
        om = OracleModel(w, L, d, h, kv, F, V, n_ctx=n_ctx, attn_cap=4096, gate_thr=0.0, kv_half=1)
        kc = om.k_cache.reshape(L, n_ctx, kvd)
        vc = om.v_cache.reshape(L, n_ctx, kvd)
        for l in range(L):
            kk = np.zeros((n_past, kvd), np.float32)
            vv = np.zeros((n_past, kvd), np.float32)
            assert P.vx_model_read_kv(mp, l, n_past, kk, vv) == 0, N.product_error()
            # the cache holds binary16 values only
            assert np.array_equal(kk, kk.astype(np.float16).astype(np.float32))
            assert np.array_equal(vv, vv.astype(np.float16).astype(np.float32))
            assert np.abs(kk).max() > 0 and np.abs(vv).max() > 0
            kc[l, :n_past] = kk
            vc[l, :n_past] = vv
    finally:
        P.vx_model_destroy(mp)
    om.cache_len = n_past
    ref = np.zeros((k + 1, V), np.float32)
    assert O.or_forward_all(om.ptr, toks[n_past:], k + 1, ref) == 0
    diff = np.abs(got.astype(np.float64) - ref)
    print(f"max |diff| {diff.max():.3e}; one-row forward vs verify row 0 {np.abs(one - got[0]).max():.3e}")
    assert close(got, ref), max_violation(got, ref)
    assert close(one, ref[0]), max_violation(one, ref[0])


def test_kv_half_refused_where_unsupported(P):
    mp = synth(P, 1, 256, 4, 2, 512, 512, 64, seed=9)
    try:
        # forwards of more rows would take the separate row kernels (fp32 cache only)
        assert set_kv_half(P, mp, 1, pro_max_rows=1) != 0
        assert set_kv_half(P, mp, 1, fused=0) != 0
        assert set_kv_half(P, mp, 2) != 0
        assert set_kv_half(P, mp, 1) == 0, N.product_error()
        assert set_kv_half(P, mp, 0) == 0, N.product_error()
    finally:
        P.vx_model_destroy(mp)
    mp = synth(P, 1, 384, 4, 2, 512, 512, 64, seed=9)   # head_dim 96
    try:
        assert set_kv_half(P, mp, 1) != 0
    finally:
        P.vx_model_destroy(mp)


def test_kv_half_speculative_greedy_equals_target_greedy(P):
    """Greedy speculative decoding with both caches in fp16 emits the target's
    own greedy sequence (target-only forwards with the same fp16 cache), up
    to the first near-tie of the target's logits."""
    V, n_gen = 512, 32
    print("kv_half speculative greedy: 2L target / 1L draft, d256 4/2 heads", flush=True)
    tm = synth(P, 2, 256, 4, 2, 512, V, 256, seed=11, thr=0.0)
    dm = synth(P, 1, 256, 4, 2, 512, V, 256, seed=12, thr=0.0)
    tg = synth(P, 2, 256, 4, 2, 512, V, 256, seed=11, thr=0.0)
    st = None
    try:
        for m in (tm, dm, tg):
            assert set_kv_half(P, m, 1) == 0, N.product_error()
        st = P.vx_speculative_create(dm, tm, 4)
        assert st
        P.vx_speculative_set_temp(st, 0.0, 1.0)
        prompt = np.random.default_rng(3).integers(0, V, 12).astype(np.int32)
        out = np.zeros(n_gen, np.int32)
        assert P.vx_speculative_generate(st, prompt.copy(), len(prompt), out, n_gen) == n_gen, N.product_error()
        lg = np.zeros(V, np.float32)
        assert P.vx_model_forward(tg, prompt, len(prompt), lg) == 0, N.product_error()
        for i in range(n_gen):
            top2 = np.sort(lg)[-2:]
            if top2[1] - top2[0] < 1e-4:
                break   # certified tie: the sequences may part here
            t = int(np.argmax(lg))
            assert out[i] == t, (i, out[:i + 1])
            assert P.vx_model_forward(tg, np.array([t], np.int32), 1, lg) == 0, N.product_error()
    finally:
        if st:
            P.vx_speculative_destroy(st)
        for m in (tm, dm, tg):
            P.vx_model_destroy(m)


def _half_steps(mine, gpu):
    """Largest difference between two rows of binary16 values, in binary16
    steps of the larger magnitude (2^-10 of it), among the elements whose
    difference exceeds 2^-16 of the row's largest magnitude: fp32 sums over a
    few hundred terms that cancel can differ by a few 2^-24 of the sum of the
    terms' magnitudes, many binary16 steps of a small result."""
    slack = 2.0 ** -16 * float(np.abs(gpu).max())
    a = mine.astype(np.float64)
    b = gpu.astype(np.float64)
    diff = np.abs(a - b)
    step = 2.0 ** -10 * np.maximum(np.abs(a), np.abs(b))
    excess = np.where(diff > slack, diff / np.maximum(step, 1e-300), 0.0)
    return int(np.count_nonzero(diff)), float(excess.max())


@pytest.mark.parametrize("hd", [64, 128])
def test_kv_half_every_batch_size(P, tmp_path, hd):
    """The fp16 cache at every verify batch size 1..16 after the same prefix,
    against the oracle with the same rounding.  Two fp32 values a few ulps
    apart can round to neighbouring binary16 values, and the difference then
    reaches every later row and layer, so the oracle attends over the GPU's
    own stored rows (its cache-store hook) and the rows are checked one by
    one: row j's K/V as the oracle computes them over the GPU's rows before j
    must be within one binary16 step of what the GPU stored (or 2^-16 of the
    row's largest magnitude), and the logits
    to the usual bar.  A run without the hook checks layer 0 of the block,
    whose inputs are the embeddings alone, against rows the oracle stores
    itself."""
    from test_gpu_model import GpuModel, make
    h = 4
    path, raw, (L, d, h, kv, ff, V) = make(tmp_path, 500 + hd, L=2, d=h * hd, h=h, kv=2, ff=2 * h * hd, V=500)
    n_ctx, n_past, kvd = 4096, 37, kv * hd
    g = GpuModel(P, path)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=n_ctx, kv_half=1)
    kc = om.k_cache.reshape(L, n_ctx, kvd)
    vc = om.v_cache.reshape(L, n_ctx, kvd)
    own_k = np.zeros((L, kvd), np.float32)
    own_v = np.zeros((L, kvd), np.float32)
    om.m.kv_own_k = own_k.ctypes.data_as(C.c_void_p)
    om.m.kv_own_v = own_v.ctypes.data_as(C.c_void_p)
    rng = np.random.default_rng(hd + 1)
    prefix = rng.integers(0, V, n_past).astype(np.int32)
    n_diff = n_all = 0
    try:
        assert set_kv_half(P, g.mp, 1) == 0, N.product_error()
        g.forward(prefix)
        for M in range(1, 17):
            print(f"kv_half verify batch of {M} rows, head_dim {hd}", flush=True)
            block = rng.integers(0, V, M).astype(np.int32)
            P.vx_model_kv_truncate(g.mp, n_past)
            got = g.verify(block)
            n = n_past + M
            gk = np.zeros((L, n, kvd), np.float32)
            gv = np.zeros((L, n, kvd), np.float32)
            for l in range(L):
                assert P.vx_model_read_kv(g.mp, l, n, gk[l], gv[l]) == 0, N.product_error()
            assert np.array_equal(gk, gk.astype(np.float16).astype(np.float32))
            assert np.array_equal(gv, gv.astype(np.float16).astype(np.float32))
            # layer 0 of the block, stored by the oracle itself after the GPU's prefix
            kc[:, :n] = gk
            vc[:, :n] = gv
            om.m.kv_keep = 0
            om.cache_len = n_past
            scratch = np.zeros((M, V), np.float32)
            assert O.or_forward_all(om.ptr, block, M, scratch) == 0
            for mine, gpu in ((kc[0, n_past:n], gk[0, n_past:]), (vc[0, n_past:n], gv[0, n_past:])):
                for r in range(M):
                    nd, worst = _half_steps(mine[r], gpu[r])
                    assert worst <= 1.0, ("layer 0", M, r, nd, worst)
            # row by row over the GPU's rows
            kc[:, :n] = gk
            vc[:, :n] = gv
            om.m.kv_keep = 1
            ref = np.zeros((M, V), np.float32)
            row = np.zeros((1, V), np.float32)
            for j in range(M):
                om.cache_len = n_past + j
                assert O.or_forward_all(om.ptr, block[j:j + 1], 1, row) == 0
                ref[j] = row[0]
                p = n_past + j
                for mine, gpu in ((own_k, gk[:, p]), (own_v, gv[:, p])):
                    for l in range(L):
                        nd, worst = _half_steps(mine[l], gpu[l])
                        assert worst <= 1.0, (M, j, l, nd, worst)
                        n_diff += nd
                        n_all += kvd
            assert close(got, ref), (M, max_violation(got, ref))
    finally:
        g.close()
    print(f"own K/V elements differing by one binary16 step: {n_diff} of {n_all}")
