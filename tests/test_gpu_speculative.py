"""End-to-end speculative decoding on the GPU against the oracle.

Greedy (T = 0): the emitted sequence must equal target-only greedy decoding
(the reference CLI's loop, src/main.c:303-312), computed both with the
product's single-token forward and with the oracle.

Sampled (T > 0): every round is replayed on the oracle with the same seeded
uniforms: the draft tokens must be the oracle sampler's draws from the draft
model's logits, and the emitted tokens the oracle's acceptance decisions on the
target's logits (teacher-forced over the committed sequence).  A divergence is
accepted only as a certified tie: a uniform within 1e-5 of the acceptance
ratio, or a draw whose CDF threshold sits within 1e-6 of the boundary between
two neighbouring tokens.  The replay then follows the GPU's choice; an
uncertified divergence fails.
"""
import ctypes as C

import numpy as np
import pytest

import _native as N
from _gguf import llama_gguf
from _oracle_model import OracleModel
from test_gpu_accept import near_boundary

pytestmark = pytest.mark.gpu
O = N.oracle()
M64 = (1 << 64) - 1


def splitmix64(x):
    x = (x + 0x9E3779B97F4A7C15) & M64
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & M64
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & M64
    return x ^ (x >> 31)


def uniform(seed, stream, index):
    r = splitmix64(seed ^ splitmix64(((stream << 48) & M64) ^ index))
    return np.float32((r >> 40) / float(1 << 24))


@pytest.fixture(scope="module")
def P():
    if not N.product_available():
        pytest.fail("product library not built")
    L = N.product()
    assert L.vxh_init() == 0, L.vxh_last_error()
    return L


@pytest.fixture(scope="module")
def models(tmp_path_factory):
    d = tmp_path_factory.mktemp("spec")
    V = 256
    rng = np.random.default_rng(77)
    tpath, dpath = str(d / "target.gguf"), str(d / "draft.gguf")
    traw = llama_gguf(tpath, rng, 2, 128, 4, 2, 256, V, std=0.08)
    draw = llama_gguf(dpath, rng, 1, 64, 2, 1, 128, V, std=0.08)
    return (tpath, traw, (2, 128, 4, 2, 256, V)), (dpath, draw, (1, 64, 2, 1, 128, V))


def load(P, path):
    mp = C.POINTER(N.VxModelDev)()
    assert P.vx_model_create(path.encode(), C.byref(mp)) == 0, N.product_error()
    return mp


def oracle_logits(raw, shape, seq):
    L, d, h, kv, ff, V = shape
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=256)
    out = np.zeros((len(seq), V), np.float32)
    O.or_forward_all(om.ptr, np.asarray(seq, np.int32), len(seq), out)
    return out


def test_greedy_equals_target_greedy_decode(P, models):
    (tpath, traw, tsh), (dpath, draw, dsh) = models
    V = tsh[5]
    prompt = np.random.default_rng(5).integers(0, V, 10).astype(np.int32)
    n_gen = 40
    tm, dm = load(P, tpath), load(P, dpath)
    st = P.vx_speculative_create(dm, tm, 4)
    assert st
    try:
        P.vx_speculative_set_temp(st, 0.0, 1.0)
        out = np.zeros(n_gen, np.int32)
        n = P.vx_speculative_generate(st, prompt.copy(), len(prompt), out, n_gen)
        assert n == n_gen, N.product_error()
        # target-only greedy decode with the product's forward
        tg = load(P, tpath)
        seq = list(prompt)
        lg = np.zeros(V, np.float32)
        assert P.vx_model_forward(tg, np.array(seq, np.int32), len(seq), lg) == 0
        ref = []
        for _ in range(n_gen):
            t = int(np.argmax(lg))
            ref.append(t)
            assert P.vx_model_forward(tg, np.array([t], np.int32), 1, lg) == 0
        P.vx_model_destroy(tg)
        # and with the oracle, teacher-forced over the reference sequence
        ol = oracle_logits(traw, tsh, list(prompt) + ref[:-1])
        oref = [int(np.argmax(ol[len(prompt) - 1 + i])) for i in range(n_gen)]
        gaps = [np.diff(np.sort(ol[len(prompt) - 1 + i])[-2:])[0] for i in range(n_gen)]
        for i in range(n_gen):
            if gaps[i] < 1e-4:
                break  # certified tie: sequences may diverge from here
            assert out[i] == ref[i] == oref[i], (i, out[:i + 1], ref[:i + 1], oref[:i + 1])
        stats = N.VxSpecStats()
        P.vx_speculative_get_stats(st, C.byref(stats))
        assert stats.emitted == n_gen and stats.rounds > 0
    finally:
        P.vx_speculative_destroy(st)
        P.vx_model_destroy(tm)
        P.vx_model_destroy(dm)


@pytest.mark.parametrize("k", [1, 2, 5, 8, 15])
def test_greedy_self_draft_accepts_everything(P, models, k):
    """The target as its own draft, greedy: every draft is accepted, each
    round emits k + 1 tokens (verify batches of 2..16 rows, and the one-row
    draft steps), and the tokens are the target's own greedy sequence."""
    (tpath, traw, tsh), _ = models
    V, n_gen = tsh[5], 36
    print(f"greedy self-draft k={k}", flush=True)
    prompt = np.arange(7, dtype=np.int32)
    tm, dm = load(P, tpath), load(P, tpath)
    st = P.vx_speculative_create(dm, tm, k)
    assert st, N.product_error()
    try:
        P.vx_speculative_set_temp(st, 0.0, 1.0)
        out = np.zeros(n_gen, np.int32)
        assert P.vx_speculative_generate(st, prompt.copy(), 7, out, n_gen) == n_gen, N.product_error()
        stats = N.VxSpecStats()
        P.vx_speculative_get_stats(st, C.byref(stats))
        assert stats.accepted == stats.drafted, (stats.accepted, stats.drafted)
        assert stats.rounds == (n_gen + k) // (k + 1)
        # target-only greedy decode on a fresh copy of the target
        tg = load(P, tpath)
        try:
            lg = np.zeros(V, np.float32)
            assert P.vx_model_forward(tg, prompt, 7, lg) == 0, N.product_error()
            for i in range(n_gen):
                t = int(np.argmax(lg))
                assert out[i] == t, (i, out[:i + 1])
                assert P.vx_model_forward(tg, np.array([t], np.int32), 1, lg) == 0, N.product_error()
        finally:
            P.vx_model_destroy(tg)
    finally:
        P.vx_speculative_destroy(st)
        P.vx_model_destroy(tm)
        P.vx_model_destroy(dm)


@pytest.mark.parametrize("T,top_p,k", [(0.8, 1.0, 4), (1.0, 0.9, 4), (0.8, 1.0, 1), (1.0, 0.9, 15),
                                       (0.8, 0.0, 4)])
def test_sampled_replay_matches_oracle(P, models, T, top_p, k):
    (tpath, traw, tsh), (dpath, draw, dsh) = models
    V = tsh[5]
    n_gen, seed = 48, 2024
    print(f"sampled replay T={T} top_p={top_p} k={k}", flush=True)
    prompt = np.random.default_rng(6).integers(0, V, 9).astype(np.int32)
    tm, dm = load(P, tpath), load(P, dpath)
    st = P.vx_speculative_create(dm, tm, k)
    max_rounds = n_gen + 1
    tr_d = np.full(max_rounds * k, -1, np.int32)
    tr_e = np.full(max_rounds * (k + 1), -1, np.int32)
    tr_a = np.full(max_rounds, -1, np.int32)
    try:
        P.vx_speculative_set_temp(st, T, top_p)
        P.vx_speculative_set_seed(st, seed)
        P.vx_speculative_set_trace(st, N._ptr(tr_d), N._ptr(tr_e), N._ptr(tr_a), max_rounds)
        out = np.zeros(n_gen, np.int32)
        n = P.vx_speculative_generate(st, prompt.copy(), len(prompt), out, n_gen)
        assert n == n_gen, N.product_error()
        stats = N.VxSpecStats()
        P.vx_speculative_get_stats(st, C.byref(stats))
        # decode is repeatable from the prefilled state
        out2 = np.zeros(n_gen, np.int32)
        assert P.vx_speculative_decode(st, out2, n_gen) == n_gen
        assert np.array_equal(out, out2)
    finally:
        P.vx_speculative_destroy(st)
        P.vx_model_destroy(tm)
        P.vx_model_destroy(dm)

    committed = list(prompt)
    emitted_total = []
    ties = []
    for r in range(stats.rounds):
        n0 = len(committed)
        drafts = [int(t) for t in tr_d[r * k:(r + 1) * k] if t >= 0]
        kk = len(drafts)
        seq = committed + drafts
        # draft model: logits for positions n0-1 .. n0-2+kk (teacher forced
        # over the GPU's drafts, so a certified divergence does not stop the replay)
        Q = np.zeros((max(kk, 1), V), np.float32)
        if kk:
            dl = oracle_logits(draw, dsh, seq[:n0 - 1 + kk])
            for j in range(kk):
                u = uniform(seed, 1, r * k + j)
                tok = O.or_sample_top_p(np.ascontiguousarray(dl[n0 - 1 + j]), V, T, top_p, float(u),
                                        Q[j].ctypes.data_as(C.c_void_p))
                if tok != drafts[j]:
                    assert certified_draw(Q[j], u, tok, drafts[j]), ("uncertified draft divergence", r, j,
                                                                     tok, drafts[j])
                    ties.append(("draft", r, j))
        tl = oracle_logits(traw, tsh, seq)[n0 - 1:n0 + kk]
        u = np.array([uniform(seed, 2, r * (k + 1) + j) for j in range(kk)] +
                     [uniform(seed, 2, r * (k + 1) + k)], np.float32)
        o = np.zeros(kk + 1, np.int32)
        na = C.c_int()
        ne = O.or_accept_sampled(np.ascontiguousarray(tl.ravel()), V, np.ascontiguousarray(Q[:max(kk, 1)].ravel()),
                                 V, np.array(drafts + [0], np.int32), kk, T, u, o, C.byref(na))
        got = [int(t) for t in tr_e[r * (k + 1):(r + 1) * (k + 1)] if t >= 0]
        if list(o[:ne]) != got or na.value != tr_a[r]:
            assert certified_accept(tl, Q, drafts, T, u, got, int(tr_a[r]), list(o[:ne]), na.value), \
                ("uncertified accept divergence", r, got, list(o[:ne]))
            ties.append(("accept", r))
        committed += got
        emitted_total += got
    print(f"rounds {stats.rounds}, accepted {stats.accepted}/{stats.drafted}, certified divergences {ties}")
    assert len(ties) <= 2
    assert len(emitted_total) >= n_gen
    assert emitted_total[:n_gen] == list(out)


def adjacent_in_support(w, a, b):
    """a and b both carry mass and no token between them does."""
    lo, hi = min(a, b), max(a, b)
    return w[a] > 0 and w[b] > 0 and not np.any(w[lo + 1:hi] > 0)


def certified_draw(w, u, tok_oracle, tok_gpu):
    """A draw that differs only across one CDF boundary: the threshold of u sits
    within 1e-6 of a prefix boundary (fp32 expf differences between the GPU and
    the host libm move it) and the two tokens are neighbours in the support."""
    w = np.asarray(w, np.float64)
    return near_boundary(w, u) and adjacent_in_support(w, tok_oracle, tok_gpu)


def certified_accept(tl, Q, drafts, T, u, got, na_g, want, na_o):
    """Certificate for the first decision where the GPU round and the oracle
    round differ: the ratio test (|u_j - alpha_j| < 1e-5), or the residual /
    bonus draw across one CDF boundary."""
    kk = len(drafts)
    j = min(na_g, na_o)
    V = tl.shape[1]
    p = np.zeros(V, np.float32)
    O.or_softmax_temp(np.ascontiguousarray(tl[j]), V, T, p)
    if j < kk and na_g != na_o:
        alpha = min(1.0, float(p[drafts[j]]) / max(float(Q[j][drafts[j]]), 1e-10))
        return abs(float(u[j]) - alpha) < 1e-5
    if j < kk:
        w = np.maximum(0.0, p.astype(np.float64) - Q[j])
    else:
        w = p.astype(np.float64)
    return len(got) == len(want) and got[:-1] == want[:-1] and certified_draw(w, float(u[kk]), want[-1], got[-1])


def test_decode_after_a_dropped_cache_fails_before_launching(P, tmp_path):
    """Changing kv_half drops a model's KV cache (and the prefilled rows with
    it): decode must refuse with an error instead of running on a missing or
    fresh cache."""
    path = str(tmp_path / "hd64.gguf")
    llama_gguf(path, np.random.default_rng(8), 1, 256, 4, 2, 256, 256, std=0.08)   # head_dim 64
    tm, dm = load(P, path), load(P, path)
    st = P.vx_speculative_create(dm, tm, 4)
    try:
        P.vx_speculative_set_temp(st, 0.0, 1.0)
        prompt = np.arange(6, dtype=np.int32)
        assert P.vx_speculative_prefill(st, prompt, 6) == 6
        opt = N.VxModelOptions()
        P.vx_model_get_options(tm, C.byref(opt))
        opt.kv_half = 1
        assert P.vx_model_set_options(tm, C.byref(opt)) == 0, N.product_error()
        assert not tm.contents.k_cache
        out = np.zeros(8, np.int32)
        assert P.vx_speculative_decode(st, out, 8) == 0
        assert "prefill again" in N.product_error()
        # prefill again: decoding works on the new (fp16) cache
        assert P.vx_speculative_prefill(st, prompt, 6) == 6
        assert P.vx_speculative_decode(st, out, 8) == 8, N.product_error()
    finally:
        P.vx_speculative_destroy(st)
        P.vx_model_destroy(tm)
        P.vx_model_destroy(dm)


def test_draft_context_smaller_than_target(P, models):
    """The loop is bounded by the target's context only (src/speculative.c:244,
    :257): once the draft's cache is full, rounds are target-only, and greedy
    output still equals target-only greedy decoding."""
    (tpath, traw, tsh), (dpath, draw, dsh) = models
    V = tsh[5]
    tm, dm = load(P, tpath), load(P, dpath)
    dm.contents.config.n_ctx = 14          # 10 prompt positions + 4
    st = P.vx_speculative_create(dm, tm, 4)
    n_gen = 20
    prompt = np.random.default_rng(15).integers(0, V, 10).astype(np.int32)
    try:
        P.vx_speculative_set_temp(st, 0.0, 1.0)
        out = np.zeros(n_gen, np.int32)
        assert P.vx_speculative_generate(st, prompt.copy(), len(prompt), out, n_gen) == n_gen, N.product_error()
        stats = N.VxSpecStats()
        P.vx_speculative_get_stats(st, C.byref(stats))
        assert stats.drafted < 4 * stats.rounds      # some rounds ran without drafts
        tg = load(P, tpath)
        lg = np.zeros(V, np.float32)
        assert P.vx_model_forward(tg, prompt, len(prompt), lg) == 0
        ref = []
        for _ in range(n_gen):
            t = int(np.argmax(lg))
            ref.append(t)
            assert P.vx_model_forward(tg, np.array([t], np.int32), 1, lg) == 0
        P.vx_model_destroy(tg)
        assert list(out) == ref
    finally:
        P.vx_speculative_destroy(st)
        P.vx_model_destroy(tm)
        P.vx_model_destroy(dm)


def test_generate_argument_checks_and_stream_entry(P, models):
    """vx_speculative_generate returns 0 tokens for a NULL state, prompt or
    output, an empty prompt or max_tokens < 1 (src/speculative.c:240-241);
    vx_speculative_generate_stream(token) is generate over the one-token
    prompt (src/speculative.c:296-300): same seed, same tokens."""
    (tpath, traw, tsh), (dpath, draw, dsh) = models
    proto = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int)
    gen = proto(("vx_speculative_generate", P))
    stream = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int)(("vx_speculative_generate_stream", P))
    outs = []
    for use_stream in (False, True):
        tm, dm = load(P, tpath), load(P, dpath)
        st = P.vx_speculative_create(dm, tm, 3)
        assert st, N.product_error()
        try:
            P.vx_speculative_set_temp(st, 0.8, 1.0)
            P.vx_speculative_set_seed(st, 99)
            prompt = np.array([17], np.int32)
            out = np.full(20, -5, np.int32)
            if not use_stream:
                assert gen(None, prompt.ctypes.data, 1, out.ctypes.data, 20) == 0
                assert gen(st, None, 1, out.ctypes.data, 20) == 0
                assert gen(st, prompt.ctypes.data, 1, None, 20) == 0
                assert gen(st, prompt.ctypes.data, 0, out.ctypes.data, 20) == 0
                assert gen(st, prompt.ctypes.data, 1, out.ctypes.data, 0) == 0
                assert np.all(out == -5)
                assert gen(st, prompt.ctypes.data, 1, out.ctypes.data, 20) == 20, N.product_error()
            else:
                assert stream(None, 17, out.ctypes.data, 20) == 0
                assert stream(st, 17, out.ctypes.data, 20) == 20, N.product_error()
            outs.append(out.copy())
        finally:
            P.vx_speculative_destroy(st)
            P.vx_model_destroy(tm)
            P.vx_model_destroy(dm)
    assert np.array_equal(outs[0], outs[1])
    assert np.all((outs[0] >= 0) & (outs[0] < tsh[5]))
    # draft counts 1..15 (a verify batch holds at most 16 rows); NULL models
    tm, dm = load(P, tpath), load(P, dpath)
    try:
        create = C.CFUNCTYPE(C.c_void_p, C.c_void_p, C.c_void_p, C.c_int)(("vx_speculative_create", P))
        for k in (0, -1, 16, 100):
            assert not P.vx_speculative_create(dm, tm, k), k
        assert not create(None, C.cast(tm, C.c_void_p), 4)
        assert not create(C.cast(dm, C.c_void_p), None, 4)
        for k in (1, 15):
            st = P.vx_speculative_create(dm, tm, k)
            assert st, (k, N.product_error())
            P.vx_speculative_destroy(st)
    finally:
        P.vx_model_destroy(tm)
        P.vx_model_destroy(dm)


@pytest.mark.parametrize("n_gen", [1, 2, 3])
def test_fewer_tokens_than_one_round(P, models, n_gen):
    """max_tokens below k + 1: the round drafts only what can still be
    emitted (src/speculative.c:258-263) and generate returns exactly
    max_tokens tokens, the target's own greedy ones."""
    (tpath, traw, tsh), _ = models
    V = tsh[5]
    prompt = np.arange(3, 12, dtype=np.int32)
    tm, dm = load(P, tpath), load(P, tpath)
    st = P.vx_speculative_create(dm, tm, 8)
    assert st, N.product_error()
    try:
        P.vx_speculative_set_temp(st, 0.0, 1.0)
        out = np.full(8, -5, np.int32)
        assert P.vx_speculative_generate(st, prompt.copy(), len(prompt), out, n_gen) == n_gen, N.product_error()
        assert np.all(out[n_gen:] == -5)
        stats = N.VxSpecStats()
        P.vx_speculative_get_stats(st, C.byref(stats))
        assert stats.rounds == 1 and stats.drafted == n_gen - 1 and stats.emitted == n_gen
    finally:
        P.vx_speculative_destroy(st)
        P.vx_model_destroy(tm)
        P.vx_model_destroy(dm)
    tg = load(P, tpath)
    try:
        lg = np.zeros(V, np.float32)
        assert P.vx_model_forward(tg, prompt, len(prompt), lg) == 0
        for i in range(n_gen):
            t = int(np.argmax(lg))
            assert out[i] == t, (i, out[:n_gen])
            assert P.vx_model_forward(tg, np.array([t], np.int32), 1, lg) == 0
    finally:
        P.vx_model_destroy(tg)
