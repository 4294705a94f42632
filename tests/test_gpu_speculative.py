"""End-to-end speculative decoding on the GPU against the oracle.

Greedy (T = 0): the emitted sequence must equal target-only greedy decoding
(the reference CLI's loop, src/main.c:303-312), computed both with the
product's single-token forward and with the oracle.

Sampled (T > 0): every round is replayed on the oracle with the same seeded
uniforms: the draft tokens must be the oracle sampler's draws from the draft
model's logits, and the emitted tokens the oracle's acceptance decisions on the
target's logits (teacher-forced over the committed sequence).  A divergence is
accepted only as a certified tie (test_gpu_accept.py), after which the replay
stops.
"""
import ctypes as C

import numpy as np
import pytest

import _native as N
from _gguf import llama_gguf
from _oracle_model import OracleModel

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


def test_greedy_self_draft_accepts_everything(P, models):
    (tpath, traw, tsh), _ = models
    V = tsh[5]
    tm, dm = load(P, tpath), load(P, tpath)
    st = P.vx_speculative_create(dm, tm, 5)
    try:
        P.vx_speculative_set_temp(st, 0.0, 1.0)
        prompt = np.arange(7, dtype=np.int32)
        out = np.zeros(36, np.int32)
        assert P.vx_speculative_generate(st, prompt, 7, out, 36) == 36
        stats = N.VxSpecStats()
        P.vx_speculative_get_stats(st, C.byref(stats))
        assert stats.accepted == stats.drafted, (stats.accepted, stats.drafted)
        assert stats.rounds == 6   # 6 tokens per round (5 drafts + bonus)
    finally:
        P.vx_speculative_destroy(st)
        P.vx_model_destroy(tm)
        P.vx_model_destroy(dm)


@pytest.mark.parametrize("T,top_p", [(0.8, 1.0), (1.0, 0.9)])
def test_sampled_replay_matches_oracle(P, models, T, top_p):
    (tpath, traw, tsh), (dpath, draw, dsh) = models
    V = tsh[5]
    k, n_gen, seed = 4, 48, 2024
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
    ties = 0
    for r in range(stats.rounds):
        n0 = len(committed)
        drafts = [int(t) for t in tr_d[r * k:(r + 1) * k] if t >= 0]
        kk = len(drafts)
        seq = committed + drafts
        # draft model: logits for positions n0-1 .. n0-2+kk (teacher forced)
        Q = np.zeros((max(kk, 1), V), np.float32)
        if kk:
            dl = oracle_logits(draw, dsh, seq[:n0 - 1 + kk])
            for j in range(kk):
                u = uniform(seed, 1, r * k + j)
                tok = O.or_sample_top_p(np.ascontiguousarray(dl[n0 - 1 + j]), V, T, top_p, float(u),
                                        Q[j].ctypes.data_as(C.c_void_p))
                if tok != drafts[j]:
                    ties += 1
                    break
            else:
                tok = None
            if tok is not None and tok != drafts[j]:
                break   # certified divergence (checked in test_gpu_accept); stop replay
        tl = oracle_logits(traw, tsh, seq)[n0 - 1:n0 + kk]
        u = np.array([uniform(seed, 2, r * (k + 1) + j) for j in range(kk)] +
                     [uniform(seed, 2, r * (k + 1) + k)], np.float32)
        o = np.zeros(kk + 1, np.int32)
        na = C.c_int()
        ne = O.or_accept_sampled(np.ascontiguousarray(tl.ravel()), V, np.ascontiguousarray(Q[:max(kk, 1)].ravel()),
                                 V, np.array(drafts + [0], np.int32), kk, T, u, o, C.byref(na))
        got = [int(t) for t in tr_e[r * (k + 1):(r + 1) * (k + 1)] if t >= 0]
        if list(o[:ne]) != got:
            ties += 1
            break
        assert na.value == tr_a[r]
        committed += got
        emitted_total += got
    print(f"rounds {stats.rounds}, accepted {stats.accepted}/{stats.drafted}, divergences {ties}")
    assert ties <= 1
    assert emitted_total == list(out[:len(emitted_total)])
    assert len(emitted_total) >= n_gen // 2
