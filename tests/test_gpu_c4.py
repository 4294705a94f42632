"""Config 4 (the benchmark's workload) end to end: speculative decoding of a
32-layer d4096 32/32-head FFN 11008 V 32000 Q4_0 target with a 22-layer
d2048 32/4-head FFN 5632 draft, k = 8, against a 2048-token context
(vx_speculative_generate, src/speculative.c:238-294).

* Greedy at full size: the emitted tokens equal the product's own target-only
  greedy decode (the reference CLI's loop, src/main.c:303-312), up to the
  first near-tie (top-2 gap < 1e-4) of the target-only logits.
* Sampled at T = 0.8, top_p = 1.0 with seeded uniforms, on 2 of the 32 target
  layers and 2 of the 22 draft layers (every per-layer shape, the real
  2048-token caches): the oracle prefills both models itself, every row of
  the GPU's caches is compared with its rows, and every round is replayed
  there -- draft draws from the oracle draft's
  logits, accept/reject and resample decisions from the oracle target's
  logits on the same uniforms.  A divergence must carry a certificate
  (test_gpu_speculative.certified_draw / certified_accept).
"""
import ctypes as C

import numpy as np
import pytest

import _native as N
from test_gpu_configs import synth, read_weights, oracle_prefilled, set_threshold
from test_gpu_speculative import uniform, certified_draw, certified_accept

pytestmark = pytest.mark.gpu
O = N.oracle()

TARGET = dict(d=4096, h=32, kv=32, F=11008, V=32000)
DRAFT = dict(d=2048, h=32, kv=4, F=5632, V=32000)
K, PROMPT = 8, 2048


@pytest.fixture(scope="module")
def P():
    if not N.product_available():
        pytest.fail("product library not built")
    L = N.product()
    assert L.vxh_init() == 0, L.vxh_last_error()
    return L


def make(P, shape, n_layers, n_ctx, seed):
    s = shape
    return synth(P, n_layers, s["d"], s["h"], s["kv"], s["F"], s["V"], n_ctx, seed=seed)


def test_c4_greedy_full_size_equals_target_greedy(P):
    n_gen = 64
    print("C4 greedy: 32L d4096 target + 22L d2048 draft, k=8, prompt 2048, 64 tokens", flush=True)
    n_ctx = PROMPT + n_gen + K + 8
    tm = make(P, TARGET, 32, n_ctx, seed=4001)
    dm = make(P, DRAFT, 22, n_ctx, seed=4002)
    st = P.vx_speculative_create(dm, tm, K)
    try:
        prompt = np.random.default_rng(404).integers(0, TARGET["V"], PROMPT).astype(np.int32)
        P.vx_speculative_set_temp(st, 0.0, 1.0)
        out = np.zeros(n_gen, np.int32)
        assert P.vx_speculative_generate(st, prompt.copy(), PROMPT, out, n_gen) == n_gen, N.product_error()
        stats = N.VxSpecStats()
        P.vx_speculative_get_stats(st, C.byref(stats))
        # target-only greedy decode on the same target, from an empty cache
        P.vx_model_kv_truncate(tm, 0)
        V = TARGET["V"]
        lg = np.zeros(V, np.float32)
        assert P.vx_model_forward(tm, prompt, PROMPT, lg) == 0, N.product_error()
        ref, gaps = [], []
        for _ in range(n_gen):
            srt = np.sort(lg)
            gaps.append(float(srt[-1] - srt[-2]))
            t = int(np.argmax(lg))
            ref.append(t)
            assert P.vx_model_forward(tm, np.array([t], np.int32), 1, lg) == 0, N.product_error()
    finally:
        P.vx_speculative_destroy(st)
        P.vx_model_destroy(tm)
        P.vx_model_destroy(dm)
    tie = [i for i, g in enumerate(gaps) if g < 1e-4]
    n_cmp = tie[0] if tie else n_gen
    print(f"rounds {stats.rounds}, accepted {stats.accepted}/{stats.drafted}; tokens compared {n_cmp} "
          f"(first near-tie: {tie[:1]}); min top-2 gap {min(gaps):.2e}")
    assert n_cmp >= n_gen // 2
    assert list(out[:n_cmp]) == ref[:n_cmp]


def test_c4_sampled_replay_on_the_oracle(P):
    """2 + 2 layers of the config-4 shapes, T = 0.8, top_p = 1.0."""
    T, top_p, seed, max_tokens = 0.8, 1.0, 4343, 5
    Lt, Ld = 2, 2
    print("C4 sampled replay: 2 of 32 target layers, 2 of 22 draft layers, k=8, T=0.8, ctx 2048", flush=True)
    n_ctx = PROMPT + max_tokens + K + 8
    tm = make(P, TARGET, Lt, n_ctx, seed=4101)
    dm = make(P, DRAFT, Ld, n_ctx, seed=4102)
    st = P.vx_speculative_create(dm, tm, K)
    max_rounds = max_tokens + 1
    tr_d = np.full(max_rounds * K, -1, np.int32)
    tr_e = np.full(max_rounds * (K + 1), -1, np.int32)
    tr_a = np.full(max_rounds, -1, np.int32)
    V = TARGET["V"]
    try:
        prompt = np.random.default_rng(4141).integers(0, V, PROMPT).astype(np.int32)
        P.vx_speculative_set_temp(st, T, top_p)
        P.vx_speculative_set_seed(st, seed)
        P.vx_speculative_set_trace(st, N._ptr(tr_d), N._ptr(tr_e), N._ptr(tr_a), max_rounds)
        # the prompt prefill with the FFN gate-skip off on both sides (over
        # ~5e7 gate decisions some sit within rounding of 0.01), the decode
        # rounds at the reference's 0.01
        set_threshold(P, tm, 0.0)
        set_threshold(P, dm, 0.0)
        assert P.vx_speculative_prefill(st, prompt, PROMPT) == PROMPT, N.product_error()
        set_threshold(P, tm, 0.01)
        set_threshold(P, dm, 0.01)
        # both oracle models prefill prompt[0 .. PROMPT-1) themselves; the GPU
        # caches are compared with theirs row by row
        s, d = TARGET, DRAFT
        wt = read_weights(P, tm, Lt, s["d"], s["kv"] * (s["d"] // s["h"]), s["F"], V, 2, 2)
        ot = oracle_prefilled(P, tm, wt, Lt, s["d"], s["h"], s["kv"], s["F"], V, n_ctx, prompt[:PROMPT - 1], 4096,
                              "C4 target prefill")
        wd = read_weights(P, dm, Ld, d["d"], d["kv"] * (d["d"] // d["h"]), d["F"], V, 2, 2)
        od = oracle_prefilled(P, dm, wd, Ld, d["d"], d["h"], d["kv"], d["F"], V, n_ctx, prompt[:PROMPT - 1], 4096,
                              "C4 draft prefill")
        ot.m.gate_thr = od.m.gate_thr = 0.01
        out = np.zeros(max_tokens, np.int32)
        assert P.vx_speculative_decode(st, out, max_tokens) == max_tokens, N.product_error()
        stats = N.VxSpecStats()
        P.vx_speculative_get_stats(st, C.byref(stats))
    finally:
        P.vx_speculative_destroy(st)
        P.vx_model_destroy(tm)
        P.vx_model_destroy(dm)

    committed = list(prompt)
    emitted, ties = [], []
    draft_len = PROMPT - 1          # tokens whose rows the oracle draft cache holds
    for r in range(stats.rounds):
        n0 = len(committed)
        drafts = [int(t) for t in tr_d[r * K:(r + 1) * K] if t >= 0]
        kk = len(drafts)
        Q = np.zeros((max(kk, 1), V), np.float32)
        if kk:
            # catch-up rows committed[draft_len .. n0), then the drafts fed back
            feed = committed[draft_len:n0] + drafts[:kk - 1]
            od.cache_len = draft_len
            dl = np.zeros((len(feed), V), np.float32)
            assert O.or_forward_all(od.ptr, np.array(feed, np.int32), len(feed), dl) == 0
            dl = dl[n0 - 1 - draft_len:]
            for j in range(kk):
                u = uniform(seed, 1, r * K + j)
                tok = O.or_sample_top_p(np.ascontiguousarray(dl[j]), V, T, top_p, float(u),
                                        Q[j].ctypes.data_as(C.c_void_p))
                if tok != drafts[j]:
                    assert certified_draw(Q[j], u, tok, drafts[j]), ("uncertified draft divergence", r, j)
                    ties.append(("draft", r, j))
        ot.cache_len = n0 - 1
        tl = np.zeros((kk + 1, V), np.float32)
        assert O.or_forward_all(ot.ptr, np.array([committed[n0 - 1]] + drafts, np.int32), kk + 1, tl) == 0
        u = np.array([uniform(seed, 2, r * (K + 1) + j) for j in range(kk)] +
                     [uniform(seed, 2, r * (K + 1) + K)], np.float32)
        o = np.zeros(kk + 1, np.int32)
        na = C.c_int()
        ne = O.or_accept_sampled(np.ascontiguousarray(tl.ravel()), V, np.ascontiguousarray(Q.ravel()), V,
                                 np.array(drafts + [0], np.int32), kk, T, u, o, C.byref(na))
        got = [int(t) for t in tr_e[r * (K + 1):(r + 1) * (K + 1)] if t >= 0]
        if list(o[:ne]) != got or na.value != tr_a[r]:
            assert certified_accept(tl, Q, drafts, T, u, got, int(tr_a[r]), list(o[:ne]), na.value), \
                ("uncertified accept divergence", r, got, list(o[:ne]))
            ties.append(("accept", r))
        n_acc = int(tr_a[r])
        if kk:
            draft_len = n0 + min(n_acc, kk - 1)
        committed += got
        emitted += got
    print(f"rounds {stats.rounds}, accepted {stats.accepted}/{stats.drafted}, emitted {emitted[:max_tokens]}, "
          f"certified divergences {ties}")
    assert stats.rounds >= 2
    assert len(ties) <= 1
    assert emitted[:max_tokens] == list(out)
