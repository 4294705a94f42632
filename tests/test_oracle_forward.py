"""Pin the oracle's composed forward (oracle/oracle.c or_forward) against the
reference engine's own vx_model_forward (src/model.c:391-628), built from its
sources without AVX2 (oracle/_ref/libvxref_scalar.so), one OpenMP thread.

The reference calls attn_o in place (src/model.c:544); with one thread that is
a deterministic row-by-row recurrence, which the oracle reproduces under
attn_o_inplace=1.  With attn_o_inplace=0 (the engine's out-of-place semantics)
the oracle is compared against the reference on models without an
attn_output tensor, where the reference skips that product.
"""
import contextlib
import ctypes as C
import os

import numpy as np
import pytest

import _native as N
from _gguf import llama_gguf, GGML_F32, GGML_Q8_0, GGML_Q4_0
from _oracle_model import OracleModel

O = N.oracle()
_libc = C.CDLL("libc.so.6")
_M_PERTURB = -6      # glibc mallopt parameter


@contextlib.contextmanager
def zero_filled_malloc():
    """glibc's M_PERTURB with byte 0xff fills every fresh malloc chunk with
    0x00 (perturb ^ 0xff).  The reference's x86 Q4_0 GEMV reads four floats
    past x (src/simd/avx2.c:351-352); for the down projection those are the
    8-float pad between ffn_h and ffn_h2 of a malloc'd scratch
    (src/model.c:413-433) that nothing writes, so its value is heap garbage
    unless malloc hands out zeroed memory -- which is the oracle's reading."""
    _libc.mallopt(_M_PERTURB, 0xff)
    try:
        yield
    finally:
        _libc.mallopt(_M_PERTURB, 0)


pytestmark = pytest.mark.skipif(not N.ref_available("scalar"), reason="reference build absent")


def ref_forward_logits(path, tokens, n_vocab, n_ctx=None, chunks=None, kind="scalar"):
    R = N.ref(kind)
    R.vx_set_n_threads(1)
    mp = C.POINTER(N.VxModel)()
    err = R.vx_model_create(path.encode(), C.byref(mp))
    assert err == 0, err
    if n_ctx is not None:
        mp.contents.config.n_ctx = n_ctx
    outs = []
    try:
        chunks = chunks or [1] * len(tokens)
        i = 0
        for c in chunks:
            lg = np.zeros(n_vocab, np.float32)
            t = np.ascontiguousarray(tokens[i:i + c], dtype=np.int32)
            assert R.vx_model_forward(mp, t, c, lg) == 0
            outs.append(lg)
            i += c
        cfg = mp.contents.config
        conf = (cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.n_embd, cfg.n_head_dim, cfg.n_ff,
                cfg.n_vocab, cfg.n_ctx)
        return np.stack(outs), conf, mp.contents.cache_len
    finally:
        R.vx_model_destroy(mp)


CASES = [
    # layers, d, heads, kv, ff, vocab, attn_output, emb, out, layer matrices
    (2, 64, 4, 2, 128, 96, True, GGML_Q4_0, GGML_Q4_0, GGML_Q4_0),
    (2, 128, 4, 1, 256, 160, False, GGML_Q4_0, GGML_Q4_0, GGML_Q4_0),
    (1, 96, 3, 3, 192, 64, True, GGML_Q8_0, GGML_Q8_0, GGML_Q4_0),
    # F32 matrices (src/model.c:174-179, 206-211) and an F32 embedding (:459-463)
    (2, 64, 4, 2, 128, 96, True, GGML_F32, GGML_F32, GGML_F32),
    (1, 96, 3, 1, 192, 64, False, GGML_Q4_0, GGML_F32, GGML_F32),
]


@pytest.mark.parametrize("case", CASES)
def test_oracle_forward_matches_reference(tmp_path, case):
    L, d, h, kv, ff, V, with_o, et, ot, mt = case
    rng = np.random.default_rng(sum(case[:6]))
    path = str(tmp_path / "m.gguf")
    raw = llama_gguf(path, rng, L, d, h, kv, ff, V, std=0.05, with_attn_output=with_o,
                     norm_random=True, emb_type=et, out_type=ot, matrix_type=mt)
    tokens = rng.integers(0, V, 12).astype(np.int32)
    ref_logits, conf, ref_len = ref_forward_logits(path, tokens, V)
    assert conf[:7] == (L, h, kv, d, d // h, ff, V)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=4096, attn_o_inplace=1)
    got = np.zeros((len(tokens), V), np.float32)
    for i, t in enumerate(tokens):
        assert O.or_forward(om.ptr, np.array([t], np.int32), 1, got[i]) == 0
    assert om.cache_len == ref_len == len(tokens)
    assert N.close(got, ref_logits, atol=1e-5, rtol=1e-5), N.max_violation(got, ref_logits, 1e-5, 1e-5)
    if not with_o:
        # no attn_output: in-place vs out-of-place is moot, both must agree
        om2 = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=4096, attn_o_inplace=0)
        got2 = np.zeros((len(tokens), V), np.float32)
        O.or_forward_all(om2.ptr, tokens, len(tokens), got2)
        assert np.array_equal(got2, got)


def test_oracle_forward_multi_token_call_and_all(tmp_path):
    """vx_model_forward with n_tokens > 1 returns the LAST token's logits and
    advances cache_len by n; or_forward_all's rows equal one-token calls."""
    rng = np.random.default_rng(21)
    L, d, h, kv, ff, V = 2, 64, 4, 2, 128, 80
    path = str(tmp_path / "m.gguf")
    raw = llama_gguf(path, rng, L, d, h, kv, ff, V, std=0.05, with_attn_output=False)
    tokens = rng.integers(0, V, 10).astype(np.int32)
    ref_logits, _, ref_len = ref_forward_logits(path, tokens, V, chunks=[4, 6])
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=4096)
    allv = np.zeros((10, V), np.float32)
    O.or_forward_all(om.ptr, tokens, 10, allv)
    assert ref_len == 10
    assert N.close(allv[3], ref_logits[0], atol=1e-5, rtol=1e-5)
    assert N.close(allv[9], ref_logits[1], atol=1e-5, rtol=1e-5)


def test_oracle_forward_context_clamp_and_cap(tmp_path):
    """Positions beyond n_ctx overwrite slot n_ctx-1 (src/model.c:279-286)."""
    rng = np.random.default_rng(22)
    L, d, h, kv, ff, V = 1, 64, 2, 1, 128, 48
    path = str(tmp_path / "m.gguf")
    raw = llama_gguf(path, rng, L, d, h, kv, ff, V, std=0.05, with_attn_output=False)
    tokens = rng.integers(0, V, 9).astype(np.int32)
    ref_logits, _, ref_len = ref_forward_logits(path, tokens, V, n_ctx=6)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=6)
    got = np.zeros((9, V), np.float32)
    for i, t in enumerate(tokens):
        O.or_forward(om.ptr, np.array([t], np.int32), 1, got[i])
    assert om.cache_len == ref_len
    assert N.close(got, ref_logits, atol=1e-5, rtol=1e-5)


AVX2_CASES = [
    # layers, d, heads, kv, ff, vocab, attn_output, emb, out
    (2, 64, 4, 2, 128, 96, True, GGML_Q4_0, GGML_Q4_0),
    (2, 128, 4, 1, 256, 160, False, GGML_Q4_0, GGML_Q4_0),
    (1, 96, 3, 3, 192, 64, True, GGML_Q8_0, GGML_Q8_0),
]


@pytest.mark.skipif(not N.ref_available("avx2gemv"), reason="reference AVX2-GEMV build absent")
@pytest.mark.parametrize("case", AVX2_CASES)
def test_oracle_avx2_lane_forward_matches_reference_avx2_gemv_build(tmp_path, case):
    """The AVX2-lane composition (q4_mode 1: every GEMV in the lane pattern of
    src/simd/avx2.c:311-370, the 4-float x tails of src/model.c:425-435, the
    down projection's zero pad) against the reference's own forward with its
    x86 GEMV dispatch (src/model.c:174-244) and AVX2 attention dot products
    (:312-325) compiled in, and tensor.c's portable RoPE/softmax/RMSNorm/SiLU
    (libvxref_avx2gemv.so; the x86 RoPE reads uninitialised angles, so the
    full x86 build cannot pin this).  The reference's down-projection tail is
    unwritten heap memory; it runs under zero_filled_malloc so that tail is
    the zero pad the oracle reads.  One thread, so the reference's in-place
    attn_o is the oracle's row-by-row recurrence (attn_o_inplace = 1).  The
    lane pattern moves logits by O(1) against exact mode, so the 1e-5 bar
    below catches any wrong GEMV, tail or wiring; what remains is the
    attention's 8-wide dot-product order."""
    L, d, h, kv, ff, V, with_o, et, ot = case
    rng = np.random.default_rng(sum(case[:6]) + 11)
    path = str(tmp_path / "m.gguf")
    raw = llama_gguf(path, rng, L, d, h, kv, ff, V, std=0.05, with_attn_output=with_o,
                     norm_random=True, emb_type=et, out_type=ot)
    tokens = rng.integers(0, V, 12).astype(np.int32)
    with zero_filled_malloc():
        ref_logits, conf, ref_len = ref_forward_logits(path, tokens, V, kind="avx2gemv")
    assert conf[:7] == (L, h, kv, d, d // h, ff, V)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=4096, q4_mode=1, attn_o_inplace=1)
    got = np.zeros((len(tokens), V), np.float32)
    for i, t in enumerate(tokens):
        assert O.or_forward(om.ptr, np.array([t], np.int32), 1, got[i]) == 0
    assert om.cache_len == ref_len == len(tokens)
    assert N.close(got, ref_logits, atol=1e-5, rtol=1e-5), N.max_violation(got, ref_logits, 1e-5, 1e-5)
    # the lane pattern is visible: exact mode differs by far more than the bar
    ex = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=4096, q4_mode=0, attn_o_inplace=1)
    exact = np.zeros((len(tokens), V), np.float32)
    for i, t in enumerate(tokens):
        assert O.or_forward(ex.ptr, np.array([t], np.int32), 1, exact[i]) == 0
    assert np.abs(exact - ref_logits).max() > 1e-3



LAYER_MAJOR_CASES = [
    # layers, d, heads, kv, ff, vocab, matrix type, tokens, n_ctx, cap, attn_o_inplace, kv_half, biases
    (2, 64, 4, 2, 128, 96, GGML_Q4_0, 40, 4096, 4096, 0, 0, False),
    (2, 64, 4, 2, 128, 96, GGML_Q4_0, 40, 4096, 4096, 1, 0, True),
    (1, 64, 2, 1, 128, 48, GGML_Q4_0, 37, 20, 10, 0, 0, False),     # context clamp and cap
    (2, 96, 3, 3, 192, 64, GGML_Q8_0, 23, 4096, 0, 0, 1, True),     # fp16 KV rows
    (1, 64, 4, 4, 96, 40, GGML_F32, 17, 4096, 4096, 1, 0, False),
    (1, 32, 2, 1, 64, 24, GGML_Q4_0, 300, 512, 4096, 0, 0, False),  # two 256-token chunks
]


@pytest.mark.parametrize("case", LAYER_MAJOR_CASES)
def test_layer_major_forward_is_bit_identical(tmp_path, case):
    """or_forward / or_forward_all run a call's tokens layer by layer
    (matrices dequantised once per chunk, tokens in vector lanes); they must
    give the token-major restatement's results bit for bit: logits, every
    cache row, cache_len, the gate-hook records and inverted gate decisions,
    from an empty cache and from a partly filled one."""
    L, d, h, kv, ff, V, mt, n, n_ctx, cap, inplace, kvh, biases = case
    rng = np.random.default_rng(sum(case[:8]) + 5)
    path = str(tmp_path / "m.gguf")
    raw = llama_gguf(path, rng, L, d, h, kv, ff, V, std=0.05, norm_random=True, emb_type=mt, out_type=mt,
                     matrix_type=mt)
    if biases:
        kvd = kv * (d // h)
        for l in range(L):
            raw[f"blk.{l}.attn_q.bias"] = rng.normal(0, 0.1, d).astype(np.float32)
            raw[f"blk.{l}.attn_k.bias"] = rng.normal(0, 0.1, kvd).astype(np.float32)
            raw[f"blk.{l}.attn_v.bias"] = rng.normal(0, 0.1, kvd).astype(np.float32)
    tokens = rng.integers(0, V, n).astype(np.int32)

    def model():
        return OracleModel(raw, L, d, h, kv, ff, V, n_ctx=n_ctx, attn_cap=cap, attn_o_inplace=inplace,
                           kv_half=kvh, gate_thr=0.01)

    def run(fn_all, om, toks, all_rows):
        near = np.zeros((len(toks), L), np.float32)
        idx = np.zeros((len(toks), L), np.int32)
        om.m.gate_near, om.m.gate_near_idx = near.ctypes.data, idx.ctypes.data
        om.m.flip = 2
        om.m.flip_tok[0], om.m.flip_layer[0], om.m.flip_col[0] = 1, 0, 3
        om.m.flip_tok[1], om.m.flip_layer[1], om.m.flip_col[1] = len(toks) - 1, L - 1, 7
        out = np.zeros((len(toks), V) if all_rows else V, np.float32)
        assert fn_all(om, toks, out, all_rows) == 0
        om.m.gate_near, om.m.gate_near_idx, om.m.flip = None, None, 0
        return out, near, idx

    def batched(om, toks, out, a):
        return (O.or_forward_all if a else O.or_forward)(om.ptr, toks, len(toks), out)

    def tokenwise(om, toks, out, a):
        return O.or_forward_tokenwise(om.ptr, toks, len(toks), out, a)

    for all_rows in (True, False):
        for split in (0, n // 3):
            res = []
            for fn in (batched, tokenwise):
                om = model()
                if split:   # a partly filled cache, written by the other restatement
                    pre = np.zeros(V, np.float32)
                    other = tokenwise if fn is batched else batched
                    assert other(om, tokens[:split], pre, False) == 0
                r = run(fn, om, tokens[split:], all_rows)
                res.append(r + (om.k_cache.copy(), om.v_cache.copy(), om.cache_len))
            (a, an, ai, ak, av, al), (b, bn, bi, bk, bv, bl) = res
            assert al == bl
            assert np.array_equal(a, b), (all_rows, split, np.abs(a - b).max())
            assert np.array_equal(ak, bk) and np.array_equal(av, bv)
            assert np.array_equal(an, bn) and np.array_equal(ai, bi)


@pytest.mark.parametrize("kvh", [0, 1])
def test_cache_store_hook(tmp_path, kvh):
    """The cache-store hook (or_model.kv_keep): over cache rows the oracle
    stored itself, one token at a time with the hook gives the logits of the
    plain forward bit for bit, leaves the cache as it was, and hands back
    each layer's computed row (rounded as the cache stores it) equal to the
    stored one.  A changed caller row is what later tokens attend over."""
    L, d, h, kv, ff, V, n = 2, 64, 4, 2, 128, 96, 12
    kvd = kv * (d // h)
    rng = np.random.default_rng(31 + kvh)
    path = str(tmp_path / "m.gguf")
    raw = llama_gguf(path, rng, L, d, h, kv, ff, V, std=0.05, norm_random=True, matrix_type=GGML_Q4_0)
    tokens = rng.integers(0, V, n).astype(np.int32)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=64, kv_half=kvh)
    full = np.zeros((n, V), np.float32)
    assert O.or_forward_all(om.ptr, tokens, n, full) == 0
    kc, vc = om.k_cache.reshape(L, 64, kvd), om.v_cache.reshape(L, 64, kvd)
    k0, v0 = kc.copy(), vc.copy()
    own_k = np.zeros((L, kvd), np.float32)
    own_v = np.zeros((L, kvd), np.float32)
    om.m.kv_own_k = own_k.ctypes.data_as(C.c_void_p)
    om.m.kv_own_v = own_v.ctypes.data_as(C.c_void_p)
    om.m.kv_keep = 1
    row = np.zeros((1, V), np.float32)
    for j in range(n):
        om.cache_len = j
        assert O.or_forward_all(om.ptr, tokens[j:j + 1], 1, row) == 0
        assert np.array_equal(row[0], full[j]), j
        assert np.array_equal(own_k, k0[:, j]) and np.array_equal(own_v, v0[:, j]), j
    assert np.array_equal(kc, k0) and np.array_equal(vc, v0)
    # a caller row that differs from the computed one is the one attended over
    kc[0, 3] += 0.25
    om.cache_len = 0
    changed = np.zeros((n, V), np.float32)
    assert O.or_forward_all(om.ptr, tokens, n, changed) == 0
    assert np.array_equal(changed[:3], full[:3])
    assert not np.array_equal(changed[3], full[3])
    assert np.array_equal(kc[0, 3], k0[0, 3] + 0.25)
