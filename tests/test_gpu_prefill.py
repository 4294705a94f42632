"""Large-M prompt prefill (vx_model_forward of a long prompt: chunks of up to
512 rows through vxh_gemm_rows, vxh_rope_kv_rows, vxh_attention and
vxh_swiglu_rows) against the oracle, which runs the prompt one token per
forward like the reference (src/speculative.c:100-107, src/model.c:391-628).

Checked at the fp32 bar (1e-4 + 1e-3 |ref|): the last token's logits, every
cached K/V row of every layer, and the logits of a verify step run on the
prefilled cache.  The same prompt through the batched decode forward
(prefill_min_rows = 0) agrees with the large-M path at the same bar.
"""
import ctypes as C

import numpy as np
import pytest

import _native as N
from _gguf import llama_gguf, GGML_Q4_0, GGML_Q8_0
from _native import close, max_violation
from _oracle_model import OracleModel

pytestmark = pytest.mark.gpu
O = N.oracle()


@pytest.fixture(scope="module")
def P():
    if not N.product_available():
        pytest.fail("product library not built")
    L = N.product()
    assert L.vxh_init() == 0, L.vxh_last_error()
    return L


def load(P, path, n_ctx, prefill_min_rows=None):
    """The FFN gate-skip is off (threshold 0) on both sides: with ~4e5 gate
    decisions per prompt one may sit within rounding of 0.01 and move a row
    by ~1e-3; the skip itself is tested at 0.01 where such a decision is
    certified (test_gpu_configs.py)."""
    mp = C.POINTER(N.VxModelDev)()
    assert P.vx_model_create(path.encode(), C.byref(mp)) == 0, N.product_error()
    mp.contents.config.n_ctx = n_ctx
    opt = N.VxModelOptions()
    P.vx_model_get_options(mp, C.byref(opt))
    opt.ffn_gate_threshold = 0.0
    if prefill_min_rows is not None:
        opt.prefill_min_rows = prefill_min_rows
    assert P.vx_model_set_options(mp, C.byref(opt)) == 0
    return mp


CASES = [
    # layers, d, heads, kv, ff, vocab, matrix type, prompt length
    (2, 256, 4, 2, 512, 512, GGML_Q4_0, 512),
    (2, 256, 8, 2, 640, 300, GGML_Q4_0, 600),
    (1, 192, 3, 3, 384, 256, GGML_Q8_0, 300),
    (1, 256, 2, 1, 256, 64, GGML_Q4_0, 300),      # head_dim 128: two chunks per attention wavefront
]


@pytest.mark.parametrize("case", CASES)
def test_prefill_matches_oracle(P, tmp_path, case):
    L, d, h, kv, ff, V, mt, n = case
    print(f"prefill {n} tokens: {L}L d{d} {h}/{kv} heads ff{ff} V{V} {'Q4_0' if mt == GGML_Q4_0 else 'Q8_0'}",
          flush=True)
    rng = np.random.default_rng(sum(case))
    path = str(tmp_path / "m.gguf")
    raw = llama_gguf(path, rng, L, d, h, kv, ff, V, std=0.05, norm_random=True, emb_type=mt, out_type=mt,
                     matrix_type=mt)
    n_ctx = 1024
    prompt = rng.integers(0, V, n).astype(np.int32)
    mp = load(P, path, n_ctx)
    mb = load(P, path, n_ctx, prefill_min_rows=0)
    try:
        got = np.zeros(V, np.float32)
        assert P.vx_model_forward(mp, prompt, n, got) == 0, N.product_error()
        assert mp.contents.cache_len == n
        base = np.zeros(V, np.float32)
        assert P.vx_model_forward(mb, prompt, n, base) == 0, N.product_error()
        hd, kvd = d // h, kv * (d // h)
        kv_gpu = []
        for l in range(L):
            k = np.zeros((n, kvd), np.float32)
            v = np.zeros((n, kvd), np.float32)
            assert P.vx_model_read_kv(mp, l, n, k, v) == 0, N.product_error()
            kv_gpu.append((k, v))
        toks = rng.integers(0, V, 5).astype(np.int32)
        ver = np.zeros((5, V), np.float32)
        assert P.vx_model_verify(mp, toks, 5, ver) == 0, N.product_error()
    finally:
        P.vx_model_destroy(mp)
        P.vx_model_destroy(mb)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=n_ctx, gate_thr=0.0)
    ref = np.zeros(V, np.float32)
    assert O.or_forward(om.ptr, prompt, n, ref) == 0
    print(f"last-token logits: max |diff| {np.abs(got.astype(np.float64) - ref).max():.2e} "
          f"(batched path {np.abs(base.astype(np.float64) - ref).max():.2e})")
    assert close(got, ref), max_violation(got, ref)
    assert close(got, base), max_violation(got, base)
    kc = om.k_cache.reshape(L, n_ctx, kvd)
    vc = om.v_cache.reshape(L, n_ctx, kvd)
    for l, (k, v) in enumerate(kv_gpu):
        assert close(k, kc[l, :n]), ("K", l, max_violation(k, kc[l, :n]))
        assert close(v, vc[l, :n]), ("V", l, max_violation(v, vc[l, :n]))
    vref = np.zeros((5, V), np.float32)
    assert O.or_forward_all(om.ptr, toks, 5, vref) == 0
    print(f"verify after prefill: max |diff| {np.abs(ver.astype(np.float64) - vref).max():.2e}")
    assert close(ver, vref), max_violation(ver, vref)
