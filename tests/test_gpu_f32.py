"""F32 weight matrices (src/model.c:174-179, 206-211: apply_gemv and
apply_gemv_sparse_rows run an fp32 GEMV on them; :459-463: an F32 embedding
row is copied as it is) against the oracle, whose F32 forward is pinned to the
reference build in test_oracle_forward.py.

An F32 matrix lives on the device as plain fp32 rows and is multiplied by
vx_gemm_f32_kernel: the activation panel decoded to fp32 (hi + lo) in LDS,
products and sums in fp64.  Models with F32 layer or output matrices run the
plain-panel batched forward.  Checked at the fp32 bar (1e-4 + 1e-3 |ref|):
token-by-token logits, a 5-row verify batch, a 60-token prompt (batched
chunks), every cached K/V row, and the bit-exact read-back of an F32 matrix.
The FFN gate-skip is off on both sides (threshold 0): the GPU's F32 products
are exact, the oracle's fp32 sums are not, so a gate within rounding of a
nonzero threshold may fall either way (the skip itself is tested elsewhere).
"""
import ctypes as C

import numpy as np
import pytest

import _native as N
from _gguf import llama_gguf, GGML_F32, GGML_Q4_0, GGML_Q8_0
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


def load(P, path, n_ctx):
    mp = C.POINTER(N.VxModelDev)()
    assert P.vx_model_create(path.encode(), C.byref(mp)) == 0, N.product_error()
    mp.contents.config.n_ctx = n_ctx
    opt = N.VxModelOptions()
    P.vx_model_get_options(mp, C.byref(opt))
    opt.ffn_gate_threshold = 0.0
    assert P.vx_model_set_options(mp, C.byref(opt)) == 0
    return mp


CASES = [
    # layers, d, heads, kv, ff, vocab, embedding, output, layer matrices
    (2, 256, 4, 2, 512, 300, GGML_F32, GGML_F32, GGML_F32),
    (2, 192, 3, 1, 384, 256, GGML_Q4_0, GGML_F32, GGML_F32),
    (2, 256, 8, 2, 640, 200, GGML_F32, GGML_F32, GGML_Q4_0),
    (1, 128, 2, 2, 256, 128, GGML_Q8_0, GGML_Q8_0, GGML_F32),
]
NAMES = {GGML_F32: "F32", GGML_Q4_0: "Q4_0", GGML_Q8_0: "Q8_0"}


@pytest.mark.parametrize("case", CASES)
def test_f32_model_matches_oracle(P, tmp_path, case):
    L, d, h, kv, ff, V, et, ot, mt = case
    print(f"F32 model: {L}L d{d} {h}/{kv} heads ff{ff} V{V}; embedding {NAMES[et]}, output {NAMES[ot]}, "
          f"layers {NAMES[mt]}", flush=True)
    rng = np.random.default_rng(sum(case[:6]) + 7)
    path = str(tmp_path / "m.gguf")
    raw = llama_gguf(path, rng, L, d, h, kv, ff, V, std=0.05, norm_random=True, emb_type=et, out_type=ot,
                     matrix_type=mt)
    n_ctx = 256
    hd, kvd = d // h, kv * (d // h)
    prompt = rng.integers(0, V, 60).astype(np.int32)
    toks = rng.integers(0, V, 3).astype(np.int32)
    ver_toks = rng.integers(0, V, 5).astype(np.int32)
    mp = load(P, path, n_ctx)
    try:
        lp = np.zeros(V, np.float32)
        assert P.vx_model_forward(mp, prompt, len(prompt), lp) == 0, N.product_error()
        step = np.zeros((len(toks), V), np.float32)
        for i, t in enumerate(toks):
            assert P.vx_model_forward(mp, np.array([t], np.int32), 1, step[i]) == 0, N.product_error()
        ver = np.zeros((5, V), np.float32)
        assert P.vx_model_verify(mp, ver_toks, 5, ver) == 0, N.product_error()
        n_cached = mp.contents.cache_len
        kv_gpu = []
        for l in range(L):
            k = np.zeros((n_cached, kvd), np.float32)
            v = np.zeros((n_cached, kvd), np.float32)
            assert P.vx_model_read_kv(mp, l, n_cached, k, v) == 0, N.product_error()
            kv_gpu.append((k, v))
        if mt == GGML_F32:
            name = "blk.0.ffn_up.weight"
            back = np.zeros((ff, d), np.float32)
            assert P.vx_model_read_tensor(mp, name.encode(), back.ctypes.data_as(C.c_void_p), back.nbytes) == 0, \
                N.product_error()
            assert np.array_equal(back, raw[name])
    finally:
        P.vx_model_destroy(mp)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=n_ctx, gate_thr=0.0)
    ref_p = np.zeros(V, np.float32)
    assert O.or_forward(om.ptr, prompt, len(prompt), ref_p) == 0
    ref_s = np.zeros((len(toks), V), np.float32)
    for i, t in enumerate(toks):
        assert O.or_forward(om.ptr, np.array([t], np.int32), 1, ref_s[i]) == 0
    ref_v = np.zeros((5, V), np.float32)
    assert O.or_forward_all(om.ptr, ver_toks, 5, ref_v) == 0
    for what, got, ref in (("prompt", lp, ref_p), ("steps", step, ref_s), ("verify", ver, ref_v)):
        print(f"{what}: max |diff| {np.abs(got.astype(np.float64) - ref).max():.2e}")
        assert close(got, ref), (what, max_violation(got, ref))
    kc = om.k_cache.reshape(L, n_ctx, kvd)
    vc = om.v_cache.reshape(L, n_ctx, kvd)
    for l, (k, v) in enumerate(kv_gpu):
        assert close(k, kc[l, :n_cached]), ("K", l, max_violation(k, kc[l, :n_cached]))
        assert close(v, vc[l, :n_cached]), ("V", l, max_violation(v, vc[l, :n_cached]))


def test_f32_model_refuses_the_fp16_cache(P, tmp_path):
    rng = np.random.default_rng(5)
    path = str(tmp_path / "m.gguf")
    llama_gguf(path, rng, 1, 128, 2, 2, 256, 64, std=0.05, emb_type=GGML_F32, out_type=GGML_F32,
               matrix_type=GGML_F32)
    mp = load(P, path, 64)
    try:
        opt = N.VxModelOptions()
        P.vx_model_get_options(mp, C.byref(opt))
        opt.kv_half = 1
        assert P.vx_model_set_options(mp, C.byref(opt)) != 0
        assert "F32" in N.product_error()
    finally:
        P.vx_model_destroy(mp)
