"""GPU parity of the model forward / batched verify against the oracle.

Models are small random-init Llama GGUFs written by tests/_gguf.py.  The
oracle runs the reference data flow token by token (oracle/oracle.c
or_forward, pinned against the reference engine in test_oracle_forward.py);
the GPU runs the same tokens in batches.  Bar: logits within
1e-4 + 1e-3*|ref|; greedy argmax identical unless the top-2 gap is < 1e-4.
"""
import ctypes as C

import numpy as np
import pytest

import _native as N
from _gguf import llama_gguf, GGML_F32, GGML_Q8_0, GGML_Q4_0
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


class GpuModel:
    def __init__(self, P, path, n_ctx=None, q4_kernel=0, cap=4096):
        self.P = P
        self.mp = C.POINTER(N.VxModelDev)()
        rc = P.vx_model_create(path.encode(), C.byref(self.mp))
        assert rc == 0, (rc, N.product_error())
        if n_ctx is not None:
            self.mp.contents.config.n_ctx = n_ctx
        opt = N.VxModelOptions()
        P.vx_model_get_options(self.mp, C.byref(opt))
        opt.q4_kernel = q4_kernel
        opt.attn_cap = cap
        assert P.vx_model_set_options(self.mp, C.byref(opt)) == 0
        self.V = self.mp.contents.config.n_vocab

    def forward(self, toks):
        lg = np.zeros(self.V, np.float32)
        t = np.ascontiguousarray(toks, np.int32)
        assert self.P.vx_model_forward(self.mp, t, len(t), lg) == 0, N.product_error()
        return lg

    def verify(self, toks):
        t = np.ascontiguousarray(toks, np.int32)
        lg = np.zeros((len(t), self.V), np.float32)
        assert self.P.vx_model_verify(self.mp, t, len(t), lg) == 0, N.product_error()
        return lg

    @property
    def cache_len(self):
        return self.mp.contents.cache_len

    def close(self):
        self.P.vx_model_destroy(self.mp)


def make(tmp_path, seed, L=2, d=128, h=4, kv=2, ff=256, V=300, **kw):
    rng = np.random.default_rng(seed)
    path = str(tmp_path / f"m{seed}.gguf")
    raw = llama_gguf(path, rng, L, d, h, kv, ff, V, std=0.05, norm_random=True, **kw)
    return path, raw, (L, d, h, kv, ff, V)


@pytest.mark.parametrize("q4_kernel", [0, 1])
def test_forward_token_by_token(P, tmp_path, q4_kernel):
    print(f"forward token-by-token q4_kernel={q4_kernel}", flush=True)
    path, raw, (L, d, h, kv, ff, V) = make(tmp_path, 41)
    g = GpuModel(P, path, q4_kernel=q4_kernel)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=4096, q4_mode=q4_kernel)
    rng = np.random.default_rng(1)
    toks = rng.integers(0, V, 20).astype(np.int32)
    try:
        for i, t in enumerate(toks):
            a = g.forward([t])
            b = np.zeros(V, np.float32)
            O.or_forward(om.ptr, np.array([t], np.int32), 1, b)
            assert close(a, b), (i, max_violation(a, b))
        assert g.cache_len == om.cache_len == 20
    finally:
        g.close()


@pytest.mark.parametrize("q4_kernel", [0, 1])
def test_verify_batch_matches_sequential(P, tmp_path, q4_kernel):
    """Batched verify of k+1 rows after a prefix == teacher-forced sequential
    single-token forwards of the oracle (the reference verify semantics)."""
    print(f"verify batch q4_kernel={q4_kernel}", flush=True)
    path, raw, (L, d, h, kv, ff, V) = make(tmp_path, 42, L=3, d=256, h=8, kv=2, ff=512, V=500)
    g = GpuModel(P, path, q4_kernel=q4_kernel)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=4096, q4_mode=q4_kernel)
    rng = np.random.default_rng(2)
    prefix = rng.integers(0, V, 37).astype(np.int32)
    block = rng.integers(0, V, 9).astype(np.int32)
    try:
        g.forward(prefix)                      # batched prefill (16 + 16 + 5)
        got = g.verify(block)
        ref_all = np.zeros((37 + 9, V), np.float32)
        O.or_forward_all(om.ptr, np.concatenate([prefix, block]), 46, ref_all)
        ref = ref_all[37:]
        assert close(got, ref), max_violation(got, ref)
        for j in range(9):
            top = np.sort(ref[j])[-2:]
            if top[1] - top[0] > 1e-4:
                assert got[j].argmax() == ref[j].argmax()
        assert g.cache_len == 46
        # KV cache contents match the oracle's
        kvd = kv * (d // h)
        for l in range(L):
            k = np.zeros(46 * kvd, np.float32)
            v = np.zeros(46 * kvd, np.float32)
            assert P.vx_model_read_kv(g.mp, l, 46, k, v) == 0
            off = l * 4096 * kvd
            assert close(k, om.k_cache[off:off + 46 * kvd])
            assert close(v, om.v_cache[off:off + 46 * kvd])
    finally:
        g.close()


def test_q8_embedding_output_and_no_attn_output(P, tmp_path):
    path, raw, (L, d, h, kv, ff, V) = make(tmp_path, 43, L=2, d=96, h=3, kv=3, ff=192, V=200,
                                           emb_type=GGML_Q8_0, out_type=GGML_Q8_0,
                                           with_attn_output=False)
    g = GpuModel(P, path)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=4096)
    toks = np.random.default_rng(3).integers(0, V, 12).astype(np.int32)
    try:
        got = g.verify(toks)
        ref = np.zeros((12, V), np.float32)
        O.or_forward_all(om.ptr, toks, 12, ref)
        assert close(got, ref), max_violation(got, ref)
    finally:
        g.close()


def test_context_clamp(P, tmp_path):
    """Tokens past n_ctx overwrite the last slot (src/model.c:279-286)."""
    path, raw, (L, d, h, kv, ff, V) = make(tmp_path, 44, L=1, d=64, h=2, kv=1, ff=128, V=64)
    g = GpuModel(P, path, n_ctx=6)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=6)
    toks = np.random.default_rng(4).integers(0, V, 9).astype(np.int32)
    try:
        got = g.verify(toks)
        ref = np.zeros((9, V), np.float32)
        O.or_forward_all(om.ptr, toks, 9, ref)
        assert close(got, ref), max_violation(got, ref)
        assert g.cache_len == om.cache_len
    finally:
        g.close()


def test_attention_cap(P, tmp_path):
    """Attention reads only the first `cap` positions (src/model.c:304-305)."""
    path, raw, (L, d, h, kv, ff, V) = make(tmp_path, 45, L=1, d=64, h=4, kv=2, ff=128, V=80)
    g = GpuModel(P, path, cap=8)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=4096, attn_cap=8)
    toks = np.random.default_rng(5).integers(0, V, 21).astype(np.int32)
    try:
        got = g.verify(toks)
        ref = np.zeros((21, V), np.float32)
        O.or_forward_all(om.ptr, toks, 21, ref)
        assert close(got, ref), max_violation(got, ref)
    finally:
        g.close()


def test_read_tensor_roundtrip(P, tmp_path):
    path, raw, (L, d, h, kv, ff, V) = make(tmp_path, 46, L=1, d=64, h=2, kv=1, ff=96, V=70)
    g = GpuModel(P, path)
    try:
        for name in ("token_embd.weight", "output.weight", "blk.0.attn_q.weight", "blk.0.attn_k.weight",
                     "blk.0.attn_v.weight", "blk.0.attn_output.weight", "blk.0.ffn_gate.weight",
                     "blk.0.ffn_up.weight", "blk.0.ffn_down.weight"):
            want = raw[name]
            buf = np.zeros(want.nbytes, np.uint8)
            assert P.vx_model_read_tensor(g.mp, name.encode(), N._ptr(buf), buf.nbytes) == 0, name
            assert buf.tobytes() == want.tobytes(), name
    finally:
        g.close()


def test_kv_truncate_and_reverify(P, tmp_path):
    """Rolling cache_len back and re-running positions reproduces the logits."""
    path, raw, (L, d, h, kv, ff, V) = make(tmp_path, 47)
    g = GpuModel(P, path)
    toks = np.random.default_rng(6).integers(0, V, 14).astype(np.int32)
    try:
        g.forward(toks[:5])
        a = g.verify(toks[5:14])
        P.vx_model_kv_truncate(g.mp, 5)
        assert g.cache_len == 5
        b = g.verify(toks[5:14])
        assert np.array_equal(a, b)
        # src/model.c:384-389: a length past cache_len changes nothing, a
        # negative one empties the cache, a NULL model is ignored
        P.vx_model_kv_truncate(g.mp, 40)
        assert g.cache_len == 14
        C.CFUNCTYPE(None, C.c_void_p, C.c_int)(("vx_model_kv_truncate", P))(None, 3)
        P.vx_model_kv_truncate(g.mp, -2)
        assert g.cache_len == 0
        c = g.verify(toks[:14])
        assert np.array_equal(c[5:], a)
    finally:
        g.close()


@pytest.mark.parametrize("hd,mtype", [(64, GGML_Q4_0), (128, GGML_Q4_0), (128, GGML_Q8_0)])
def test_verify_every_batch_size(P, tmp_path, hd, mtype):
    """Verify batches of every size 1..16 after the same prefix (each size
    has its own kernel instantiations: the one- and two-row decode path with
    the attention combine in the output projection, the q|k|v attention at
    up to 16 rows, the 64-row-tile GEMMs from 5 rows; Q4_0 and Q8_0 layers)
    against the oracle's teacher-forced forward over prefix + block."""
    h = 4
    d = h * hd
    path, raw, (L, d, h, kv, ff, V) = make(tmp_path, 300 + hd + mtype, L=2, d=d, h=h, kv=2, ff=2 * d, V=500,
                                           matrix_type=mtype)
    g = GpuModel(P, path)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=4096)
    rng = np.random.default_rng(hd)
    prefix = rng.integers(0, V, 37).astype(np.int32)
    try:
        g.forward(prefix)
        for M in range(1, 17):
            print(f"verify batch of {M} rows, head_dim {hd}, matrix type {mtype}", flush=True)
            block = rng.integers(0, V, M).astype(np.int32)
            P.vx_model_kv_truncate(g.mp, 37)
            got = g.verify(block)
            ref_all = np.zeros((37 + M, V), np.float32)
            om.cache_len = 0               # the oracle's forward starts at its cache_len
            O.or_forward_all(om.ptr, np.concatenate([prefix, block]), 37 + M, ref_all)
            ref = ref_all[37:]
            assert close(got, ref), (M, max_violation(got, ref))
            for j in range(M):
                top = np.sort(ref[j])[-2:]
                if top[1] - top[0] > 1e-4:
                    assert got[j].argmax() == ref[j].argmax(), (M, j)
            assert g.cache_len == 37 + M
    finally:
        g.close()


@pytest.mark.parametrize("emb", [GGML_Q4_0, GGML_F32])
def test_token_ids_outside_the_vocabulary(P, tmp_path, emb):
    """Negative ids embed as a zero row (src/model.c:457).  Ids at or past
    n_vocab do too: the reference's F32 table checks the row against its
    size (src/model.c:461-463), its quantized lookup reads past the table,
    and the engine gives zeros for both.  A verify batch, one-row forwards
    and a prompt long enough for the batched prefill, against the oracle fed
    -1 in place of every id outside [0, n_vocab)."""
    path, raw, (L, d, h, kv, ff, V) = make(tmp_path, 91 + emb, emb_type=emb)
    rng = np.random.default_rng(emb)
    toks = rng.integers(0, V, 60).astype(np.int32)
    toks[[1, 9, 20, 33, 52]] = [-1, V, V + 1000, -7, 2**31 - 1]
    safe = np.where((toks < 0) | (toks >= V), -1, toks).astype(np.int32)
    ref = np.zeros((60, V), np.float32)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=4096)
    assert O.or_forward_all(om.ptr, safe, 60, ref) == 0
    g = GpuModel(P, path)
    try:
        got = g.verify(toks[:9])                  # rows 0..8 in one verify batch
        assert close(got, ref[:9]), max_violation(got, ref[:9])
        for i in range(9, 12):                     # one-row forwards
            one = g.forward(toks[i:i + 1])
            assert close(one, ref[i]), (i, max_violation(one, ref[i]))
    finally:
        g.close()
    g = GpuModel(P, path)
    try:
        last = g.forward(toks)                     # 60 tokens: the batched prefill
        assert close(last, ref[59]), max_violation(last, ref[59])
    finally:
        g.close()


def test_forward_and_verify_argument_checks(P, tmp_path):
    """The reference's argument checks (src/model.c:391-392): a NULL model,
    token array or logits buffer is VX_ERR_PARAM; zero or a negative count of
    tokens runs nothing (VX_OK; the logits and the cache stay as they were)."""
    path, raw, (L, d, h, kv, ff, V) = make(tmp_path, 61)
    g = GpuModel(P, path)
    proto = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p)
    try:
        g.forward(np.array([3, 4], np.int32))
        toks = np.array([5], np.int32)
        lg = np.full(V, 7.0, np.float32)
        mp = C.cast(g.mp, C.c_void_p)
        for name in ("vx_model_forward", "vx_model_verify"):
            f = proto((name, P))
            assert f(None, toks.ctypes.data, 1, lg.ctypes.data) == -4
            assert f(mp, None, 1, lg.ctypes.data) == -4
            assert f(mp, toks.ctypes.data, 1, None) == -4
            assert f(mp, toks.ctypes.data, 0, lg.ctypes.data) == 0
            assert f(mp, toks.ctypes.data, -3, lg.ctypes.data) == 0
            assert np.all(lg == 7.0) and g.cache_len == 2
    finally:
        g.close()


@pytest.mark.parametrize("mtype", [GGML_Q4_0, GGML_Q8_0])
def test_odd_shapes(P, tmp_path, mtype):
    """Widths with an odd number of 32-element blocks (n_embd 96: 3 blocks,
    n_ff 160: 5), three heads of 32, one kv head, and a vocabulary that is
    not a multiple of 32 rows (77): the padded block and row tiles must not
    leak into any sum.  One-row forwards, a verify batch and a prompt long
    enough for the batched prefill against the oracle."""
    path, raw, (L, d, h, kv, ff, V) = make(tmp_path, 131 + mtype, L=2, d=96, h=3, kv=1, ff=160, V=77,
                                           matrix_type=mtype)
    rng = np.random.default_rng(mtype + 3)
    toks = rng.integers(0, V, 64).astype(np.int32)
    ref = np.zeros((64, V), np.float32)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=4096)
    assert O.or_forward_all(om.ptr, toks, 64, ref) == 0
    g = GpuModel(P, path)
    try:
        for i in range(3):
            one = g.forward(toks[i:i + 1])
            assert close(one, ref[i]), (i, max_violation(one, ref[i]))
        got = g.verify(toks[3:12])
        assert close(got, ref[3:12]), max_violation(got, ref[3:12])
    finally:
        g.close()
    g = GpuModel(P, path)
    try:
        last = g.forward(toks)
        assert close(last, ref[63]), max_violation(last, ref[63])
    finally:
        g.close()


@pytest.mark.parametrize("d,h,kv", [(384, 6, 2), (640, 5, 1)])
def test_uneven_query_groups(P, tmp_path, d, h, kv):
    """Query heads per kv head that are not powers of two (3 at head_dim 64,
    5 at 128), so that the (head, row) query vectors of a kv head fill the
    attention's 16-vector groups unevenly, at one row and verify batches of
    9 and 15, against the oracle."""
    path, raw, (L, d, h, kv, ff, V) = make(tmp_path, 150 + h, L=2, d=d, h=h, kv=kv, ff=2 * d, V=300)
    rng = np.random.default_rng(h)
    toks = rng.integers(0, V, 40).astype(np.int32)
    ref = np.zeros((40, V), np.float32)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=4096)
    assert O.or_forward_all(om.ptr, toks, 40, ref) == 0
    g = GpuModel(P, path)
    try:
        got = g.verify(toks[:15])
        assert close(got, ref[:15]), max_violation(got, ref[:15])
        one = g.forward(toks[15:16])
        assert close(one, ref[15]), max_violation(one, ref[15])
        got = g.verify(toks[16:25])
        assert close(got, ref[16:25]), max_violation(got, ref[16:25])
        got = g.verify(toks[25:40])
        assert close(got, ref[25:40]), max_violation(got, ref[25:40])
    finally:
        g.close()


@pytest.mark.parametrize("emb", [GGML_Q4_0, GGML_Q8_0, GGML_F32])
def test_tied_output_matrix(P, tmp_path, emb):
    """A model without output.weight projects its logits with the token
    embedding (src/format.c:237-238), here Q4_0, Q8_0 or F32: one-row
    forwards and a verify batch against the oracle."""
    path, raw, (L, d, h, kv, ff, V) = make(tmp_path, 170 + emb, emb_type=emb, with_output=False)
    assert "output.weight" not in raw
    rng = np.random.default_rng(emb + 11)
    toks = rng.integers(0, V, 12).astype(np.int32)
    ref = np.zeros((12, V), np.float32)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=4096)
    assert O.or_forward_all(om.ptr, toks, 12, ref) == 0
    g = GpuModel(P, path)
    try:
        for i in range(3):
            one = g.forward(toks[i:i + 1])
            assert close(one, ref[i]), (i, max_violation(one, ref[i]))
        got = g.verify(toks[3:12])
        assert close(got, ref[3:12]), max_violation(got, ref[3:12])
    finally:
        g.close()


@pytest.mark.parametrize("mtype,q4_kernel", [(GGML_Q4_0, 0), (GGML_Q4_0, 1), (GGML_Q8_0, 0)])
def test_synthetic_weight_scale_in_the_forward(P, tmp_path, mtype, q4_kernel):
    """vx_set_synthetic_weight_scale multiplies every dequantized weight of
    the reference's forward (src/quantize.c:7-15 via vx_dequantize): the
    embedding rows and the exact-mode matrices; the x86 Q4_0 kernel reads
    its blocks directly and is not scaled (src/model.c:212-244).  Scale 0.5
    against the oracle with the same scale, one-row forwards and a verify
    batch."""
    path, raw, (L, d, h, kv, ff, V) = make(tmp_path, 190 + mtype + q4_kernel, matrix_type=mtype)
    rng = np.random.default_rng(mtype + q4_kernel)
    toks = rng.integers(0, V, 12).astype(np.int32)
    ref = np.zeros((12, V), np.float32)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=4096, q4_mode=q4_kernel, wscale=0.5)
    assert O.or_forward_all(om.ptr, toks, 12, ref) == 0
    unscaled = np.zeros((12, V), np.float32)
    om1 = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=4096, q4_mode=q4_kernel)
    assert O.or_forward_all(om1.ptr, toks, 12, unscaled) == 0
    assert not close(ref, unscaled)     # the scale changes the logits
    g = GpuModel(P, path, q4_kernel=q4_kernel)
    P.vx_set_synthetic_weight_scale(0.5)
    try:
        for i in range(3):
            one = g.forward(toks[i:i + 1])
            assert close(one, ref[i]), (i, max_violation(one, ref[i]))
        got = g.verify(toks[3:12])
        assert close(got, ref[3:12]), max_violation(got, ref[3:12])
    finally:
        P.vx_set_synthetic_weight_scale(1.0)
        g.close()


def test_prompt_longer_than_the_context(P, tmp_path):
    """A 110-token prompt into an 80-position cache: the batched prefill
    fills the 80 positions, the other 30 tokens run one at a time on the
    last slot (src/model.c:279-286); the last logits, cache_len and every
    cached row against the oracle, then a verify batch that keeps
    overwriting that slot."""
    path, raw, (L, d, h, kv, ff, V) = make(tmp_path, 201, L=2, d=128, h=4, kv=2, ff=256, V=200)
    kvd = kv * (d // h)
    g = GpuModel(P, path, n_ctx=80)
    om = OracleModel(raw, L, d, h, kv, ff, V, n_ctx=80)
    toks = np.random.default_rng(201).integers(0, V, 119).astype(np.int32)
    try:
        last = g.forward(toks[:110])
        ref = np.zeros((110, V), np.float32)
        assert O.or_forward_all(om.ptr, toks[:110], 110, ref) == 0
        assert close(last, ref[109]), max_violation(last, ref[109])
        assert g.cache_len == om.cache_len == 80
        kc = om.k_cache.reshape(L, 80, kvd)
        vc = om.v_cache.reshape(L, 80, kvd)
        for l in range(L):
            kk = np.zeros((80, kvd), np.float32)
            vv = np.zeros((80, kvd), np.float32)
            assert P.vx_model_read_kv(g.mp, l, 80, kk, vv) == 0, N.product_error()
            assert close(kk, kc[l]) and close(vv, vc[l]), l
        got = g.verify(toks[110:119])
        ref = np.zeros((9, V), np.float32)
        assert O.or_forward_all(om.ptr, toks[110:119], 9, ref) == 0
        assert close(got, ref), max_violation(got, ref)
    finally:
        g.close()
