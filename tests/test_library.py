"""CPU tests of the engine library (no GPU needed): it loads, exports exactly
the entry points its headers declare, its host-side format helpers are
bit-exact, its GGUF loader derives the reference's configuration, and the
compute entry points fail loudly when no GPU is present."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

import _native as N
from _gguf import llama_gguf, write_gguf, T_U32, T_F32, T_STR, GGML_Q4_0

O = N.oracle()
HAVE_GPU = os.path.exists("/dev/kfd")


@pytest.fixture(scope="module")
def P():
    if not N.product_available():
        pytest.fail("product library not built (run __graft_entry__.build())")
    return N.product()


def declared_functions():
    names = set()
    for h in ("veltrix.h", "model.h", "speculative.h", "quantize.h", "veltrix_gpu.h", "vxh.h"):
        text = open(os.path.join(N.REPO, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b((?:vx|vxh)_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_exports_match_headers(P):
    out = subprocess.run(["nm", "-D", "--defined-only", N.PRODUCT_SO], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if ln.split()[-1].startswith(("vx_", "vxh_"))}
    declared = declared_functions()
    assert declared, "no declarations parsed"
    assert declared - exported == set(), f"declared but not exported: {sorted(declared - exported)}"
    assert exported - declared == set(), f"exported but not declared: {sorted(exported - declared)}"


def test_host_fp16_helpers_bitexact(P):
    for h in range(0, 65536, 3):
        a, b = P.vx_fp16_to_fp32(h), O.or_fp16_to_fp32(h)
        assert (a == b) or (np.isnan(a) and np.isnan(b))
    rng = np.random.default_rng(1)
    for v in np.concatenate([rng.normal(0, 1, 2000), rng.normal(0, 1e-5, 200), [0.0, 7e4, -1e-9]]):
        assert P.vx_fp32_to_fp16(float(np.float32(v))) == O.or_fp32_to_fp16(float(np.float32(v)))


def test_host_quantize_row_bitexact(P):
    rng = np.random.default_rng(2)
    for n in (32, 64, 4096):
        x = rng.normal(0, 0.02, n).astype(np.float32)
        a = np.zeros(n // 32, N.Q4_BLOCK)
        b = np.zeros(n // 32, N.Q4_BLOCK)
        P.vx_quantize_row_q4_0(x, N._ptr(a), n)
        O.or_quantize_row_q4_0(x, N._ptr(b), n)
        assert a.tobytes() == b.tobytes()
    assert P.vx_quantized_size(4096, 2) == 128 * 18
    assert P.vx_quantized_size(4096, 8) == 128 * 34


def test_uniform_stream_is_splitmix64(P):
    from test_gpu_speculative import uniform
    for seed, stream, idx in ((0, 1, 0), (4242, 2, 17), (2 ** 63 + 5, 1, 12345)):
        assert np.float32(P.vx_uniform(seed, stream, idx)) == uniform(seed, stream, idx)
        u = P.vx_uniform(seed, stream, idx)
        assert 0.0 <= u < 1.0 and u * 2 ** 24 == int(u * 2 ** 24)


def read_config(P, path):
    P.vx_model_read_config.restype = C.c_int
    P.vx_model_read_config.argtypes = [C.c_char_p, C.POINTER(N.VxModelConfig)]
    cfg = N.VxModelConfig()
    rc = P.vx_model_read_config(path.encode(), C.byref(cfg))
    return rc, cfg


def ref_config(path):
    R = N.ref("scalar")
    mp = C.POINTER(N.VxModel)()
    rc = R.vx_model_create(path.encode(), C.byref(mp))
    if rc != 0:
        return rc, None
    c = mp.contents.config
    out = {f: getattr(c, f) for f, _ in N.VxModelConfig._fields_ if f != "n_threads"}
    R.vx_model_destroy(mp)
    return rc, out


@pytest.mark.skipif(not N.ref_available("scalar"), reason="reference build absent")
def test_gguf_config_matches_reference_loader(P, tmp_path):
    rng = np.random.default_rng(3)
    path = str(tmp_path / "a.gguf")
    llama_gguf(path, rng, 3, 128, 4, 2, 256, 300, rope_theta=500000.0)
    rc, cfg = read_config(P, path)
    assert rc == 0
    rrc, ref = ref_config(path)
    assert rrc == 0
    mine = {f: getattr(cfg, f) for f, _ in N.VxModelConfig._fields_ if f != "n_threads"}
    assert mine == ref
    assert (cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.n_embd, cfg.n_ff, cfg.n_vocab) == (3, 4, 2, 128, 256, 300)
    assert cfg.rope_theta == 500000.0 and cfg.n_ctx == 4096 and cfg.n_head_dim == 32


@pytest.mark.skipif(not N.ref_available("scalar"), reason="reference build absent")
def test_gguf_scan_quirks_match_reference(P, tmp_path):
    """Without a vocab_size key the reference's shared scan cursor moves past
    the KV section, so rope.freq_base and general.architecture are never read
    (src/gguf.c:293-356, 523-536); n_vocab then comes from token_embd and
    n_ff from ffn_gate (src/format.c:287-322)."""
    d, V, F = 64, 100, 128
    blk = lambda r, c: np.zeros((r, c // 32), N.Q4_BLOCK).tobytes()
    tensors = [("token_embd.weight", GGML_Q4_0, [d, V], blk(V, d)),
               ("blk.0.attn_q.weight", GGML_Q4_0, [d, d], blk(d, d)),
               ("blk.0.ffn_gate.weight", GGML_Q4_0, [d, F], blk(F, d))]
    kv = [("general.architecture", T_STR, "gemma"),
          ("llama.block_count", T_U32, 1),
          ("llama.attention.head_count", T_U32, 2),
          ("llama.embedding_length", T_U32, d),
          ("llama.rope.freq_base", T_F32, 1234.0)]
    path = str(tmp_path / "q.gguf")
    write_gguf(path, kv, tensors)
    rc, cfg = read_config(P, path)
    assert rc == 0
    assert cfg.rope_theta == 10000.0 and cfg.arch == 1      # fallback theta, default llama arch
    assert cfg.n_vocab == V and cfg.n_ff == F and cfg.n_kv_heads == 2
    rrc, ref = ref_config(path)
    assert rrc == 0
    mine = {f: getattr(cfg, f) for f, _ in N.VxModelConfig._fields_ if f != "n_threads"}
    assert mine == ref


def test_gguf_errors(P, tmp_path):
    p = str(tmp_path / "bad.gguf")
    open(p, "wb").write(b"NOTGGUF" + b"\0" * 64)
    assert read_config(P, p)[0] == -2          # VX_ERR_FORMAT
    assert read_config(P, str(tmp_path / "missing.gguf"))[0] == -1   # VX_ERR_FILE


@pytest.mark.skipif(HAVE_GPU, reason="checks the no-GPU behaviour")
def test_compute_entry_points_fail_loudly_without_gpu(P, tmp_path):
    rng = np.random.default_rng(4)
    W = N.rand_q4_0(rng, 8, 64)
    x = rng.normal(0, 1, 68).astype(np.float32)
    y = np.zeros(8, np.float32)
    P.vx_gemv_q4_0(N._ptr(W), x, y, 8, 64)
    assert np.all(np.isnan(y))
    assert b"device" in P.vx_last_error().lower() or b"hip" in P.vx_last_error().lower()
    path = str(tmp_path / "m.gguf")
    llama_gguf(path, rng, 1, 64, 2, 1, 128, 50)
    mp = C.POINTER(N.VxModelDev)()
    assert P.vx_model_create(path.encode(), C.byref(mp)) != 0


def test_integration_snippet_compiles_and_links(P, tmp_path):
    """The C caller in INTEGRATION.md, written against the reference API,
    compiles unchanged against include/ and links against the library."""
    doc = open(os.path.join(N.REPO, "INTEGRATION.md")).read()
    blocks = re.findall(r"```c\n(.*?)```", doc, flags=re.S)
    assert blocks, "no C block in INTEGRATION.md"
    src = tmp_path / "app.c"
    src.write_text(blocks[0])
    libdir = os.path.dirname(N.PRODUCT_SO)
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", os.path.join(N.REPO, "include"),
                        str(src), "-o", str(tmp_path / "app"), "-L", libdir, "-lveltrix_amd",
                        "-Wl,-rpath," + libdir], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_attention_refuses_caches_past_32_bit_offsets(P):
    """The attention kernels address a layer's cache rows with 32-bit byte
    offsets; a layer of 4 GiB or more is refused on the host, before any
    launch (and before the arguments are touched), at the size where fp32
    and fp16 caches reach 2^32 bytes."""
    P.vxh_attention.restype = C.c_int
    P.vxh_attention.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]
    # 2^18 rows x 4096 fp32 = 2^32 bytes: one byte past the last 32-bit offset
    rc = P.vxh_attention(None, 1, 0, 1 << 18, 32, 32, 128, 0, None, None, None, 4096, None, None)
    assert rc == -5, rc                   # VXH_ERR_UNSUPPORTED
    assert b"4 GiB" in P.vxh_last_error()
    P.vxh_attention_qkv_f16.restype = C.c_int
    P.vxh_attention_qkv_f16.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p,
                                        C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int,
                                        C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p,
                                        C.c_int, C.c_void_p, C.c_void_p]
    # fp16: 2^19 rows x 4096 halves = 2^32 bytes; the q|k|v sums must look valid to reach the check
    buf = (C.c_double * 16)()
    rc = P.vxh_attention_qkv_f16(C.addressof(buf), 4096 * 3, None, 0, None, None, None, None, None, 1 << 20, 1, 0,
                                 1 << 19, 32, 32, 128, 0, C.addressof(buf), C.addressof(buf), None, 4096, None, None)
    assert rc == -5, (rc, P.vxh_last_error())
    assert b"4 GiB" in P.vxh_last_error()


def test_parity_helper_row_budget():
    """The parity bar's fallback: an element beyond 1e-4 + 1e-3|oracle| passes
    only within the oracle's own worst fp32 error of its row."""
    rng = np.random.default_rng(3)
    exact = rng.normal(0, 100, (4, 50))
    exact[:, 0] = 1e-3                                  # near-zero results
    oracle = exact + rng.normal(0, 3e-4, exact.shape)   # fp32-sum-sized errors
    budget = np.abs(oracle - exact).max(axis=1)
    gpu = exact.copy()
    gpu[:, 0] = exact[:, 0] + 0.9 * budget              # off the bar, inside the budget
    assert N.parity(gpu, oracle, exact)[0]
    gpu[2, 0] = exact[2, 0] + 1.1 * budget[2]           # outside the row's budget
    assert not N.parity(gpu, oracle, exact)[0]
    gpu = oracle + 2e-4                                 # within the bar wherever |oracle| > 0.1
    gpu[:, 0] = oracle[:, 0] + 1.0                      # a dropped term
    assert not N.parity(gpu, oracle, exact)[0]
