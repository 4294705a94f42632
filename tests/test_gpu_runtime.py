"""Runtime behaviour: page-locked staging and asynchronous uploads
(vxh_host_alloc, vxh_upload_async) -- the copies the speculative rounds
enqueue without a host wait land in stream order, before the stream's next
kernel, and the staging may be rewritten once the stream has been
synchronised -- and device memory returned by the destroy calls."""
import ctypes as C

import numpy as np
import pytest

import _native as N

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def P():
    if not N.product_available():
        pytest.fail("product library not built")
    L = N.bind_vxh(N.product())
    assert L.vxh_init() == 0, L.vxh_last_error()
    return L


def test_async_uploads_land_in_stream_order(P):
    n = 4096
    s = C.c_void_p()
    assert P.vxh_stream_create(C.byref(s)) == 0, P.vxh_last_error()
    h = C.c_void_p()
    assert P.vxh_host_alloc(C.byref(h), 2 * n * 4) == 0, P.vxh_last_error()
    stage = np.ctypeslib.as_array(C.cast(h, C.POINTER(C.c_float)), shape=(2 * n,))
    d = N.DevBuf(P, nbytes=n * 4)
    rng = np.random.default_rng(7)
    for rnd in range(3):
        a = rng.normal(size=n).astype(np.float32)
        b = rng.normal(size=n).astype(np.float32)
        stage[:n], stage[n:] = a, b
        # two copies from different staging halves, then a kernel that
        # overwrites the first quarter: the kernel runs after both copies
        assert P.vxh_upload_async(d.ptr, h, n * 4, s) == 0
        assert P.vxh_upload_async(d.ptr, C.c_void_p(h.value + n * 4), n * 2, s) == 0
        assert P.vxh_fill_f32(d.ptr, float(rnd) + 0.5, n // 4, s) == 0
        assert P.vxh_stream_sync(s) == 0
        got = d.get(np.float32, n)
        want = a.copy()
        want[: n // 2] = b[: n // 2]
        want[: n // 4] = rnd + 0.5
        assert np.array_equal(got, want), rnd
    d.free()
    assert P.vxh_host_free(h) == 0
    assert P.vxh_stream_destroy(s) == 0


def _free_device_bytes():
    hip = C.CDLL("libamdhip64.so")
    free, total = C.c_size_t(), C.c_size_t()
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def test_destroy_returns_device_memory(P, tmp_path):
    """Models (weights, KV cache, workspaces, prefill buffers) and
    speculative states (sampling workspaces, staging) created, run and
    destroyed ten times: the device's free memory ends where the first
    cycle left it."""
    from _gguf import llama_gguf
    rng = np.random.default_rng(3)
    V = 512
    tpath, dpath = str(tmp_path / "t.gguf"), str(tmp_path / "d.gguf")
    llama_gguf(tpath, rng, 2, 256, 4, 2, 512, V, std=0.05)
    llama_gguf(dpath, rng, 1, 128, 2, 1, 256, V, std=0.05)
    prompt = rng.integers(0, V, 70).astype(np.int32)   # long enough for the batched prefill

    def cycle():
        tm, dm = C.POINTER(N.VxModelDev)(), C.POINTER(N.VxModelDev)()
        assert P.vx_model_create(tpath.encode(), C.byref(tm)) == 0, N.product_error()
        assert P.vx_model_create(dpath.encode(), C.byref(dm)) == 0, N.product_error()
        st = P.vx_speculative_create(dm, tm, 4)
        assert st, N.product_error()
        out = np.zeros(24, np.int32)
        P.vx_speculative_set_temp(st, 0.8, 1.0)
        assert P.vx_speculative_generate(st, prompt.copy(), len(prompt), out, 24) == 24, N.product_error()
        P.vx_speculative_destroy(st)
        P.vx_model_destroy(tm)
        P.vx_model_destroy(dm)
        assert P.vxh_stream_sync(None) == 0

    cycle()
    base = _free_device_bytes()
    for _ in range(9):
        cycle()
    lost = base - _free_device_bytes()
    print(f"device bytes not returned after 9 more cycles: {lost}")
    assert lost < 4 << 20, lost
