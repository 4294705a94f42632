"""Page-locked staging and asynchronous uploads (vxh_host_alloc,
vxh_upload_async): the copies the speculative rounds enqueue without a host
wait land in stream order, before the stream's next kernel, and the staging
may be rewritten once the stream has been synchronised."""
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
