"""GPU checks of the runtime half of the C ABI: device copies, the caching
pool (core/src/StoragePool.cpp:5-24's role, for device memory) and events."""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    from kansaiml_amd import _native as N
    from kansaiml_amd.device import DeviceTensor
    assert N.available(), "no gfx950 device"
    return N, DeviceTensor


@pytest.mark.parametrize("nbytes,offset", [(16, 0), (4096, 0), (1 << 20, 0), (1000, 0), (4096, 3), (33, 1)])
def test_memcpy_d2d(rt, nbytes, offset):
    N, D = rt
    gen = np.random.Generator(np.random.PCG64(nbytes + offset))
    host = gen.integers(0, 256, nbytes + offset, dtype=np.uint8).view(np.int8)
    src = D.from_host(host)
    dst = D([nbytes + offset], "int8")
    N.call("kh_memcpy_d2d", ctypes.c_void_p(dst.addr + offset), ctypes.c_void_p(src.addr + offset), nbytes)
    got = dst.numpy()
    np.testing.assert_array_equal(got[offset:], host[offset:])


def test_pool_reuses_blocks(rt):
    N, D = rt
    N.call("kh_pool_trim")
    before = N.pool_stats()["driver_allocs"]
    for _ in range(5):
        t = D([3, 1000], "float32")
        t.release()
    after = N.pool_stats()
    assert after["driver_allocs"] - before == 1
    assert after["cached"] >= 12000


def test_free_of_foreign_pointer_is_an_error(rt):
    N, D = rt
    t = D([64], "int8")
    with pytest.raises(RuntimeError):
        N.call("kh_free", ctypes.c_void_p(t.addr + 16))


def test_events_time_work(rt):
    N, D = rt
    e0, e1 = N.Event(), N.Event()
    a = D([1 << 24], "int8")
    b = D([1 << 24], "int8")
    e0.record()
    N.call("kh_memcpy_d2d", b.ptr, a.ptr, 1 << 24)
    e1.record()
    assert e0.elapsed_ms(e1) > 0.0


def test_invalid_arguments_raise(rt):
    N, D = rt
    with pytest.raises(RuntimeError):
        N.call("kh_quantize_rows", None, -1, 4, None, None)
    with pytest.raises(RuntimeError):
        N.call("kh_gemm_i8", None, None, 4, 4, 4, None, 0, None, 0, None, None, None)


def test_mfma_probe_reports_rate_and_clock():
    """kh_probe_mfma_i8: a positive int8 rate no higher than the published
    5.0 POP/s, a shader clock in (0, 2.5 GHz], and an error (not a fault) for
    an operand buffer smaller than compute units x 64 KiB."""
    import ctypes

    import numpy as np

    from kansaiml_amd import _native as N
    from kansaiml_amd.device import DeviceTensor as D
    cus = N.device_info()["cus"]
    nbytes = cus * 64 * 1024
    ops = D.from_host(np.random.Generator(np.random.PCG64(1)).integers(-127, 128, nbytes, dtype=np.int8))
    tops, mhz = ctypes.c_double(), ctypes.c_double()
    N.call("kh_probe_mfma_i8", ops.ptr, nbytes, 200, ctypes.byref(tops), ctypes.byref(mhz))
    assert 0.0 < tops.value <= 5100.0
    assert 0.0 < mhz.value <= 2500.0
    with pytest.raises(RuntimeError):
        N.call("kh_probe_mfma_i8", ops.ptr, nbytes - 16, 200, ctypes.byref(tops), ctypes.byref(mhz))


def test_stream_read_probe_runs_and_checks_arguments():
    from kansaiml_amd import _native as N
    from kansaiml_amd.device import DeviceTensor as D
    buf = D([5 * 65536 + 48], "int8")  # a partial last workgroup
    N.call("kh_probe_stream_read", buf.ptr, buf.nbytes)
    N.synchronize()
    with pytest.raises(RuntimeError):
        N.call("kh_probe_stream_read", buf.ptr, 7)
    with pytest.raises(RuntimeError):
        N.call("kh_probe_stream_read", None, 4096)


def test_from_flat_and_tolist(rt):
    """kansai.from_flat / Tensor.tolist (core/src/Tensor.cpp:94-100, 133-137;
    python/bindings.cpp:44, 133-134): values rounded to binary32 on the way
    in, widened exactly on the way out, shape kept, empty tensors allowed."""
    N, D = rt
    vals = [0.1, -2.5, 1e-40, 3.4e38, 1.0 / 3.0, -0.0, 7.0]
    t = D.from_flat(vals, [7])
    assert t.shape == [7] and t.dtype == "float32"
    got = t.tolist()
    assert got == [float(np.float32(v)) for v in vals]
    assert all(type(v) is float for v in got)
    m = D.from_flat(range(6), (2, 3))
    assert m.shape == [2, 3] and m.tolist() == [0.0, 1.0, 2.0, 3.0, 4.0, 5.0]
    assert D.from_flat([], [0, 4]).tolist() == []
