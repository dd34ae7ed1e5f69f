"""The C ABI's argument checks (the reference backend contract: a bad call
reports an error status and a message, MetalOps.mm:259-261 -- RuntimeError
from the binding -- and never launches work).  Each call below names an
invalid argument; the check runs before any kernel is queued, and the stream
stays usable afterwards."""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def G():
    from kansaiml_amd import _native as N
    from kansaiml_amd.device import DeviceTensor as D
    assert N.available(), "no gfx950 device"
    return N, D


def test_invalid_arguments_are_reported(G):
    N, D = G
    a = D([64, 512], "int8")
    b = D([512, 512], "int8")
    sa, sb = D([1], "float64"), D([512], "float64")
    out = D([64, 512])
    x = D([64, 512])
    w = D([512])
    q = D([64, 512], "int8")
    npp = ctypes.c_int()
    cases = [
        # the int32 accumulator bound: 133144 * 127 * 127 < 2^31 <= 133145 * 127 * 127
        (("kh_gemm_i8", a.ptr, b.ptr, 64, 512, 133145, sa.ptr, 0, sb.ptr, 1, None, out.ptr, None), "overflow"),
        (("kh_gemm_i8", a.ptr, b.ptr, -1, 512, 512, sa.ptr, 0, sb.ptr, 1, None, out.ptr, None), "negative shape"),
        (("kh_gemm_i8", a.ptr, b.ptr, 64, 512, 512, sa.ptr, 0, sb.ptr, 1, None, None, None), "neither out nor acc_out"),
        (("kh_gemm_i8", a.ptr, b.ptr, 64, 512, 512, None, 0, sb.ptr, 1, None, out.ptr, None), "scales required"),
        (("kh_gemm_i8_ex", a.ptr, b.ptr, 64, 512, 512, sa.ptr, 0, sb.ptr, 1, None, 7, None, out.ptr, None, 0,
          ctypes.byref(npp)), "unknown activation"),
        (("kh_matmul_f32", x.ptr, x.ptr, None, 64, 512, 512, None), "null out"),
        (("kh_quantize_tensor", x.ptr, -1, q.ptr, sa.ptr), "negative size"),
        (("kh_quantize_tensor", x.ptr, 64, q.ptr, None), "null scale"),
        (("kh_quantize_rows", x.ptr, 64, 512, q.ptr, None), "null scales"),
        (("kh_dequantize_tensor", q.ptr, 64, None, out.ptr), "null pointer"),
        (("kh_layernorm", x.ptr, 4, 2048, w.ptr, w.ptr, 1e-5, out.ptr), "longer than 1024"),
        (("kh_causal_attention", x.ptr, 1, 8, 2, 32, out.ptr), "head dimension 64"),
        (("kh_causal_attention", x.ptr, 0, 8, 2, 64, out.ptr), "bad shape"),
        (("kh_attention_ex", x.ptr, 1, 8, 2, 64, 2, out.ptr, None, 0, None), "causal must be 0 or 1"),
        (("kh_linear_i8", x.ptr, 1, 512, b.ptr, 512, sb.ptr, 1, None, q.ptr, sa.ptr, None), "null out"),
        (("kh_graph_launch", None), "null graph"),
        (("kh_graph_capture_end", ctypes.byref(ctypes.c_void_p())), "no capture"),
    ]
    for args, fragment in cases:
        with pytest.raises(RuntimeError, match=fragment):
            N.call(*args)
    # a pointer the pool did not hand out is refused
    with pytest.raises(RuntimeError, match="not allocated by kh_alloc"):
        N.call("kh_free", ctypes.c_void_p(0x1000))
    # nothing was queued: the stream is clean and the next valid call works
    N.synchronize()
    xs = np.random.Generator(np.random.PCG64(1)).standard_normal((64, 512)).astype(np.float32)
    xd = D.from_host(xs)
    N.call("kh_quantize_tensor", xd.ptr, xs.size, q.ptr, sa.ptr)
    N.synchronize()
    m = float(np.abs(xs).astype(np.float64).max())
    assert sa.numpy()[0] == m / 127.0
