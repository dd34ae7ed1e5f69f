"""kh_linear_i8_noalloc: the allocation-free variant of kh_linear_i8.

Called through the C ABI.  Its output must equal kh_linear_i8's bit for bit
(both are the per-token quantize, the exact int32 GEMM and the binary64
dequantize epilogue), on two calls in a row, the second with a smaller input
(the fixed scratch array keeps the first call's codes), with no pool
allocation and no use of the library's scratch area meanwhile.  Sizes beyond
the fixed array are rejected."""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    from kansaiml_amd import _native as N
    from kansaiml_amd.device import DeviceTensor
    assert N.available(), "no gfx950 device"
    N.call("kh_init", 0)  # the no-alloc entry point never initialises a device itself
    return N, DeviceTensor


def _case(D, M, K, N_, seed, per_col=True):
    g = np.random.Generator(np.random.PCG64(seed))
    x = g.standard_normal((M, K), dtype=np.float32)
    w = g.integers(-127, 128, size=(N_, K), dtype=np.int8)
    sb = (g.random(N_ if per_col else 1) * 1e-3 + 1e-4).astype(np.float64)
    bias = g.standard_normal(N_, dtype=np.float32)
    return {"x": D.from_host(x), "w": D.from_host(w), "sb": D.from_host(sb), "bias": D.from_host(bias),
            "M": M, "K": K, "N": N_, "per_col": int(per_col)}


def _with_alloc(N, D, c):
    q = D.empty([c["M"], c["K"]], "int8")
    sx = D.empty([max(c["M"], 1)], "float64")
    out = D.empty([c["M"], c["N"]], "float32")
    N.call("kh_linear_i8", c["x"].ptr, c["M"], c["K"], c["w"].ptr, c["N"], c["sb"].ptr, c["per_col"],
           c["bias"].ptr, q.ptr, sx.ptr, out.ptr)
    return out.numpy().view(np.uint32)


# (first call, second smaller call): the skinny GEMM after a per-row quantize,
# the one-launch decode kernel (M <= 2), and the tiled GEMM for larger M.
PAIRS = [
    ((32, 4096, 4096, True), (8, 4096, 1024, True)),
    ((16, 8192, 1024, True), (8, 16384, 512, False)),  # shapes kh_linear_i8 runs with a K split
    ((2, 4096, 11008, True), (1, 2048, 512, True)),
    ((512, 2048, 1024, True), (64, 512, 512, False)),
]


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_linear_i8(lib, first, second):
    N, D = lib
    cases = [_case(D, *first[:3], seed=11, per_col=first[3]), _case(D, *second[:3], seed=12, per_col=second[3])]
    want = [_with_alloc(N, D, c) for c in cases]
    outs = [D.empty([c["M"], c["N"]], "float32") for c in cases]
    N.synchronize()
    before = N.pool_stats()
    scratch_before = N.scratch_stats()
    for c, out in zip(cases, outs):
        print(f"noalloc M={c['M']} K={c['K']} N={c['N']}", flush=True)
        N.call("kh_linear_i8_noalloc", c["x"].ptr, c["M"], c["K"], c["w"].ptr, c["N"], c["sb"].ptr, c["per_col"],
               c["bias"].ptr, out.ptr)
    N.synchronize()
    # (pool_stats counts kh_alloc requests too: a block taken from a free list
    # and returned would leave the byte counts unchanged)
    assert N.pool_stats() == before, "the no-alloc entry point drew from the pool"
    # The library scratch (outside the pool) is neither requested nor grown:
    # a path through it would count a request even where it no longer grows.
    assert N.scratch_stats() == scratch_before, "the no-alloc entry point used the library scratch"
    for w, out in zip(want, outs):
        np.testing.assert_array_equal(out.numpy().view(np.uint32), w)


def test_noalloc_rejects_sizes_beyond_the_array(lib):
    N, D = lib
    out = ctypes.c_void_p(1)  # never dereferenced: the size check comes first
    with pytest.raises(RuntimeError, match="exceeds the fixed scratch"):
        N.call("kh_linear_i8_noalloc", None, 4096, 16, None, 16, None, 1, None, out)
    with pytest.raises(RuntimeError, match="exceed the fixed scratch"):
        N.call("kh_linear_i8_noalloc", None, 1024, 4096, None, 16, None, 1, None, out)
