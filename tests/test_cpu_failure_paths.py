"""Failure paths on the CPU (no GPU in this container):

  * the capability probe and the interpreter without a device: kh_available()
    returns 0 and never raises (MetalOps.hpp:15-18 of the reference), and
    run_hip raises RuntimeError as run_metal does without Metal
    (python/kansai/kir.py:1647-1648 of the reference);
  * status codes mapped to the reference's exceptions: an allocation failure
    (the pool exhausted) raises MemoryError, like std::bad_alloc from
    core/src/Storage.cpp:30 there, through DeviceTensor with a stub library
    that refuses kh_alloc;
  * the host-side argument checks that stand between a caller and an
    out-of-bounds device read (LayerNorm parameters, attention's qkv shape)
    and QLinear's option checks, all raised before any device call;
  * the C oracle under AddressSanitizer and UndefinedBehaviorSanitizer.
"""

import ctypes
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "kansaiml_amd", "lib", "libkansai_hip.so")

needs_lib = pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")


def _has_gpu():
    from kansaiml_amd import _native as N
    return N.available()


@needs_lib
def test_available_is_zero_without_a_device():
    from kansaiml_amd import _native as N
    if _has_gpu():
        pytest.skip("a gfx950 device is present")
    assert N.lib().kh_available() == 0
    assert N.available() is False


@needs_lib
def test_run_hip_raises_runtime_error_without_a_device():
    from kansaiml_amd import kir
    if _has_gpu():
        pytest.skip("a gfx950 device is present")
    g = kir.Graph()
    x = g.placeholder([2, 3])
    g.output = g.add("relu", [x], [2, 3])
    with pytest.raises(RuntimeError, match="no gfx950"):
        kir.run_hip(g, np.zeros((2, 3), np.float32))
    with pytest.raises(RuntimeError, match="no gfx950"):
        kir.run_hip_planned(g, kir.plan_memory(g), None, np.zeros((2, 3), np.float32))


class _StubLib:
    """Stands in for the loaded library: kh_alloc reports the pool exhausted."""

    def __init__(self):
        self.calls = []

    def kh_alloc(self, nbytes, out):
        self.calls.append(("kh_alloc", nbytes))
        return 3  # KH_ERR_OOM

    def kh_last_error(self):
        return b"kh_alloc: out of device memory for 1099511627776 bytes"

    def kh_free(self, p):
        self.calls.append(("kh_free", p))
        return 0


def test_pool_exhaustion_raises_memory_error(monkeypatch):
    from kansaiml_amd import _native as N
    from kansaiml_amd.device import DeviceTensor
    stub = _StubLib()
    monkeypatch.setattr(N, "_lib", stub)
    with pytest.raises(MemoryError, match="out of device memory"):
        DeviceTensor([1 << 38], "float32")
    assert stub.calls == [("kh_alloc", 1 << 40)]


@pytest.mark.parametrize("rc,exc", [(1, RuntimeError), (2, RuntimeError), (3, MemoryError), (4, ValueError),
                                    (5, RuntimeError)])
def test_status_codes_map_to_reference_exceptions(monkeypatch, rc, exc):
    from kansaiml_amd import _native as N
    monkeypatch.setattr(N, "_lib", _StubLib())
    with pytest.raises(exc):
        N.check(rc, "stub")
    N.check(0)


def _fake(shape, dtype="float32"):
    """A DeviceTensor that owns no device memory (argument checks only)."""
    from kansaiml_amd.device import DeviceTensor
    t = object.__new__(DeviceTensor)
    t.ptr, t.shape, t.dtype, t.nbytes, t._owned, t.absmax_parts, t._base = (
        ctypes.c_void_p(0), list(shape), dtype, 0, False, None, None)
    return t


@pytest.mark.parametrize("fn", ["layer_norm", "layer_norm_quant", "layer_norm_quant_rows"])
@pytest.mark.parametrize("wshape,bshape", [([383], [384]), ([384], [1]), ([384, 1], [384])])
def test_layer_norm_parameters_checked(fn, wshape, bshape):
    from kansaiml_amd import hip as H
    x = _fake([16, 384])
    with pytest.raises((RuntimeError, TypeError)):
        getattr(H, fn)(x, _fake(wshape), _fake(bshape))
    with pytest.raises(TypeError):
        getattr(H, fn)(x, _fake([384], "int8"), _fake([384]))


@pytest.mark.parametrize("qkv_shape,batch,seq,heads,d_model", [
    ([512, 1152], 2, 256, 6, 384),    # rows != batch * seq
    ([512, 1151], 2, 256, 6, 384),    # not 3 * d_model columns
    ([512, 1152], 2, 256, 4, 384),    # head size 96, the kernel's is 64
    ([512, 960], 2, 256, 5, 320),     # fine shape, but ...
])
def test_attention_shape_checked(qkv_shape, batch, seq, heads, d_model):
    from kansaiml_amd import hip as H
    qkv = _fake(qkv_shape)
    if qkv_shape == [512, 960]:
        batch = 3  # ... rows != batch * seq
    with pytest.raises(RuntimeError):
        H.attention(qkv, batch, seq, heads, d_model)


@pytest.mark.parametrize("mshape", [[8, 7], [3, 1, 8, 8], [1, 3, 8, 8], [2, 2, 2, 8, 8], [9]])
def test_attention_mask_shape_checked(mshape):
    """A mask that does not broadcast to [batch, heads, seq, seq] (key axis
    last and full) is refused before any device call."""
    from kansaiml_amd import hip as H
    with pytest.raises(RuntimeError, match="broadcast"):
        H.attention(_fake([16, 384]), 2, 8, 2, 128, mask=_fake(mshape))
    with pytest.raises(TypeError, match="float32"):
        H.attention(_fake([16, 384]), 2, 8, 2, 128, mask=_fake([8, 8], "float64"))


@needs_lib
@pytest.mark.parametrize("elems,strides,msg", [
    (0, (0, 0, 64), "null or empty"),               # empty mask
    (64, (-1, 0, 8), "negative stride"),
    (1 << 40, (0, 0, 8), "2 GiB"),                  # size past 32-bit offsets
    (64, (1 << 33, 0, 8), "2 GiB"),                 # stride past 32-bit offsets
    (64, (0, 1 << 30, 1 << 30), "2 GiB"),           # strides whose reach passes 32-bit offsets
    (63, (0, 0, 8), "reach past"),                  # [8, 8] mask one element short
])
def test_attention_mask_abi_checks(elems, strides, msg):
    """kh_attention_masked's own checks of the mask's size and strides
    (called through the C ABI with fake pointers: every check comes before
    the first device access)."""
    from kansaiml_amd import _native as N
    fake = ctypes.c_void_p(256)
    with pytest.raises(Exception, match=msg):
        N.call("kh_attention_masked", fake, 1, 8, 2, 64, 1, fake, elems, *strides, fake, None)


@pytest.mark.parametrize("kw", [{"act_granularity": "col"}, {"act_granularity": "token"}, {"mode": "fp8"}])
def test_qlinear_rejects_unknown_options(kw):
    from kansaiml_amd.quantize import QLinear

    class Lin:  # never touched: the option check comes first
        weight = None
        bias = None

    with pytest.raises(ValueError):
        QLinear(Lin(), **{"mode": "int8", **kw})


def test_oracle_under_address_and_undefined_sanitizers():
    """The C restatement driven by oracle/oracle_selftest.c in a build with
    -fsanitize=address,undefined and no recovery: any out-of-bounds access,
    overflow or other undefined behaviour aborts the run."""
    r = subprocess.run(["make", "-s", "-B", "-C", os.path.join(ROOT, "oracle"), "sanitize"], capture_output=True,
                       text=True)
    assert r.returncode == 0, r.stderr
    exe = os.path.join(ROOT, "oracle", "lib", "oracle_selftest_san")
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    env.pop("LD_PRELOAD", None)
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "oracle selftest: ok" in r.stdout
