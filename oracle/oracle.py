"""CPU oracle for the int8 quantize -> int8 matmul -> dequantize path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg import this module, as the checker; the
product package (kansaiml_amd/) never imports it and has no CPU fallback.

Three layers, each citing the reference it follows:

* ``py_*``   pure-Python restatements of python/kansai/quantize.py:50-77
             using CPython's own ``round()`` and binary64 floats, exactly
             the operations the reference executes.  Small inputs only.
* ``ko_*``   ctypes wrappers over oracle/kansai_oracle.c (the C
             restatement, built into oracle/lib/ by oracle/Makefile).
* ``ref_*``  ctypes wrappers over the reference's own compiled
             backend/cpu/src/Ops.cpp (oracle/_ref/, see oracle/Makefile).
"""

from __future__ import annotations

import ctypes
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(HERE, "lib", "libkansai_oracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libkansai_cpu_ref.so")

KO_OK = 0
KO_NONFINITE = 4


class NonFiniteError(ValueError):
    """Raised where the reference's round() would raise on NaN/inf."""


# ---------------------------------------------------------------------------
# Pure-Python restatement (quantize.py:50-77), the semantics themselves.
# ---------------------------------------------------------------------------

def f32(x: float) -> float:
    """binary64 -> binary32 (round to nearest even) -> binary64; what
    core.from_flat does to each element (python/bindings.cpp:133-134)."""
    return struct.unpack("<f", struct.pack("<f", x))[0]


def py_quantize_symmetric(flat):
    """quantize.py:66-70 on a list of Python floats (already fp32 values)."""
    max_abs = max((abs(v) for v in flat), default=0.0)
    scale = max_abs / 127.0 if max_abs > 0.0 else 1.0
    q = [max(-127, min(127, round(v / scale))) for v in flat]
    return q, scale


def py_dequantize(q, scale):
    """quantize.py:76 plus from_flat's binary32 narrowing."""
    return [f32(v * scale) for v in q]


# ---------------------------------------------------------------------------
# C restatement (oracle/kansai_oracle.c)
# ---------------------------------------------------------------------------

_lib = None
_ref = None


def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_LIB):
            raise FileNotFoundError(f"{ORACLE_LIB} missing: run `make -C oracle`")
        L = ctypes.CDLL(ORACLE_LIB)
        i64 = ctypes.c_int64
        vp = ctypes.c_void_p
        for name, args, res in [
            ("ko_quantize_tensor", [vp, i64, vp, vp], ctypes.c_int),
            ("ko_quantize_rows", [vp, i64, i64, vp, vp], ctypes.c_int),
            ("ko_quantize_cols_packed", [vp, i64, i64, vp, vp], ctypes.c_int),
            ("ko_quantize_tensor_packed", [vp, i64, i64, vp, vp], ctypes.c_int),
            ("ko_dequantize_tensor", [vp, i64, ctypes.c_double, vp], None),
            ("ko_dequantize_rows", [vp, i64, i64, vp, vp], None),
            ("ko_gemm_i8", [vp, vp, i64, i64, i64, vp], None),
            ("ko_epilogue", [vp, i64, i64, vp, i64, vp, i64, vp, vp], None),
            ("ko_matmul_f32", [vp, vp, vp, i64, i64, i64], None),
            ("ko_add_bias", [vp, vp, vp, i64, i64], None),
        ]:
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _f32c(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def _check(rc):
    if rc == KO_NONFINITE:
        raise NonFiniteError("cannot quantize a non-finite value (NaN or inf)")
    if rc != KO_OK:
        raise RuntimeError(f"oracle error {rc}")


def ko_quantize_tensor(x):
    x = _f32c(x)
    q = np.empty(x.shape, np.int8)
    s = np.zeros(1, np.float64)
    _check(lib().ko_quantize_tensor(_ptr(x), x.size, _ptr(q), _ptr(s)))
    return q, float(s[0])


def ko_quantize_rows(x):
    x = _f32c(x)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.int8)
    s = np.zeros(rows, np.float64)
    _check(lib().ko_quantize_rows(_ptr(x), rows, cols, _ptr(q), _ptr(s)))
    return q, s


def ko_quantize_cols_packed(w):
    w = _f32c(w)
    k, n = w.shape
    q = np.empty((n, k), np.int8)
    s = np.zeros(n, np.float64)
    _check(lib().ko_quantize_cols_packed(_ptr(w), k, n, _ptr(q), _ptr(s)))
    return q, s


def ko_quantize_tensor_packed(w):
    w = _f32c(w)
    k, n = w.shape
    q = np.empty((n, k), np.int8)
    s = np.zeros(1, np.float64)
    _check(lib().ko_quantize_tensor_packed(_ptr(w), k, n, _ptr(q), _ptr(s)))
    return q, float(s[0])


def ko_dequantize_tensor(q, scale):
    q = np.ascontiguousarray(q, dtype=np.int8)
    out = np.empty(q.shape, np.float32)
    lib().ko_dequantize_tensor(_ptr(q), q.size, float(scale), _ptr(out))
    return out


def ko_dequantize_rows(q, scales):
    q = np.ascontiguousarray(q, dtype=np.int8)
    s = np.ascontiguousarray(scales, dtype=np.float64)
    rows, cols = q.shape
    out = np.empty((rows, cols), np.float32)
    lib().ko_dequantize_rows(_ptr(q), rows, cols, _ptr(s), _ptr(out))
    return out


def ko_gemm_i8(a, bt):
    """a: [M,K] int8, bt: [N,K] int8 (packed weight) -> int32 [M,N]."""
    a = np.ascontiguousarray(a, dtype=np.int8)
    bt = np.ascontiguousarray(bt, dtype=np.int8)
    M, K = a.shape
    N, K2 = bt.shape
    assert K == K2
    acc = np.empty((M, N), np.int32)
    lib().ko_gemm_i8(_ptr(a), _ptr(bt), M, N, K, _ptr(acc))
    return acc


def ko_epilogue(acc, sa, sb, bias=None):
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    M, N = acc.shape
    sa = np.ascontiguousarray(np.atleast_1d(sa), dtype=np.float64)
    sb = np.ascontiguousarray(np.atleast_1d(sb), dtype=np.float64)
    assert sa.size in (1, M) and sb.size in (1, N)
    out = np.empty((M, N), np.float32)
    bp = None
    if bias is not None:
        bias = _f32c(bias)
        assert bias.size == N
        bp = _ptr(bias)
    lib().ko_epilogue(_ptr(acc), M, N, _ptr(sa), sa.size, _ptr(sb), sb.size, bp, _ptr(out))
    return out


def ko_matmul_f32(a, b):
    a, b = _f32c(a), _f32c(b)
    M, K = a.shape
    K2, N = b.shape
    assert K == K2
    out = np.empty((M, N), np.float32)
    lib().ko_matmul_f32(_ptr(a), _ptr(b), _ptr(out), M, K, N)
    return out


def ko_add_bias(x, bias):
    x, bias = _f32c(x), _f32c(bias)
    out = np.empty(x.shape, np.float32)
    lib().ko_add_bias(_ptr(x), _ptr(bias), _ptr(out), x.shape[0], x.shape[1])
    return out


# ---------------------------------------------------------------------------
# The reference's own compiled CPU kernels (oracle/_ref)
# ---------------------------------------------------------------------------

def ref_available() -> bool:
    return os.path.exists(REF_LIB)


def ref():
    global _ref
    if _ref is None:
        if not ref_available():
            raise FileNotFoundError(f"{REF_LIB} missing: run `make -C oracle` where /root/reference exists")
        R = ctypes.CDLL(REF_LIB)
        i64 = ctypes.c_int64
        vp = ctypes.c_void_p
        R.kref_matmul.argtypes = [vp, vp, vp, i64, i64, i64]
        R.kref_matmul.restype = None
        R.kref_add_bias_broadcast.argtypes = [vp, vp, vp, i64, i64]
        R.kref_add_bias_broadcast.restype = None
        R.kref_batched_matmul_shared.argtypes = [vp, vp, vp, i64, i64, i64, i64]
        R.kref_batched_matmul_shared.restype = None
        R.kref_add_broadcast_rank3.argtypes = [vp, vp, vp, i64, i64, i64]
        R.kref_add_broadcast_rank3.restype = None
        _ref = R
    return _ref


def ref_matmul(a, b):
    """kan::cpu::matmul (backend/cpu/src/Ops.cpp:322-339), the real code."""
    a, b = _f32c(a), _f32c(b)
    M, K = a.shape
    _, N = b.shape
    out = np.empty((M, N), np.float32)
    ref().kref_matmul(_ptr(a), _ptr(b), _ptr(out), M, K, N)
    return out


def ref_add_bias(x, bias):
    """kan::cpu::add_bias_broadcast (backend/cpu/src/Ops.cpp:34-38)."""
    x, bias = _f32c(x), _f32c(bias)
    out = np.empty(x.shape, np.float32)
    ref().kref_add_bias_broadcast(_ptr(x), _ptr(bias), _ptr(out), x.shape[0], x.shape[1])
    return out


def ref_batched_matmul(a, b):
    """kan::cpu::batched_matmul (backend/cpu/src/Ops.cpp:427-437) as
    Tensor::matmul's batched path calls it for a [batch, M, K] left operand
    and a shared 2-D right operand (core/src/Tensor.cpp:364-393)."""
    a, b = _f32c(a), _f32c(b)
    B, M, K = a.shape
    _, N = b.shape
    out = np.empty((B, M, N), np.float32)
    ref().kref_batched_matmul_shared(_ptr(a), _ptr(b), _ptr(out), B, M, K, N)
    return out


def ref_add_broadcast(x, bias):
    """kan::cpu::add_broadcast (backend/cpu/src/Ops.cpp:121-125) for
    [batch, M, N] + [N], the general path Tensor::add takes for a rank-3
    activation plus a bias (core/src/Tensor.cpp:158-166)."""
    x, bias = _f32c(x), _f32c(bias)
    B, M, N = x.shape
    out = np.empty(x.shape, np.float32)
    ref().kref_add_broadcast_rank3(_ptr(x), _ptr(bias), _ptr(out), B, M, N)
    return out


# ---------------------------------------------------------------------------
# Composite: the int8 Linear of config C1 (quantize x and W, int8 GEMM,
# dequantize epilogue + bias).
# ---------------------------------------------------------------------------

def int8_linear(x, w, bias=None, x_gran="tensor", w_gran="tensor"):
    """x: [M,K] fp32, w: [K,N] fp32 ([in,out], nn.py:77).  Returns
    (y fp32 [M,N], acc int32 [M,N], qx, sx, qw_packed, sw)."""
    if x_gran == "tensor":
        qx, sx = ko_quantize_tensor(x)
        sx = np.array([sx])
    else:
        qx, sx = ko_quantize_rows(x)
    if w_gran == "tensor":
        qw, sw = ko_quantize_tensor_packed(w)
        sw = np.array([sw])
    else:
        qw, sw = ko_quantize_cols_packed(w)
    acc = ko_gemm_i8(qx, qw)
    y = ko_epilogue(acc, sx, sw, bias)
    return y, acc, qx, sx, qw, sw
