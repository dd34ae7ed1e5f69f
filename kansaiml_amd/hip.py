"""The HIP backend's tensor-level operations.

The role core/src/MetalOps.cpp plays for the reference's Metal backend
(core/src/MetalOps.cpp:8-140): check shapes, allocate the output (here from
the device pool), call the raw-pointer kernel.  Every function takes and
returns DeviceTensors; work is queued on the library stream and nothing
waits unless a result is downloaded or synchronize() is called.
"""

from __future__ import annotations

import ctypes

from . import _native as N
from .device import DeviceTensor

available = N.available
synchronize = N.synchronize


def _need(t: DeviceTensor, dtype: str, ndim: int | None, what: str):
    if not isinstance(t, DeviceTensor):
        raise TypeError(f"{what}: expected a DeviceTensor, got {type(t).__name__}")
    if t.dtype != dtype:
        raise TypeError(f"{what}: expected {dtype}, got {t.dtype}")
    if ndim is not None and len(t.shape) != ndim:
        raise RuntimeError(f"{what}: expected a {ndim}-D tensor, got shape {t.shape}")


def _opt(t):
    return t.ptr if t is not None else None


def _rows(t: DeviceTensor, dtype: str, what: str):
    """An activation of rank >= 2 read as the 2-D matrix it is in memory:
    (rows, cols, leading shape), rows = the product of every axis but the
    last.  The reference's batched matmul with a rank-2 right operand
    (core/src/Tensor.cpp:364-441) reads that one matrix for every batch
    index, which is the 2-D GEMM of these rows; a per-token quantize or a
    LayerNorm is per row either way."""
    _need(t, dtype, None, what)
    if len(t.shape) < 2:
        raise RuntimeError(f"{what}: expected a tensor of rank >= 2, got shape {t.shape}")
    lead = list(t.shape[:-1])
    rows = 1
    for d in lead:
        rows *= d
    return rows, t.shape[-1], lead


def _need_residual(residual: DeviceTensor, lead: list, n: int, what: str):
    _need(residual, "float32", None, f"{what}(residual)")
    if list(residual.shape) != lead + [n]:
        raise RuntimeError(f"{what}: residual must be {lead + [n]}, got {residual.shape}")


def _need_ln_params(x: DeviceTensor, w: DeviceTensor, b: DeviceTensor, what: str):
    """LayerNorm operands: x [..., D] fp32 (rows = every leading axis) and
    weight, bias fp32 [D].  The C ABI cannot see buffer sizes, so a short
    weight or bias would be read out of bounds on the device: refuse it
    here.  Returns (rows, D)."""
    rows, D, _ = _rows(x, "float32", f"{what}(x)")
    _need(w, "float32", 1, f"{what}(weight)")
    _need(b, "float32", 1, f"{what}(bias)")
    if w.shape[0] != D or b.shape[0] != D:
        raise RuntimeError(f"{what}: weight and bias must have {D} entries, got {w.shape} and {b.shape}")
    return rows, D


# ---------------------------------------------------------------------------
# quantize / dequantize (python/kansai/quantize.py:50-77)
# ---------------------------------------------------------------------------

def quantize_tensor(x: DeviceTensor):
    """Per-tensor symmetric int8: (codes int8 like x, scale float64[1])."""
    _need(x, "float32", None, "quantize_tensor")
    q = DeviceTensor(x.shape, "int8")
    s = DeviceTensor([1], "float64")
    N.call("kh_quantize_tensor", x.ptr, x.numel(), q.ptr, s.ptr)
    return q, s


def quantize_rows(x: DeviceTensor):
    """Per-row (per-token) symmetric int8 of a tensor of rank >= 2, a row
    being the last axis: (codes like x, scales [rows])."""
    rows, cols, _ = _rows(x, "float32", "quantize_rows")
    q = DeviceTensor(x.shape, "int8")
    s = DeviceTensor([rows], "float64")
    N.call("kh_quantize_rows", x.ptr, rows, cols, q.ptr, s.ptr)
    return q, s


def quantize_cols_packed(w: DeviceTensor):
    """Per-output-channel int8 of an [in, out] weight, packed [out, in]."""
    _need(w, "float32", 2, "quantize_cols_packed")
    k, n = w.shape
    q = DeviceTensor([n, k], "int8")
    s = DeviceTensor([n], "float64")
    N.call("kh_quantize_cols_packed", w.ptr, k, n, q.ptr, s.ptr)
    return q, s


def quantize_tensor_packed(w: DeviceTensor):
    """Per-tensor int8 of an [in, out] weight, packed [out, in]."""
    _need(w, "float32", 2, "quantize_tensor_packed")
    k, n = w.shape
    q = DeviceTensor([n, k], "int8")
    s = DeviceTensor([1], "float64")
    N.call("kh_quantize_tensor_packed", w.ptr, k, n, q.ptr, s.ptr)
    return q, s


def dequantize_tensor(q: DeviceTensor, scale: DeviceTensor) -> DeviceTensor:
    _need(q, "int8", None, "dequantize_tensor")
    _need(scale, "float64", None, "dequantize_tensor(scale)")
    out = DeviceTensor(q.shape, "float32")
    N.call("kh_dequantize_tensor", q.ptr, q.numel(), scale.ptr, out.ptr)
    return out


def dequantize_rows(q: DeviceTensor, scales: DeviceTensor) -> DeviceTensor:
    rows, cols, _ = _rows(q, "int8", "dequantize_rows")
    _need(scales, "float64", 1, "dequantize_rows(scales)")
    if scales.shape[0] != rows:
        raise RuntimeError("dequantize_rows: one scale per row required")
    out = DeviceTensor(q.shape, "float32")
    N.call("kh_dequantize_rows", q.ptr, rows, cols, scales.ptr, out.ptr)
    return out


def dequantize_packed(qp: DeviceTensor, scales: DeviceTensor) -> DeviceTensor:
    """Packed [out, in] codes back to the fp32 [in, out] weight."""
    _need(qp, "int8", 2, "dequantize_packed")
    _need(scales, "float64", 1, "dequantize_packed(scales)")
    n, k = qp.shape
    if scales.shape[0] not in (1, n):
        raise RuntimeError("dequantize_packed: scales must have 1 or out entries")
    out = DeviceTensor([k, n], "float32")
    N.call("kh_dequantize_packed", qp.ptr, k, n, scales.ptr, scales.shape[0], out.ptr)
    return out


# ---------------------------------------------------------------------------
# int8 GEMM
# ---------------------------------------------------------------------------

def _scale_mode(s: DeviceTensor, count: int, what: str) -> int:
    _need(s, "float64", 1, what)
    if s.shape[0] == count and count != 1:
        return 1
    if s.shape[0] == 1:
        return 0
    raise RuntimeError(f"{what}: expected 1 or {count} scales, got {s.shape[0]}")


def gemm_i8(a: DeviceTensor, b_packed: DeviceTensor, sa: DeviceTensor | None = None,
            sb: DeviceTensor | None = None, bias: DeviceTensor | None = None, *,
            want_out: bool = True, want_acc: bool = False):
    """a [..., M, K] int8 (every leading axis folded into the rows),
    b_packed [N, K] int8 -> out fp32 [..., M, N] (fused dequantize + bias)
    and/or acc int32 [..., M, N].  Returns (out, acc)."""
    M, K, lead = _rows(a, "int8", "gemm_i8(a)")
    _need(b_packed, "int8", 2, "gemm_i8(b)")
    Nn, K2 = b_packed.shape
    if K != K2:
        raise RuntimeError(f"gemm_i8: incompatible shapes {a.shape} x {b_packed.shape}^T")
    sa_mode = sb_mode = 0
    if want_out:
        sa_mode = _scale_mode(sa, M, "gemm_i8(sa)")
        sb_mode = _scale_mode(sb, Nn, "gemm_i8(sb)")
    if bias is not None:
        _need(bias, "float32", 1, "gemm_i8(bias)")
        if bias.shape[0] != Nn:
            raise RuntimeError("gemm_i8: bias must have N entries")
    out = DeviceTensor(lead + [Nn], "float32") if want_out else None
    acc = DeviceTensor(lead + [Nn], "int32") if want_acc else None
    N.call("kh_gemm_i8", a.ptr, b_packed.ptr, M, Nn, K, _opt(sa) if want_out else None, sa_mode,
           _opt(sb) if want_out else None, sb_mode, _opt(bias), _opt(out), _opt(acc))
    return out, acc


def dequantize_acc(acc: DeviceTensor, sa: DeviceTensor, sb: DeviceTensor,
                   bias: DeviceTensor | None = None) -> DeviceTensor:
    M, Nn, _ = _rows(acc, "int32", "dequantize_acc")
    sa_mode = _scale_mode(sa, M, "dequantize_acc(sa)")
    sb_mode = _scale_mode(sb, Nn, "dequantize_acc(sb)")
    out = DeviceTensor(acc.shape, "float32")
    N.call("kh_dequantize_acc", acc.ptr, M, Nn, sa.ptr, sa_mode, sb.ptr, sb_mode, _opt(bias), out.ptr)
    return out


def linear_i8(x: DeviceTensor, b_packed: DeviceTensor, sb: DeviceTensor,
              bias: DeviceTensor | None = None, return_codes: bool = False):
    """Per-token dynamic quantize of x [..., K] fp32 (M = every leading axis),
    then the int8 GEMM with the fused epilogue: out [..., N].  With
    return_codes, also returns the activation codes (int8, x's shape) and
    per-token scales (float64 [M]) the call produced."""
    M, K, lead = _rows(x, "float32", "linear_i8(x)")
    _need(b_packed, "int8", 2, "linear_i8(w)")
    Nn, K2 = b_packed.shape
    if K != K2:
        raise RuntimeError(f"linear_i8: incompatible shapes {x.shape} x {b_packed.shape}^T")
    sb_mode = _scale_mode(sb, Nn, "linear_i8(sb)")
    if bias is not None:
        _need(bias, "float32", 1, "linear_i8(bias)")
        if bias.shape[0] != Nn:
            raise RuntimeError("linear_i8: bias must have N entries")
    q = DeviceTensor(x.shape, "int8")
    sx = DeviceTensor([M], "float64")
    out = DeviceTensor(lead + [Nn], "float32")
    N.call("kh_linear_i8", x.ptr, M, K, b_packed.ptr, Nn, sb.ptr, sb_mode, _opt(bias), q.ptr, sx.ptr, out.ptr)
    return (out, q, sx) if return_codes else out


def linear_i8_tensor(x: DeviceTensor, b_packed: DeviceTensor, sb: DeviceTensor,
                     bias: DeviceTensor | None = None, return_codes: bool = False):
    """Per-tensor dynamic quantize of x [M, K] fp32 (one scale), then the int8
    GEMM with the fused epilogue: QLinear(mode="int8",
    act_granularity="tensor").  x [..., K] gives out [..., N].  With
    return_codes, also returns the codes (int8, x's shape) and the scale
    (float64 [1])."""
    M, K, lead = _rows(x, "float32", "linear_i8_tensor(x)")
    _need(b_packed, "int8", 2, "linear_i8_tensor(w)")
    Nn, K2 = b_packed.shape
    if K != K2:
        raise RuntimeError(f"linear_i8_tensor: incompatible shapes {x.shape} x {b_packed.shape}^T")
    sb_mode = _scale_mode(sb, Nn, "linear_i8_tensor(sb)")
    if bias is not None:
        _need(bias, "float32", 1, "linear_i8_tensor(bias)")
        if bias.shape[0] != Nn:
            raise RuntimeError("linear_i8_tensor: bias must have N entries")
    q = DeviceTensor(x.shape, "int8")
    sx = DeviceTensor([1], "float64")
    out = DeviceTensor(lead + [Nn], "float32")
    N.call("kh_linear_i8_tensor", x.ptr, M, K, b_packed.ptr, Nn, sb.ptr, sb_mode, _opt(bias), q.ptr, sx.ptr, out.ptr)
    return (out, q, sx) if return_codes else out


# ---------------------------------------------------------------------------
# fp32
# ---------------------------------------------------------------------------

def matmul(a: DeviceTensor, b: DeviceTensor, bias: DeviceTensor | None = None) -> DeviceTensor:
    """kan::metal_matmul's contract (core/src/MetalOps.cpp:10-17) --
    a.shape[-1] == b.shape[0], else RuntimeError("incompatible shapes") --
    with a of any rank >= 2 against a 2-D b: Tensor::matmul's batched path
    with a shared right operand (core/src/Tensor.cpp:364-441), out
    [..., M, N].  A batched right operand has no HIP kernel here."""
    M, K, lead = _rows(a, "float32", "matmul(a)")
    _need(b, "float32", None, "matmul(b)")
    if len(b.shape) != 2:
        raise NotImplementedError(f"matmul: a batched right operand {b.shape} has no HIP kernel (the int8 path's "
                                  "weights are 2-D)")
    if K != b.shape[0]:
        raise RuntimeError("matmul: incompatible shapes")
    Nn = b.shape[1]
    if bias is not None:
        _need(bias, "float32", 1, "matmul(bias)")
        if bias.shape[0] != Nn:
            raise RuntimeError("matmul: bias must have N entries")
    out = DeviceTensor(lead + [Nn], "float32")
    N.call("kh_matmul_f32", a.ptr, b.ptr, out.ptr, M, K, Nn, _opt(bias))
    return out


def add(a: DeviceTensor, b: DeviceTensor) -> DeviceTensor:
    _need(a, "float32", None, "add")
    _need(b, "float32", None, "add")
    if list(a.shape) != list(b.shape):
        raise RuntimeError("add: shapes must match")
    out = DeviceTensor(a.shape, "float32")
    N.call("kh_add", a.ptr, b.ptr, out.ptr, a.numel())
    return out


def add_bias(x: DeviceTensor, bias: DeviceTensor, relu: bool = False) -> DeviceTensor:
    """x [..., F] + bias [F] (Tensor.cpp:158-166, the bias broadcast over
    every leading axis), optionally followed by relu."""
    rows, F, _ = _rows(x, "float32", "add_bias")
    _need(bias, "float32", 1, "add_bias(bias)")
    if bias.shape[0] != F:
        raise RuntimeError("add_bias: bias must have features entries")
    out = DeviceTensor(x.shape, "float32")
    N.call("kh_add_bias", x.ptr, bias.ptr, out.ptr, rows, F, 1 if relu else 0)
    return out


def relu(x: DeviceTensor) -> DeviceTensor:
    _need(x, "float32", None, "relu")
    out = DeviceTensor(x.shape, "float32")
    N.call("kh_relu", x.ptr, out.ptr, x.numel())
    return out


# ---------------------------------------------------------------------------
# Fused producers of a per-tensor quantize: the absmax pass rides along
# ---------------------------------------------------------------------------

ABSMAX_PARTS = 8192  # partial maxima a fused producer may write


class AbsmaxParts:
    """Per-workgroup maxima of |x| (IEEE bit patterns in an int32 buffer) that
    a producer kernel wrote alongside x, for quantize_tensor_parts."""

    def __init__(self):
        self.buf = DeviceTensor([ABSMAX_PARTS], "int32")
        self._n = ctypes.c_int(0)

    @property
    def count(self) -> int:
        return self._n.value

    def release(self):
        self.buf.release()


ACTS = {None: 0, "gelu": 1}


def gemm_i8_fused(a: DeviceTensor, b_packed: DeviceTensor, sa: DeviceTensor, sb: DeviceTensor,
                  bias: DeviceTensor | None = None, *, act: str | None = None,
                  residual: DeviceTensor | None = None, absmax: bool = False):
    """gemm_i8's fp32 output with the following elementwise steps fused into
    its epilogue (bias, then act, then residual + y) and optionally the
    absmax partials of the result.  a [..., M, K] gives out [..., M, N].
    Returns (out, AbsmaxParts | None)."""
    M, K, lead = _rows(a, "int8", "gemm_i8(a)")
    _need(b_packed, "int8", 2, "gemm_i8(b)")
    Nn, K2 = b_packed.shape
    if K != K2:
        raise RuntimeError(f"gemm_i8: incompatible shapes {a.shape} x {b_packed.shape}^T")
    if act not in ACTS:
        raise ValueError(f"gemm_i8_fused: unknown activation {act!r}")
    sa_mode = _scale_mode(sa, M, "gemm_i8(sa)")
    sb_mode = _scale_mode(sb, Nn, "gemm_i8(sb)")
    if bias is not None:
        _need(bias, "float32", 1, "gemm_i8(bias)")
        if bias.shape[0] != Nn:
            raise RuntimeError("gemm_i8: bias must have N entries")
    if residual is not None:
        _need_residual(residual, lead, Nn, "gemm_i8_fused")
    out = DeviceTensor(lead + [Nn], "float32")
    parts = AbsmaxParts() if absmax else None
    N.call("kh_gemm_i8_ex", a.ptr, b_packed.ptr, M, Nn, K, sa.ptr, sa_mode, sb.ptr, sb_mode, _opt(bias), ACTS[act],
           _opt(residual), out.ptr, parts.buf.ptr if parts else None, ABSMAX_PARTS if parts else 0,
           ctypes.byref(parts._n) if parts else None)
    return out, parts


def gemm_i8_quant(a: DeviceTensor, b_packed: DeviceTensor, sa: DeviceTensor, sb: DeviceTensor,
                  bias: DeviceTensor | None = None, *, act: str | None = None,
                  residual: DeviceTensor | None = None):
    """quantize_tensor(gemm_i8_fused(...)) without writing the fp32 result:
    returns (codes int8 [..., M, N], scale float64 [1])."""
    M, K, lead = _rows(a, "int8", "gemm_i8(a)")
    _need(b_packed, "int8", 2, "gemm_i8(b)")
    Nn, K2 = b_packed.shape
    if K != K2:
        raise RuntimeError(f"gemm_i8: incompatible shapes {a.shape} x {b_packed.shape}^T")
    if act not in ACTS:
        raise ValueError(f"gemm_i8_quant: unknown activation {act!r}")
    sa_mode = _scale_mode(sa, M, "gemm_i8(sa)")
    sb_mode = _scale_mode(sb, Nn, "gemm_i8(sb)")
    if bias is not None:
        _need(bias, "float32", 1, "gemm_i8(bias)")
        if bias.shape[0] != Nn:
            raise RuntimeError("gemm_i8: bias must have N entries")
    if residual is not None:
        _need_residual(residual, lead, Nn, "gemm_i8_quant")
    q = DeviceTensor(lead + [Nn], "int8")
    s = DeviceTensor([1], "float64")
    N.call("kh_gemm_i8_quant", a.ptr, b_packed.ptr, M, Nn, K, sa.ptr, sa_mode, sb.ptr, sb_mode, _opt(bias),
           ACTS[act], _opt(residual), q.ptr, s.ptr)
    return q, s


def gemm_i8_quant_rows(a: DeviceTensor, b_packed: DeviceTensor, sa: DeviceTensor, sb: DeviceTensor,
                       bias: DeviceTensor | None = None, *, act: str | None = None):
    """quantize_rows(gemm_i8_fused(...)) without writing the fp32 result:
    returns (codes int8 [..., M, N], row scales float64 [M]).  sa holds one
    scale per row of a (a per-token activation)."""
    M, K, lead = _rows(a, "int8", "gemm_i8(a)")
    _need(b_packed, "int8", 2, "gemm_i8(b)")
    Nn, K2 = b_packed.shape
    if K != K2:
        raise RuntimeError(f"gemm_i8: incompatible shapes {a.shape} x {b_packed.shape}^T")
    if act not in ACTS:
        raise ValueError(f"gemm_i8_quant_rows: unknown activation {act!r}")
    sa_mode = _scale_mode(sa, M, "gemm_i8(sa)")
    sb_mode = _scale_mode(sb, Nn, "gemm_i8(sb)")
    if bias is not None:
        _need(bias, "float32", 1, "gemm_i8(bias)")
        if bias.shape[0] != Nn:
            raise RuntimeError("gemm_i8: bias must have N entries")
    q = DeviceTensor(lead + [Nn], "int8")
    s = DeviceTensor([M], "float64")
    N.call("kh_gemm_i8_quant_rows", a.ptr, b_packed.ptr, M, Nn, K, sa.ptr, sa_mode, sb.ptr, sb_mode, _opt(bias),
           ACTS[act], q.ptr, s.ptr)
    return q, s


def gemm_i8_qload(x: DeviceTensor, parts: AbsmaxParts, b_packed: DeviceTensor, sb: DeviceTensor,
                  bias: DeviceTensor | None = None, *, act: str | None = None,
                  residual: DeviceTensor | None = None, absmax: bool = False, want_scale: bool = False):
    """gemm_i8_fused(quantize_tensor_parts(x, parts)) without writing the
    activation's codes: x fp32 [..., M, K] with the absmax partials its
    producer wrote.  Returns (out, AbsmaxParts | None), plus the
    activation's scale (float64 [1]) when want_scale."""
    M, K, lead = _rows(x, "float32", "gemm_i8_qload(x)")
    _need(b_packed, "int8", 2, "gemm_i8_qload(b)")
    if parts is None or parts.count <= 0:
        raise RuntimeError("gemm_i8_qload: the producer wrote no partials")
    Nn, K2 = b_packed.shape
    if K != K2:
        raise RuntimeError(f"gemm_i8_qload: incompatible shapes {x.shape} x {b_packed.shape}^T")
    if act not in ACTS:
        raise ValueError(f"gemm_i8_qload: unknown activation {act!r}")
    sb_mode = _scale_mode(sb, Nn, "gemm_i8_qload(sb)")
    if bias is not None:
        _need(bias, "float32", 1, "gemm_i8_qload(bias)")
        if bias.shape[0] != Nn:
            raise RuntimeError("gemm_i8_qload: bias must have N entries")
    if residual is not None:
        _need_residual(residual, lead, Nn, "gemm_i8_qload")
    out = DeviceTensor(lead + [Nn], "float32")
    scale = DeviceTensor([1], "float64") if want_scale else None
    out_parts = AbsmaxParts() if absmax else None
    N.call("kh_gemm_i8_qload", x.ptr, M, Nn, K, parts.buf.ptr, parts.count, b_packed.ptr, sb.ptr, sb_mode,
           _opt(bias), ACTS[act], _opt(residual), out.ptr, _opt(scale), out_parts.buf.ptr if out_parts else None,
           ABSMAX_PARTS if out_parts else 0, ctypes.byref(out_parts._n) if out_parts else None)
    if want_scale:
        return out, out_parts, scale
    return out, out_parts


def layer_norm_quant(x: DeviceTensor, w: DeviceTensor, b: DeviceTensor, eps: float = 1e-5):
    """quantize_tensor(layer_norm(x)) without writing the fp32 output:
    returns (codes int8 like x, scale float64 [1])."""
    rows, D = _need_ln_params(x, w, b, "layer_norm_quant")
    q = DeviceTensor(x.shape, "int8")
    s = DeviceTensor([1], "float64")
    N.call("kh_layernorm_quant", x.ptr, rows, D, w.ptr, b.ptr, eps, q.ptr, s.ptr)
    return q, s


def layer_norm_quant_rows(x: DeviceTensor, w: DeviceTensor, b: DeviceTensor, eps: float = 1e-5):
    """LayerNorm with its output quantized per row in one pass (the fp32
    values are never stored).  Returns (codes int8 like x, scales float64
    [rows])."""
    rows, D = _need_ln_params(x, w, b, "layer_norm_quant_rows")
    q = DeviceTensor(x.shape, "int8")
    s = DeviceTensor([rows], "float64")
    N.call("kh_layernorm_quant_rows", x.ptr, rows, D, w.ptr, b.ptr, eps, q.ptr, s.ptr)
    return q, s


def layer_norm(x: DeviceTensor, w: DeviceTensor, b: DeviceTensor, eps: float = 1e-5, *, absmax: bool = False):
    """LayerNorm over the last axis (nn.py:308-331).  Returns (out, AbsmaxParts | None)."""
    rows, D = _need_ln_params(x, w, b, "layer_norm")
    out = DeviceTensor(x.shape, "float32")
    parts = AbsmaxParts() if absmax else None
    N.call("kh_layernorm_ex", x.ptr, rows, D, w.ptr, b.ptr, eps, out.ptr,
           parts.buf.ptr if parts else None, ABSMAX_PARTS if parts else 0, ctypes.byref(parts._n) if parts else None)
    return out, parts


def mask_strides(mask: DeviceTensor, batch: int, heads: int, seq: int) -> tuple:
    """Element strides (batch, head, query) of an additive attention mask
    whose shape broadcasts to [batch, heads, seq, seq] (nn.py:421-422's
    scores.add(mask)): right-aligned, each axis of size 1 or the full size,
    the key axis full and contiguous.  A size-1 axis gets stride 0."""
    _need(mask, "float32", None, "attention(mask)")
    shape = list(mask.shape)
    if not 1 <= len(shape) <= 4 or shape[-1] != seq:
        raise RuntimeError(f"attention: mask {shape} does not broadcast to [{batch}, {heads}, {seq}, {seq}] with "
                           f"its last axis the {seq} keys")
    full = [batch, heads, seq, seq]
    shape4 = [1] * (4 - len(shape)) + shape
    strides, step = [0, 0, 0, 0], 1
    for ax in (3, 2, 1, 0):
        if shape4[ax] not in (1, full[ax]):
            raise RuntimeError(f"attention: mask {shape} does not broadcast to {full}")
        strides[ax] = step if shape4[ax] != 1 else 0
        step *= shape4[ax]
    return strides[0], strides[1], strides[2]


def attention(qkv: DeviceTensor, batch: int, seq: int, heads: int, d_model: int, *, causal: bool = True,
              absmax: bool = False, mask: DeviceTensor | None = None):
    """Multi-head attention core (nn.py:381-427), with the causal mask or none,
    and optionally the caller's additive mask (broadcast to [batch, heads,
    seq, seq]).  Returns (out, AbsmaxParts | None)."""
    _need(qkv, "float32", 2, "attention(qkv)")
    if heads <= 0 or d_model != heads * 64:
        raise RuntimeError(f"attention: d_model must be heads * 64 (the kernel's head size), got {d_model} "
                           f"for {heads} heads")
    if batch < 0 or seq < 0 or list(qkv.shape) != [batch * seq, 3 * d_model]:
        raise RuntimeError(f"attention: qkv must be [batch * seq, 3 * d_model] = [{batch * seq}, {3 * d_model}], "
                           f"got {qkv.shape}")
    strides = mask_strides(mask, batch, heads, seq) if mask is not None else None  # checked before allocating
    out = DeviceTensor([batch * seq, d_model], "float32")
    if mask is not None:
        sb, sh, sq = strides
        N.call("kh_attention_masked", qkv.ptr, batch, seq, heads, d_model // heads, int(bool(causal)), mask.ptr,
               mask.numel(), sb, sh, sq, out.ptr, None)
        parts = None
        if absmax:
            parts = AbsmaxParts()
            N.call("kh_absmax_parts", out.ptr, out.numel(), parts.buf.ptr, ABSMAX_PARTS, ctypes.byref(parts._n))
        return out, parts
    parts = AbsmaxParts() if absmax else None
    N.call("kh_attention_ex", qkv.ptr, batch, seq, heads, d_model // heads, int(bool(causal)), out.ptr,
           parts.buf.ptr if parts else None, ABSMAX_PARTS if parts else 0, ctypes.byref(parts._n) if parts else None)
    return out, parts


class RowParts:
    """Max |x| bits of pieces of every row of x (int32 [rows, per_row]) that a
    producer kernel wrote alongside x, for a per-row quantize of x inside
    the GEMM that consumes it (gemm_i8_qload_rows)."""

    def __init__(self, rows: int, per_row: int):
        self.buf = DeviceTensor([rows, per_row], "int32")
        self.per_row = per_row

    def release(self):
        self.buf.release()


def attention_rows(qkv: DeviceTensor, batch: int, seq: int, heads: int, d_model: int, *, causal: bool = True,
                   mask: DeviceTensor | None = None):
    """attention() also writing the max |out| bits of every (row, head).
    Returns (out, RowParts)."""
    _need(qkv, "float32", 2, "attention(qkv)")
    if heads <= 0 or d_model != heads * 64:
        raise RuntimeError(f"attention: d_model must be heads * 64 (the kernel's head size), got {d_model} "
                           f"for {heads} heads")
    if batch < 0 or seq < 0 or list(qkv.shape) != [batch * seq, 3 * d_model]:
        raise RuntimeError(f"attention: qkv must be [batch * seq, 3 * d_model] = [{batch * seq}, {3 * d_model}], "
                           f"got {qkv.shape}")
    strides = mask_strides(mask, batch, heads, seq) if mask is not None else None  # checked before allocating
    out = DeviceTensor([batch * seq, d_model], "float32")
    rp = RowParts(batch * seq, heads)
    if mask is not None:
        sb, sh, sq = strides
        N.call("kh_attention_masked", qkv.ptr, batch, seq, heads, d_model // heads, int(bool(causal)), mask.ptr,
               mask.numel(), sb, sh, sq, out.ptr, rp.buf.ptr)
        return out, rp
    N.call("kh_attention_rows", qkv.ptr, batch, seq, heads, d_model // heads, int(bool(causal)), out.ptr, rp.buf.ptr)
    return out, rp


def gemm_i8_qload_rows(x: DeviceTensor, rp: RowParts, b_packed: DeviceTensor, sb: DeviceTensor,
                       bias: DeviceTensor | None = None, *, act: str | None = None,
                       residual: DeviceTensor | None = None, want_scales: bool = False):
    """The per-row (per-token) quantize of x [..., M, K] fp32 inside the int8
    GEMM that consumes it, each row's scale from its producer's partials:
    the same output as quantize_rows(x) then gemm_i8_fused with per-row
    scales, without writing the codes.  Returns out, or (out, row scales
    float64 [M]) when want_scales."""
    M, K, lead = _rows(x, "float32", "gemm_i8_qload_rows(x)")
    _need(b_packed, "int8", 2, "gemm_i8_qload_rows(b)")
    Nn, K2 = b_packed.shape
    if K != K2:
        raise RuntimeError(f"gemm_i8_qload_rows: incompatible shapes {x.shape} x {b_packed.shape}^T")
    if list(rp.buf.shape) != [M, rp.per_row]:
        raise RuntimeError(f"gemm_i8_qload_rows: partials {rp.buf.shape} do not cover the {M} rows of x")
    if act not in ACTS:
        raise ValueError(f"gemm_i8_qload_rows: unknown activation {act!r}")
    sb_mode = _scale_mode(sb, Nn, "gemm_i8_qload_rows(sb)")
    if bias is not None:
        _need(bias, "float32", 1, "gemm_i8_qload_rows(bias)")
        if bias.shape[0] != Nn:
            raise RuntimeError("gemm_i8_qload_rows: bias must have N entries")
    if residual is not None:
        _need_residual(residual, lead, Nn, "gemm_i8_qload_rows")
    out = DeviceTensor(lead + [Nn], "float32")
    scales = DeviceTensor([M], "float64") if want_scales else None
    N.call("kh_gemm_i8_qload_rows", x.ptr, M, Nn, K, rp.buf.ptr, rp.per_row, b_packed.ptr, sb.ptr, sb_mode,
           _opt(bias), ACTS[act], _opt(residual), out.ptr, _opt(scales))
    return (out, scales) if want_scales else out


def causal_attention(qkv: DeviceTensor, batch: int, seq: int, heads: int, d_model: int, *, absmax: bool = False):
    """attention() under the causal mask."""
    return attention(qkv, batch, seq, heads, d_model, causal=True, absmax=absmax)


def quantize_tensor_parts(x: DeviceTensor, parts: AbsmaxParts):
    """quantize_tensor with the absmax partials its producer wrote."""
    _need(x, "float32", None, "quantize_tensor(x)")
    if parts.count <= 0:
        raise RuntimeError("quantize_tensor_parts: the producer wrote no partials")
    q = DeviceTensor(x.shape, "int8")
    s = DeviceTensor([1], "float64")
    N.call("kh_quantize_tensor_parts", x.ptr, x.numel(), parts.buf.ptr, parts.count, q.ptr, s.ptr)
    return q, s
