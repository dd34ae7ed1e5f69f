"""The reference's int8 quantization API (python/kansai/quantize.py), computed
on the GPU.

Same names, argument meaning and results as the reference:
  quantize_symmetric(tensor) -> (q: list[int], scale: float, shape: list[int])
  dequantize(q, scale, shape) -> fp32 tensor
  QTensor (q, scale, shape, from_tensor, dequantize, nbytes)
  qlinear(x, qweight, bias) = x @ dequantize(W) + bias
  QLinear(linear)
with the reference's arithmetic bit for bit (binary64 scale m/127, binary64
division, round half to even, clamp to [-127, 127], zero tensor -> scale 1.0;
dequantize = binary32(binary64 q * scale)), and ValueError for NaN/inf input
as the reference's round() raises.

Beyond the reference (which has no int8 kernel, quantize.py:30-44): a
QTensor here lives on the device (int8 codes + binary64 scales) and may be
per-tensor, per-row (per token) or per-column (per output channel, stored
packed [out, in] for the GEMM); QLinear(linear, mode="int8") quantizes its
input dynamically and runs the int8 GEMM with a fused dequantize + bias
epilogue.  Traced through kansaiml_amd.kir (or any tracer on the reference's
schema that has the three emitters), QLinear emits quantize /
int8_matmul / dequantize nodes.
"""

from __future__ import annotations

import math

import numpy as np

from . import _native as N
from . import hip as H
from .device import DeviceTensor, to_device


def _shape_of(t) -> list:
    return [int(s) for s in getattr(t, "shape", np.shape(t))]


class QTensor:
    """int8 codes + binary64 scales on the device.

    granularity: "tensor" (one scale, the reference's only kind), "row" (one
    per row along the last axis: per token of [batch, seq, d] activations)
    or "col" (one per column of an [in, out] weight).  packed: codes stored K-contiguous [out, in] for the GEMM (the
    logical shape stays [in, out])."""

    __slots__ = ("codes", "scales", "shape", "granularity", "packed", "owned")

    def __init__(self, codes: DeviceTensor, scales: DeviceTensor, shape, granularity: str = "tensor",
                 packed: bool = False, owned: bool = True):
        self.codes = codes
        self.scales = scales
        self.shape = list(shape)
        self.granularity = granularity
        self.packed = packed
        self.owned = owned

    # -- construction ------------------------------------------------------
    @staticmethod
    def from_tensor(tensor, granularity: str = "tensor") -> "QTensor":
        """quantize.py:95-98.  granularity "row" quantizes each row (the last
        axis, every leading axis folded into the rows) separately; a 1-D
        tensor is one row."""
        x = to_device(tensor, "float32")
        if granularity == "tensor":
            q, s = H.quantize_tensor(x)
        elif granularity == "row":
            q, s = H.quantize_rows(x if len(x.shape) >= 2 else x.reshape([1, x.numel()]))
        else:
            raise ValueError(f"from_tensor: granularity must be 'tensor' or 'row', got {granularity!r}")
        N.synchronize()  # NaN/inf -> ValueError here, as in the reference
        return QTensor(q, s, _shape_of(tensor), granularity, packed=False)

    @staticmethod
    def from_weight(weight, granularity: str = "tensor") -> "QTensor":
        """An nn.Linear weight [in, out] (python/kansai/nn.py:74-81) quantized
        per tensor or per output channel ("col") and packed [out, in]."""
        w = to_device(weight, "float32")
        if len(w.shape) != 2:
            raise ValueError("from_weight: a 2-D [in, out] weight is required")
        if granularity == "tensor":
            q, s = H.quantize_tensor_packed(w)
        elif granularity == "col":
            q, s = H.quantize_cols_packed(w)
        else:
            raise ValueError(f"from_weight: granularity must be 'tensor' or 'col', got {granularity!r}")
        N.synchronize()
        return QTensor(q, s, list(w.shape), granularity, packed=True)

    # -- the reference's accessors -------------------------------------------
    @property
    def q(self) -> list:
        """Codes as Python ints in logical (row-major) order."""
        c = self.codes.numpy()
        if self.packed:
            c = c.T
        return c.reshape(-1).astype(int).tolist()

    @property
    def scale(self):
        s = self.scales.numpy()
        return float(s[0]) if self.granularity == "tensor" else s.tolist()

    def dequantize(self) -> DeviceTensor:
        """quantize.py:73-77 / 100-101: binary32(binary64 q * scale), in the
        logical layout."""
        if self.packed:
            return H.dequantize_packed(self.codes, self.scales)
        if self.granularity == "row":
            return H.dequantize_rows(self.codes, self.scales).reshape(self.shape)
        return H.dequantize_tensor(self.codes, self.scales).reshape(self.shape)

    def nbytes(self) -> int:
        """1 byte per element (quantize.py:103-109)."""
        return math.prod(self.shape)

    def __repr__(self):
        return f"QTensor(shape={self.shape}, granularity={self.granularity}, packed={self.packed}, nbytes={self.nbytes()})"


def quantize_symmetric(tensor):
    """quantize.py:50-70: (q as list of ints in [-127, 127], scale, shape)."""
    qt = QTensor.from_tensor(tensor, "tensor")
    return qt.q, qt.scale, list(qt.shape)


def dequantize(q, scale: float, shape) -> np.ndarray:
    """quantize.py:73-77: q[i] * scale (binary64), narrowed to binary32."""
    codes = np.asarray(q, dtype=np.int64)
    if codes.min(initial=0) < -128 or codes.max(initial=0) > 127:
        raise ValueError("dequantize: codes must fit in int8")
    cd = DeviceTensor.from_host(codes.astype(np.int8).reshape(-1))
    sd = DeviceTensor.from_host(np.array([scale], np.float64))
    return H.dequantize_tensor(cd, sd).numpy().reshape(list(shape))


def qlinear(x, qweight: QTensor, bias):
    """quantize.py:115-122: x.matmul(dequantize(W)).add(bias) -- the
    reference's weight-only path -- with the dequantize and the fp32 GEMM (+
    bias in its store) on the GPU.  Returns a DeviceTensor."""
    xd = to_device(x, "float32")
    w = qweight.dequantize()
    b = to_device(bias, "float32") if bias is not None else None
    return H.matmul(xd, w, b)


class QLinear:
    """quantize.py:125-144, built from an nn.Linear-like object (.weight
    [in, out], .bias [out]).

    mode="weight_only": the reference's semantics (per-tensor weight codes,
    dequantize, fp32 GEMM + bias).
    mode="int8": the input is quantized on the fly (act_granularity "tensor"
    or "row" = per token) and multiplied in int8 with int32 accumulation; the
    dequantize + bias is the GEMM's epilogue.  weight_granularity "tensor"
    or "col" (per output channel)."""

    def __init__(self, linear, mode: str = "weight_only", act_granularity: str = "tensor",
                 weight_granularity: str = "tensor"):
        if mode not in ("weight_only", "int8"):
            raise ValueError(f"QLinear: mode must be 'weight_only' or 'int8', got {mode!r}")
        if act_granularity not in ("tensor", "row"):
            raise ValueError(f"QLinear: act_granularity must be 'tensor' or 'row', got {act_granularity!r}")
        self.mode = mode
        self.act_granularity = act_granularity
        self.qweight = QTensor.from_weight(linear.weight, weight_granularity)
        b = getattr(linear, "bias", None)
        self.bias = to_device(b, "float32") if b is not None else None

    def named_parameters(self):
        """The reference Linear's names (nn.py:77-78): the weight as its int8
        QTensor, the bias as float32."""
        yield "weight", self.qweight
        if self.bias is not None:
            yield "bias", self.bias

    def set_parameter(self, name: str, value) -> None:
        """In-place load (kansaiml_amd.serialize): a float32 weight is
        quantized with this layer's weight granularity."""
        from .serialize import assign_in_place
        target = dict(self.named_parameters()).get(name)
        if target is None:
            raise KeyError(name)
        assign_in_place(name, target, value)

    def __call__(self, x):
        if _is_traced(x):
            return self._trace(x)
        if self.mode == "weight_only":
            return qlinear(x, self.qweight, self.bias)
        xd = to_device(x, "float32")
        if self.act_granularity == "row":
            return H.linear_i8(xd, self.qweight.codes, self.qweight.scales, self.bias)
        return H.linear_i8_tensor(xd, self.qweight.codes, self.qweight.scales, self.bias)

    def _trace(self, x):
        """Records this layer into x's graph.  x is a value of this package's
        tracer or of any tracer on the reference's schema (the reference's
        kansai.kir.TraceValue, kir.py:115-147).  int8 mode needs the tracer's
        quantize / int8_matmul / dequantize emitters (the reference's tracer
        has none until they are added to it).  weight_only mode under a
        tracer without them records what the reference's own QLinear records
        there: a matmul with the dequantized weight captured as a constant
        (kir.py:129-136)."""
        from .kir import TraceValue
        has_int8 = all(callable(getattr(x, m, None)) for m in ("quantize", "int8_matmul", "dequantize"))
        if self.mode == "weight_only":
            if isinstance(x, TraceValue):
                y = x.matmul(x._coerce(self.qweight).dequantize())
            else:
                y = x.matmul(self.qweight.dequantize())
        elif has_int8:
            y = x.quantize(self.act_granularity).int8_matmul(self.qweight).dequantize()
        else:
            raise TypeError(f"QLinear(mode='int8'): the tracer's {type(x).__name__} has no quantize / int8_matmul / "
                            "dequantize emitters; add them to it (kansaiml_amd.kir.TraceValue defines the three)")
        return y.add(self.bias) if self.bias is not None else y


def _is_traced(x) -> bool:
    """True for a tracer's value: it names a graph and a node instead of
    holding storage (the reference's TraceValue, kir.py:115-127)."""
    return hasattr(x, "graph") and hasattr(x, "node_id")
