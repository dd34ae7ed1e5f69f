"""Device-resident tensors for the HIP backend.

The reference's Tensor is host-only float32 (core/include/kansai/DType.hpp:6-8,
core/include/kansai/Tensor.hpp:52-53) and its Metal backend computes on that
host memory in place (backend/metal/src/MetalOps.mm:280-287).  A discrete
MI355X cannot, so this backend keeps its own device buffer type: contiguous
row-major, one of the KIR dtype strings ("float32", "int8", "int32",
"float64"), storage drawn from the library's hipMalloc-backed pool
(kh_alloc / kh_free).  Host arrays cross the boundary only through
from_host() / numpy().
"""

from __future__ import annotations

import ctypes
import math

import numpy as np

from . import _native as N

DTYPES = {"float32": np.float32, "int8": np.int8, "int32": np.int32, "float64": np.float64}


def _dtype_name(dt) -> str:
    dt = np.dtype(dt)
    for k, v in DTYPES.items():
        if np.dtype(v) == dt:
            return k
    raise TypeError(f"unsupported dtype {dt}")


class DeviceTensor:
    """A contiguous device buffer with a shape and a KIR dtype string."""

    # absmax_parts / row_parts: the per-tensor or per-row absmax partials the
    # producing kernel wrote alongside this tensor, when a fused graph asked
    # for them (kir.py).
    # _base: the tensor a view was cut from (kept alive as long as the view).
    __slots__ = ("ptr", "shape", "dtype", "nbytes", "_owned", "absmax_parts", "row_parts", "_base", "__weakref__")

    def __init__(self, shape, dtype: str = "float32"):
        if dtype not in DTYPES:
            raise TypeError(f"unsupported dtype {dtype!r}")
        self.shape = [int(s) for s in shape]
        if any(s < 0 for s in self.shape):
            raise ValueError(f"negative dimension in {self.shape}")
        self.dtype = dtype
        self.nbytes = math.prod(self.shape) * np.dtype(DTYPES[dtype]).itemsize
        self.ptr, self._owned, self.absmax_parts, self._base = None, False, None, None  # until kh_alloc succeeds
        self.row_parts = None
        p = ctypes.c_void_p()
        N.call("kh_alloc", max(self.nbytes, 1), ctypes.byref(p))
        self.ptr = p
        self._owned = True

    # -- construction -----------------------------------------------------
    @classmethod
    def empty(cls, shape, dtype: str = "float32") -> "DeviceTensor":
        return cls(shape, dtype)

    @classmethod
    def from_host(cls, arr, dtype: str | None = None) -> "DeviceTensor":
        """Uploads a numpy array (or anything with .tolist() and .shape,
        such as the reference's kansai.Tensor)."""
        a = as_host_array(arr, dtype)
        t = cls(list(a.shape), _dtype_name(a.dtype))
        if t.nbytes:
            N.call("kh_memcpy_h2d", t.ptr, ctypes.c_void_p(a.ctypes.data), t.nbytes)
        return t

    @classmethod
    def from_flat(cls, values, shape) -> "DeviceTensor":
        """A float32 tensor of `shape` from a flat sequence of numbers, as the
        reference's kansai.from_flat (core/src/Tensor.cpp:94-100): each value
        rounded to binary32, and RuntimeError when the length does not match
        the shape (checked before anything is allocated)."""
        shape = [int(s) for s in shape]
        flat = np.asarray(values, dtype=np.float64).reshape(-1)
        if any(s < 0 for s in shape) or flat.size != math.prod(shape):
            raise RuntimeError("from_flat: data length does not match shape")
        return cls.from_host(flat.astype(np.float32).reshape(shape))

    # -- access -------------------------------------------------------------
    def numel(self) -> int:
        return math.prod(self.shape)

    def numpy(self) -> np.ndarray:
        """Downloads (waits for queued work first)."""
        out = np.empty(self.shape, DTYPES[self.dtype])
        if self.nbytes:
            N.call("kh_memcpy_d2h", ctypes.c_void_p(out.ctypes.data), self.ptr, self.nbytes)
        return out

    def tolist(self):
        """Flat list, as the reference's Tensor.tolist() (python/bindings.cpp:44)."""
        return self.numpy().reshape(-1).tolist()

    @property
    def addr(self) -> int:
        return self.ptr.value or 0

    def reshape(self, shape) -> "DeviceTensor":
        """A view sharing this buffer (the view does not own it)."""
        shape = [int(s) for s in shape]
        if math.prod(shape) != self.numel():
            raise ValueError(f"reshape: cannot view {self.shape} as {shape}")
        v = object.__new__(DeviceTensor)
        v.ptr, v.shape, v.dtype, v.nbytes, v._owned = self.ptr, shape, self.dtype, self.nbytes, False
        v.absmax_parts, v.row_parts, v._base = None, None, self
        return v

    def view(self, offset: int, shape) -> "DeviceTensor":
        """A view of elements [offset, offset + prod(shape)) of this buffer,
        in the given shape (the view does not own the memory and keeps this
        tensor alive)."""
        shape = [int(s) for s in shape]
        n = math.prod(shape)
        if offset < 0 or offset + n > self.numel():
            raise ValueError(f"view: elements [{offset}, {offset + n}) outside a tensor of {self.numel()}")
        item = np.dtype(DTYPES[self.dtype]).itemsize
        v = object.__new__(DeviceTensor)
        v.ptr = ctypes.c_void_p(self.addr + offset * item)
        v.shape, v.dtype, v.nbytes, v._owned = shape, self.dtype, n * item, False
        v.absmax_parts, v.row_parts, v._base = None, None, self
        return v

    def copy_from(self, src) -> None:
        """Overwrites this buffer with `src` (a DeviceTensor of the same dtype
        and element count: a stream-ordered device copy; or a host array:
        a synchronous upload)."""
        if isinstance(src, DeviceTensor):
            if src.dtype != self.dtype or src.numel() != self.numel():
                raise ValueError(f"copy_from: {src} does not match {self}")
            if self.nbytes:
                N.call("kh_memcpy_d2d", self.ptr, src.ptr, self.nbytes)
            return
        a = as_host_array(src, self.dtype)
        if a.size != self.numel():
            raise ValueError(f"copy_from: {a.size} elements do not match {self}")
        if self.nbytes:
            N.call("kh_memcpy_h2d", self.ptr, ctypes.c_void_p(a.ctypes.data), self.nbytes)

    def release(self):
        """Returns the buffer to the pool (idempotent)."""
        if self._owned and self.ptr:
            self._owned = False
            try:
                N.lib().kh_free(self.ptr)
            except Exception:
                pass

    def __del__(self):
        self.release()

    def __repr__(self):
        return f"DeviceTensor({self.dtype}{self.shape})"


def as_host_array(x, dtype: str | None = None) -> np.ndarray:
    """numpy view/copy of a host tensor.  numpy arrays keep their dtype
    (it must be one of DTYPES); objects with .tolist() and .shape (the
    reference's Tensor) and Python sequences become float32, the
    reference's only dtype."""
    if isinstance(x, DeviceTensor):
        x = x.numpy()
    if isinstance(x, np.ndarray):
        a = x
    elif hasattr(x, "tolist") and hasattr(x, "shape"):
        a = np.array(x.tolist(), dtype=np.float32).reshape(list(x.shape))
    else:
        a = np.asarray(x, dtype=np.float32)
    if dtype is not None:
        a = a.astype(DTYPES[dtype], copy=False)
    _dtype_name(a.dtype)  # raises for unsupported dtypes
    return np.ascontiguousarray(a)


def to_device(x, dtype: str | None = None) -> DeviceTensor:
    return x if isinstance(x, DeviceTensor) else DeviceTensor.from_host(x, dtype)
