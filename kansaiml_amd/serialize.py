"""Parameter checkpoints in the reference's KAN1 format, extended with int8
weights that load straight to the device.

The reference (python/kansai/serialize.py:17-30, 117-199) writes

    bytes 0-3    magic b"KAN1"
    bytes 4-11   header length, uint64 little-endian
    header       UTF-8 JSON {name: {"dtype", "shape", "offset", "nbytes"}}
    data         every tensor's bytes, concatenated; tensor `name` is
                 data[offset : offset + nbytes]

with float32 tensors only, named by Module.named_parameters()
(python/kansai/nn.py:19-39).  save() here writes float32 parameters byte for
byte as the reference does (same header key order, same json.dumps
separators, no padding), so a checkpoint of float32 parameters from either
side loads on the other.  load() keeps the reference's checks and messages
(bad magic, missing and unexpected names, shape mismatch, a byte count that
does not match the shape, a range past the end of the file).

The extension, for a QTensor parameter (int8 codes + binary64 scales):

    name: {"dtype": "int8", "shape": [in, out], "offset": o, "nbytes": in*out,
           "layout": "packed" | "row_major", "granularity": "tensor" | "col" | "row",
           "scales": {"dtype": "float64", "shape": [n], "offset": o2, "nbytes": 8*n}}

"packed" codes are stored [out, in] (K-contiguous), the layout the int8 GEMM
reads, so loading is one host-to-device copy of the file's bytes with no
requantization; the number of scales is 1, `out` or `in` for "tensor",
"col" and "row".  The reference's own loader rejects such an entry (its byte
count does not match float32), so an int8 checkpoint can never be misread
there as float32.

Loading memory-maps the file and uploads each tensor from the mapping.
Nothing in a checkpoint is executed: the header is parsed as JSON and the
payload is read as raw numbers.

Assignment: a module that defines set_parameter(name, value) receives each
loaded value and stores it itself (the char-LM copies into its existing
device buffers, so graphs traced against them stay valid); otherwise the
value is assigned by attribute path, as the reference's _set_by_path
(serialize.py:89-114).  Values: numpy float32 arrays, or QTensors on the
device for int8 entries.  A float32 entry loaded where the module holds a
QTensor is quantized by the module's set_parameter (the reference's
QLinear quantizes at construction, quantize.py:125-144); an int8 entry
loaded where the module holds float32 is dequantized on the device with
the reference's dequantize (quantize.py:73-77).
"""

from __future__ import annotations

import json
import math
import mmap
import struct

import numpy as np

from .device import DeviceTensor, as_host_array

_MAGIC = b"KAN1"
_ITEMSIZE = {"float32": 4, "int8": 1, "float64": 8}
_GRANULARITIES = ("tensor", "col", "row")
_LAYOUTS = ("packed", "row_major")


def _is_qtensor(v) -> bool:
    from .quantize import QTensor
    return isinstance(v, QTensor)


def _shape_of(v) -> list:
    return [int(s) for s in getattr(v, "shape", np.shape(v))]


def _set_by_path(root, path: str, value) -> None:
    """serialize.py:89-114: walk the dotted name (attribute names, list
    indices) and assign the last attribute."""
    parts = path.split(".")
    obj = root
    for part in parts[:-1]:
        obj = obj[int(part)] if isinstance(obj, (list, tuple)) else getattr(obj, part)
    setattr(obj, parts[-1], value)


def _entry_bytes(name: str, value):
    """(header entry, list of byte chunks) for one parameter."""
    if _is_qtensor(value):
        codes = value.codes.numpy()
        scales = np.ascontiguousarray(value.scales.numpy(), dtype="<f8")
        want = _scale_count(value.granularity, value.shape)
        if codes.size != math.prod(value.shape) or scales.size != want:
            raise ValueError(f"save: {name!r} is an inconsistent QTensor (codes {codes.size}, scales {scales.size})")
        meta = {"dtype": "int8", "shape": list(value.shape), "offset": 0, "nbytes": int(codes.nbytes),
                "layout": "packed" if value.packed else "row_major", "granularity": value.granularity,
                "scales": {"dtype": "float64", "shape": [int(scales.size)], "offset": 0,
                           "nbytes": int(scales.nbytes)}}
        return meta, [codes.tobytes(), scales.tobytes()]
    arr = as_host_array(value, "float32")
    data = np.ascontiguousarray(arr, dtype="<f4").tobytes()
    return {"dtype": "float32", "shape": _shape_of(arr), "offset": 0, "nbytes": len(data)}, [data]


def _scale_count(granularity: str, shape) -> int:
    if granularity == "tensor":
        return 1
    if len(shape) != 2:
        raise ValueError(f"granularity {granularity!r} needs a 2-D shape, got {list(shape)}")
    return int(shape[1]) if granularity == "col" else int(shape[0])


def save(module, path: str) -> None:
    """Writes every parameter of `module` (module.named_parameters()) to
    `path`: float32 values as the reference writes them, QTensors as int8
    entries."""
    header = {}
    chunks = []
    offset = 0
    for name, value in module.named_parameters():
        meta, data = _entry_bytes(name, value)
        meta["offset"] = offset
        offset += len(data[0])
        if "scales" in meta:
            meta["scales"]["offset"] = offset
            offset += len(data[1])
        header[name] = meta
        chunks.extend(data)
    header_bytes = json.dumps(header).encode("utf-8")
    with open(path, "wb") as f:
        f.write(_MAGIC)
        f.write(struct.pack("<Q", len(header_bytes)))
        f.write(header_bytes)
        for c in chunks:
            f.write(c)


class _Checkpoint:
    """A parsed, memory-mapped KAN1 file."""

    def __init__(self, path: str):
        self.path = path
        with open(path, "rb") as f:
            magic = f.read(4)
            if magic != _MAGIC:
                raise ValueError(f"{path}: not a Kansai checkpoint (expected magic {_MAGIC!r}, got {magic!r})")
            raw_len = f.read(8)
            if len(raw_len) != 8:
                raise ValueError(f"{path}: truncated header length")
            header_len = struct.unpack("<Q", raw_len)[0]
            header_raw = f.read(header_len)
            if len(header_raw) != header_len:
                raise ValueError(f"{path}: header runs past the end of the file")
            try:
                header = json.loads(header_raw.decode("utf-8"))
            except (UnicodeDecodeError, json.JSONDecodeError) as e:
                raise ValueError(f"{path}: unparseable header ({e})") from None
            if not isinstance(header, dict) or not all(isinstance(v, dict) for v in header.values()):
                raise ValueError(f"{path}: malformed header (expected an object of per-tensor objects)")
            self.header = header
            self.data_start = 12 + header_len
            f.seek(0, 2)
            self.size = f.tell()
            self._mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) if self.size else None

    def close(self):
        """Unmaps the file; while arrays returned by tensor() are still
        alive the mapping stays until the last of them is dropped."""
        if self._mm is not None:
            try:
                self._mm.close()
            except BufferError:
                pass
            self._mm = None

    def _array(self, name: str, meta: dict, dtype: str, count: int, what: str) -> np.ndarray:
        for key in ("offset", "nbytes"):
            if not isinstance(meta.get(key), int) or meta[key] < 0:
                raise ValueError(f"{self.path}: {name!r} has a malformed {what}{key}")
        expected = count * _ITEMSIZE[dtype]
        if meta["nbytes"] != expected:
            raise ValueError(
                f"{self.path}: {name!r} has an inconsistent header -- its {what}shape implies "
                f"{expected} bytes but the header declares {meta['nbytes']}")
        start = self.data_start + meta["offset"]
        have = max(0, min(self.size - start, meta["nbytes"]))
        if have != meta["nbytes"]:
            raise ValueError(
                f"{self.path}: {name!r}'s declared {what}byte range runs past the end of the file "
                f"(wanted {meta['nbytes']} bytes at offset {meta['offset']}, file has {have} there)")
        if count == 0:
            return np.zeros(0, {"float32": "<f4", "int8": np.int8, "float64": "<f8"}[dtype])
        np_dtype = {"float32": "<f4", "int8": np.int8, "float64": "<f8"}[dtype]
        return np.frombuffer(self._mm, dtype=np_dtype, count=count, offset=start)

    def tensor(self, name: str, want_shape):
        """The value of entry `name`: a float32 numpy array, or a QTensor on
        the device for an int8 entry (checked against want_shape first)."""
        meta = self.header[name]
        shape = meta.get("shape")
        if not isinstance(shape, list) or not all(isinstance(d, int) and d >= 0 for d in shape):
            raise ValueError(f"{self.path}: {name!r} has a malformed shape {shape!r}")
        if want_shape is not None and list(want_shape) != shape:
            raise ValueError(
                f"{self.path}: {name!r} shape mismatch -- model has {list(want_shape)}, checkpoint has {shape}")
        n = math.prod(shape)
        dtype = meta.get("dtype", "float32")
        if dtype == "float32":
            return self._array(name, meta, "float32", n, "").reshape(shape)
        if dtype != "int8":
            raise ValueError(f"{self.path}: {name!r} has unsupported dtype {dtype!r}")
        layout, gran = meta.get("layout"), meta.get("granularity")
        if layout not in _LAYOUTS or gran not in _GRANULARITIES:
            raise ValueError(f"{self.path}: {name!r} int8 entry has layout {layout!r} / granularity {gran!r}")
        if layout == "packed" and (len(shape) != 2 or gran == "row"):
            raise ValueError(f"{self.path}: {name!r} packed codes need a 2-D [in, out] shape and "
                             f"'tensor' or 'col' scales")
        sm = meta.get("scales")
        if not isinstance(sm, dict) or sm.get("dtype") != "float64":
            raise ValueError(f"{self.path}: {name!r} int8 entry has no float64 scales")
        ns = _scale_count(gran, shape)
        if sm.get("shape") != [ns]:
            raise ValueError(f"{self.path}: {name!r} needs {ns} scales for granularity {gran!r}, "
                             f"header declares {sm.get('shape')!r}")
        codes = self._array(name, meta, "int8", n, "")
        scales = self._array(name, sm, "float64", ns, "scales ")
        if n and int(codes.min()) < -127:
            raise ValueError(f"{self.path}: {name!r} holds code -128, outside the symmetric range [-127, 127]")
        if not (np.all(np.isfinite(scales)) and np.all(scales > 0)):
            raise ValueError(f"{self.path}: {name!r} has a non-finite or non-positive scale")
        from .quantize import QTensor
        stored = [shape[1], shape[0]] if layout == "packed" else shape
        return QTensor(DeviceTensor.from_host(codes.reshape(stored)), DeviceTensor.from_host(scales), shape, gran,
                       packed=(layout == "packed"))


def load(module, path: str) -> None:
    """Loads parameters from `path` into `module` in place, by name
    (serialize.py:146-199): every name and shape must match in both
    directions."""
    ck = _Checkpoint(path)
    try:
        _load_into(module, ck, path)
    finally:
        ck.close()


def _load_into(module, ck: _Checkpoint, path: str) -> None:
    named = dict(module.named_parameters())
    missing = sorted(set(named) - set(ck.header))
    unexpected = sorted(set(ck.header) - set(named))
    if missing:
        raise ValueError(f"{path}: checkpoint is missing parameter(s) the model expects: {missing}")
    if unexpected:
        raise ValueError(f"{path}: checkpoint has parameter(s) the model doesn't expect: {unexpected}")
    # Every entry is checked before anything is assigned: a bad file
    # leaves the module as it was.
    values = {name: ck.tensor(name, _shape_of(current)) for name, current in named.items()}
    setter = getattr(module, "set_parameter", None)
    for name, current in named.items():
        value = values[name]
        if setter is not None:
            setter(name, value)
            continue
        if _is_qtensor(value) and not _is_qtensor(current):
            value = value.dequantize()
            value = value if isinstance(current, DeviceTensor) else value.numpy()
        elif not _is_qtensor(value):
            if _is_qtensor(current):
                from .quantize import QTensor
                value = (QTensor.from_weight(value, current.granularity) if current.packed
                         else QTensor.from_tensor(value, current.granularity))
            elif isinstance(current, DeviceTensor):
                value = DeviceTensor.from_host(value)
            else:
                value = np.array(value, dtype=np.float32)
        _set_by_path(module, name, value)


def assign_in_place(name: str, target, value) -> None:
    """Copies a loaded value into an existing device parameter: `target` a
    QTensor (codes and scales overwritten; a float32 value is quantized with
    the target's granularity and layout first) or a DeviceTensor (an int8
    value is dequantized first).  The target keeps its identity, so graphs
    traced with it as a constant see the new values."""
    from .quantize import QTensor
    if isinstance(target, QTensor):
        if not isinstance(value, QTensor):
            value = (QTensor.from_weight(value, target.granularity) if target.packed
                     else QTensor.from_tensor(value, target.granularity))
        if (value.granularity, value.packed, list(value.shape)) != (target.granularity, target.packed,
                                                                     list(target.shape)):
            raise ValueError(
                f"{name!r}: checkpoint holds {value.granularity!r} int8 codes (packed={value.packed}) of "
                f"shape {value.shape}; the model expects {target.granularity!r} (packed={target.packed}) "
                f"of shape {target.shape}")
        target.codes.copy_from(value.codes)
        target.scales.copy_from(value.scales)
        return
    if isinstance(target, DeviceTensor):
        if isinstance(value, QTensor):
            value = value.dequantize()
        if _shape_of(value) != target.shape:
            raise ValueError(f"{name!r} shape mismatch -- model has {target.shape}, checkpoint has {_shape_of(value)}")
        target.copy_from(value)
        return
    raise TypeError(f"{name!r}: cannot assign into {type(target).__name__}")


def read_header(path: str) -> dict:
    """The parsed JSON header of a checkpoint (for inspection)."""
    ck = _Checkpoint(path)
    try:
        return ck.header
    finally:
        ck.close()
