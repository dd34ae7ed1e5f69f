"""KIR on the HIP backend: the graph schema, a tracer for the int8 path, the
memory planner, and `run_hip`, the interpreter that dispatches a graph to the
gfx950 kernels.

The schema is the reference's (python/kansai/kir.py:40-75): single-output SSA
`Node`s (id, op, inputs, shape, dtype, attrs) kept in execution order in a
`Graph` with `inputs` (placeholder ids in argument order) and `output`.
`run_hip` is duck-typed over that schema, so it also runs graphs built by the
reference's own `kir.trace`.  It mirrors `run_metal`'s contract
(kir.py:1586-1836): `run_hip(graph, *args)` returns the output value, raises
RuntimeError when the device is missing, KeyError for an op it has no kernel
for.  There is no CPU fallback for any op.

New node kinds for the int8 path (the reference quantizes outside the graph
at trace time, kir.py:129-136):

  quantize      fp32 -> int8 codes + binary64 scales (attrs: granularity
                "tensor" | "row"), value: QTensor
  int8_matmul   QTensor [M,K] x packed-weight QTensor [K,N] -> int32 [M,N]
  dequantize    QTensor -> fp32 (quantize.py:73-77), or an int8_matmul
                accumulator -> fp32 (acc * sa * sb)
  int8_linear   fusion of int8_matmul -> dequantize [-> add(bias)] into one
                GEMM with the dequantize + bias epilogue
  matmul_bias   fusion of fp32 matmul -> add(bias) (bias in the GEMM store)
  fused_bias_relu  add(bias) -> relu (the reference's pattern, kir.py:581-600)

and, for a decoder block (config C4), fused forms of what the reference
composes from generic ops (nn.py:308-478): embedding (token + position
lookup on int32 ids), layer_norm, gelu, attention (the per-head
softmax(Q K^T / sqrt(d_k) + causal mask) V core of MultiHeadAttention on a
fused Q|K|V projection, heads merged in place).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import _native as N
from . import hip as H
from .device import DeviceTensor, as_host_array


# ---------------------------------------------------------------------------
# Graph / Node (kir.py:40-75)
# ---------------------------------------------------------------------------

@dataclass
class Node:
    id: int
    op: str
    inputs: list
    shape: list
    dtype: str = "float32"
    attrs: dict = field(default_factory=dict)

    def __repr__(self):
        ins = ", ".join(f"%{i}" for i in self.inputs)
        extra = {k: v for k, v in self.attrs.items() if k not in ("value", "_dev")}
        return f"%{self.id} = {self.op}({ins})  : {self.dtype}{self.shape}" + (f"  {extra}" if extra else "")


class Graph:
    def __init__(self):
        self.nodes: list = []
        self.inputs: list = []
        self.output = None

    def add(self, op: str, inputs: list, shape: list, dtype: str = "float32", **attrs) -> int:
        nid = len(self.nodes)
        self.nodes.append(Node(nid, op, list(inputs), list(shape), dtype, dict(attrs)))
        return nid

    def placeholder(self, shape: list, dtype: str = "float32") -> int:
        nid = self.add("placeholder", [], shape, dtype)
        self.inputs.append(nid)
        return nid

    def __repr__(self):
        return "\n".join([repr(n) for n in self.nodes] + [f"return %{self.output}"])


# ---------------------------------------------------------------------------
# Tracing (kir.py:115-407, the subset on the int8 / Linear path)
# ---------------------------------------------------------------------------

def _broadcast(a: list, b: list, what: str) -> list:
    """Right-aligned NumPy broadcasting (kir.py:85-112's rule)."""
    rank = max(len(a), len(b))
    a2 = [1] * (rank - len(a)) + list(a)
    b2 = [1] * (rank - len(b)) + list(b)
    out = []
    for x, y in zip(a2, b2):
        if x != y and x != 1 and y != 1:
            raise ValueError(f"{what}: shapes are not broadcast-compatible ({a} vs {b})")
        out.append(max(x, y))
    return out


class TraceValue:
    """A traced value: graph, node id, shape, dtype; no storage."""

    __slots__ = ("graph", "node_id", "shape", "dtype")

    def __init__(self, graph: Graph, node_id: int, shape: list, dtype: str = "float32"):
        self.graph, self.node_id, self.shape, self.dtype = graph, node_id, list(shape), dtype

    def _coerce(self, other) -> "TraceValue":
        if isinstance(other, TraceValue):
            return other
        from .quantize import QTensor
        if isinstance(other, QTensor):
            nid = self.graph.add("constant", [], other.shape, "int8", value=other)
            return TraceValue(self.graph, nid, other.shape, "int8")
        shape = list(getattr(other, "shape", np.shape(other)))
        nid = self.graph.add("constant", [], shape, value=other)
        return TraceValue(self.graph, nid, shape)

    def _emit(self, op, inputs, shape, dtype="float32", **attrs):
        nid = self.graph.add(op, [t.node_id for t in inputs], shape, dtype, **attrs)
        return TraceValue(self.graph, nid, shape, dtype)

    def add(self, other):
        other = self._coerce(other)
        return self._emit("add", [self, other], _broadcast(self.shape, other.shape, "add"))

    def relu(self):
        return self._emit("relu", [self], self.shape)

    def matmul(self, other):
        """Tensor::matmul's shape rules (kir.py:164-181): 2-D x 2-D, or the
        batched path with the leading axes broadcast.  run_hip runs an
        operand of any rank >= 2 against a 2-D right operand (a Linear's
        weight) as the 2-D GEMM of its rows; a batched right operand traces
        but has no HIP kernel."""
        other = self._coerce(other)
        if len(self.shape) < 2 or len(other.shape) < 2:
            raise ValueError(f"matmul: both operands must be at least 2D, got {self.shape} vs {other.shape}")
        if self.shape[-1] != other.shape[-2]:
            raise ValueError(f"matmul: incompatible shapes {self.shape} vs {other.shape}")
        batch = _broadcast(self.shape[:-2], other.shape[:-2], "matmul")
        return self._emit("matmul", [self, other], batch + [self.shape[-2], other.shape[-1]])

    def quantize(self, granularity: str = "tensor"):
        if granularity not in ("tensor", "row"):
            raise ValueError(f"quantize: granularity must be 'tensor' or 'row', got {granularity!r}")
        if granularity == "row" and len(self.shape) < 2:
            raise ValueError("quantize: per-row granularity needs a value of rank >= 2 (a row is the last axis)")
        return self._emit("quantize", [self], self.shape, "int8", granularity=granularity)

    def int8_matmul(self, other):
        other = self._coerce(other)
        if self.dtype != "int8" or other.dtype != "int8":
            raise ValueError("int8_matmul: both operands must be quantized (int8)")
        if len(self.shape) < 2 or len(other.shape) != 2 or self.shape[-1] != other.shape[0]:
            raise ValueError(f"int8_matmul: incompatible shapes {self.shape} vs {other.shape} (activations of "
                             "rank >= 2 against a 2-D weight)")
        return self._emit("int8_matmul", [self, other], self.shape[:-1] + [other.shape[1]], "int32")

    def dequantize(self):
        if self.dtype not in ("int8", "int32"):
            raise ValueError("dequantize: operand is not quantized")
        return self._emit("dequantize", [self], self.shape, "float32")

    # -- decoder-block pieces (config C4) -----------------------------------
    def embedding(self, tok, pos):
        """self: int32 ids [B, T]; tok [V, D]; pos [T, D] -> [B*T, D]."""
        if self.dtype != "int32" or len(self.shape) != 2:
            raise ValueError("embedding: expects int32 token ids [batch, seq]")
        tok, pos = self._coerce(tok), self._coerce(pos)
        if pos.shape[0] < self.shape[1] or tok.shape[1] != pos.shape[1]:
            raise ValueError(f"embedding: tables {tok.shape} / {pos.shape} do not fit ids {self.shape}")
        return self._emit("embedding", [self, tok, pos], [self.shape[0] * self.shape[1], tok.shape[1]],
                          seq=self.shape[1])

    def layer_norm(self, weight, bias, eps: float = 1e-5):
        weight, bias = self._coerce(weight), self._coerce(bias)
        if len(self.shape) < 2 or weight.shape != [self.shape[-1]] or bias.shape != [self.shape[-1]]:
            raise ValueError("layer_norm: expects [..., D] with weight and bias of shape [D]")
        return self._emit("layer_norm", [self, weight, bias], self.shape, eps=float(eps))

    def gelu(self):
        return self._emit("gelu", [self], self.shape)

    def attention(self, batch: int, seq: int, heads: int, causal: bool = True, mask=None):
        """self: fused Q|K|V projection [batch*seq, 3*D] -> [batch*seq, D];
        causal adds the mask that hides later keys, otherwise every query
        attends over all seq keys of its sequence; `mask` (optional) is an
        additive mask added to the scaled scores, broadcast to [batch, heads,
        seq, seq] (nn.py:421-422)."""
        if len(self.shape) != 2 or self.shape[0] != batch * seq or self.shape[1] % (3 * heads):
            raise ValueError(f"attention: {self.shape} is not [batch*seq, 3*D] for {heads} heads")
        ins = [self]
        if mask is not None:
            mask = self._coerce(mask)
            try:
                if mask.shape[-1] != seq or _broadcast(mask.shape, [batch, heads, seq, seq],
                                                       "attention(mask)") != [batch, heads, seq, seq]:
                    raise ValueError
            except (ValueError, IndexError):
                raise ValueError(f"attention: mask {mask.shape} does not broadcast to "
                                 f"[{batch}, {heads}, {seq}, {seq}]") from None
            ins.append(mask)
        return self._emit("attention", ins, [self.shape[0], self.shape[1] // 3], batch=batch, seq=seq,
                          heads=heads, causal=bool(causal))

    def causal_attention(self, batch: int, seq: int, heads: int):
        return self.attention(batch, seq, heads, causal=True)


def _example_dtype(x) -> str:
    dt = getattr(x, "dtype", None)
    if isinstance(dt, str):
        return dt
    if dt is not None and np.issubdtype(np.dtype(dt), np.integer):
        return "int32"
    return "float32"


def trace(fn, *example_inputs) -> Graph:
    """Records fn applied to placeholders shaped like example_inputs
    (kir.py:393-407).  Integer examples (token ids) become int32
    placeholders."""
    g = Graph()
    args = []
    for x in example_inputs:
        shape = list(getattr(x, "shape", np.shape(x)))
        dt = _example_dtype(x)
        args.append(TraceValue(g, g.placeholder(shape, dt), shape, dt))
    g.output = fn(*args).node_id
    return g


# ---------------------------------------------------------------------------
# Fusion pass
# ---------------------------------------------------------------------------

def _users(graph) -> dict:
    users = {n.id: [] for n in graph.nodes}
    for n in graph.nodes:
        for i in n.inputs:
            users[i].append(n.id)
    return users


def _is_bias(graph, by_id, x_id, b_id) -> bool:
    xs, bs = by_id[x_id].shape, by_id[b_id].shape
    return len(xs) >= 2 and len(bs) == 1 and xs[-1] == bs[0]


def quant_fusion(graph, producer_quant: bool | str = False, qload: bool = False) -> Graph:
    """Fuses, where the intermediate has no other user:
      int8_matmul -> dequantize [-> add(bias)] [-> gelu] [-> add(x, .)]
                                                 =>  int8_linear
      with qload=True, also the per-tensor quantize of its activation:
      quantize -> int8_matmul -> ...             =>  int8_linear (qload)
      and the per-row quantize of an attention output:
      attention -> quantize(row) -> int8_matmul  =>  attention (row_absmax) -> int8_linear (qload, rows)
      matmul -> add(bias)                        =>  matmul_bias
      add(bias) -> relu                          =>  fused_bias_relu
    and, with producer_quant=True (both) or "layer_norm" (the second only),
      ... the int8_linear chain -> quantize (per tensor) => int8_linear_quant
      layer_norm -> quantize (per tensor)        =>  layer_norm_quant
    and, with producer_quant=True or "layer_norm",
      layer_norm -> quantize (per row)           =>  layer_norm_quant_rows
      ... the int8_linear chain (no residual) -> quantize (per row)
                                                 =>  int8_linear_quant_rows
    int8_linear's attrs record what it absorbed: bias (bool), act ("gelu" or
    None), residual (bool; the residual operand comes last) and qload (bool:
    operand 0 is the fp32 activation, quantized per tensor inside the GEMM,
    kh_gemm_i8_qload, so its codes are never written).  The *_quant
    nodes produce the quantized tensor directly: their kernels run the
    producer twice (absmax, then codes) and never write the fp32 values.
    That saves the fp32 intermediate's memory; on MI355X it saves time for
    LayerNorm (two passes over its input cost less than writing the fp32
    values and reading them back) but not for the GEMM, whose VALU-bound
    epilogue (binary64 dequantize, GELU) the second pass repeats.
    layer_norm_quant_rows needs no second pass: each row's scale depends on
    that row only, so one pass stores codes and scales; int8_linear_quant_rows
    neither: a workgroup owns whole rows and keeps their values in registers
    (kh_gemm_i8_quant_rows), so it is faster than the two launches it
    replaces and fuses under "layer_norm" too.
    Then every int8_linear, layer_norm or attention whose
    output feeds a per-tensor quantize is marked absmax=True: its kernel
    writes the absmax partials that quantize needs, so the quantize reads
    its input once.
    The fused node takes the place of the last node of its pattern (every
    operand, e.g. a bias constant traced after the matmul, precedes it).
    Returns a new Graph; node order is preserved, ids are renumbered."""
    by_id = {n.id: n for n in graph.nodes}
    users = _users(graph)

    def only_user(nid):
        u = users[nid]
        return u[0] if len(u) == 1 and nid != graph.output else None

    def next_free(nid):
        """The only user of nid, unless an earlier pattern already took it
        (e.g. the add of two Linear outputs, claimed as the first one's
        residual add)."""
        u = only_user(nid)
        return u if u is not None and u not in fused and u not in absorbed else None

    # Phase 1: find patterns.  fused[last] = (op, [operand ids], attrs);
    # absorbed nodes are dropped.
    fused, absorbed = {}, set()

    if producer_quant not in (False, True, "layer_norm"):
        raise ValueError(f"producer_quant must be False, True or 'layer_norm', not {producer_quant!r}")

    def tensor_quantize(nid):
        """The per-tensor quantize that is the only user of nid, if any (and
        producer fusion is on for nid's kind of node)."""
        if producer_quant is not True and producer_quant != by_id[nid].op:
            return None
        q = only_user(nid)
        if q is not None and by_id[q].op == "quantize" and by_id[q].attrs.get("granularity", "tensor") == "tensor":
            return q
        return None

    def row_quantize(nid):
        """The per-row quantize that is the only user of nid, if any (and
        producer fusion is on)."""
        if producer_quant not in (True, "layer_norm"):
            return None
        q = only_user(nid)
        if q is not None and by_id[q].op == "quantize" and by_id[q].attrs.get("granularity") == "row":
            return q
        return None

    for n in graph.nodes:
        if n.id in absorbed or n.id in fused:
            continue
        if n.op == "int8_matmul":
            dq = next_free(n.id)
            if dq is not None and by_id[dq].op == "dequantize":
                chain, ins, attrs = [n.id, dq], list(n.inputs), {"bias": False, "act": None, "residual": False}
                qa = by_id[n.inputs[0]]
                if (qload and qa.op == "quantize" and qa.attrs.get("granularity", "tensor") == "tensor"
                        and only_user(qa.id) == n.id and qa.id not in fused and qa.shape[-1] <= _QLOAD_MAX_K):
                    chain.insert(0, qa.id)
                    ins[0] = qa.inputs[0]
                    attrs["qload"] = True
                elif (qload and qa.op == "quantize" and qa.attrs.get("granularity") == "row"
                        and only_user(qa.id) == n.id and qa.id not in fused
                        and by_id[qa.inputs[0]].op in _ROW_ABSMAX_PRODUCERS
                        and only_user(qa.inputs[0]) == qa.id):
                    # The per-row quantize of a producer that writes per-row
                    # partials, inside the GEMM (kh_gemm_i8_qload_rows).
                    chain.insert(0, qa.id)
                    ins[0] = qa.inputs[0]
                    attrs["qload"] = True
                    attrs["rows"] = True
                nxt = next_free(dq)
                if nxt is not None and by_id[nxt].op == "add":
                    a_in = by_id[nxt].inputs
                    if a_in[0] == dq and _is_bias(graph, by_id, dq, a_in[1]):
                        chain.append(nxt)
                        ins.append(a_in[1])
                        attrs["bias"] = True
                        nxt = next_free(nxt)
                if nxt is not None and by_id[nxt].op == "gelu":
                    chain.append(nxt)
                    attrs["act"] = "gelu"
                    nxt = next_free(nxt)
                if nxt is not None and by_id[nxt].op == "add":
                    a_in = by_id[nxt].inputs
                    other = a_in[1] if a_in[0] == chain[-1] else a_in[0]
                    if (len(a_in) == 2 and chain[-1] in a_in and other != chain[-1]
                            and list(by_id[other].shape) == list(by_id[chain[-1]].shape)):
                        chain.append(nxt)
                        ins.append(other)
                        attrs["residual"] = True
                last = chain[-1]
                q = tensor_quantize(last) if not attrs.get("qload") else None
                qr = row_quantize(last) if not attrs.get("qload") and not attrs["residual"] else None
                if q is not None:
                    absorbed.update(chain)
                    fused[q] = ("int8_linear_quant", ins, attrs)
                elif qr is not None:
                    absorbed.update(chain)
                    fused[qr] = ("int8_linear_quant_rows", ins, attrs)
                else:
                    absorbed.update(set(chain) - {last})
                    fused[last] = ("int8_linear", ins, attrs)
                continue
        if n.op == "layer_norm":
            q = tensor_quantize(n.id)
            if q is not None:
                absorbed.add(n.id)
                fused[q] = ("layer_norm_quant", list(n.inputs), dict(n.attrs))
                continue
            q = only_user(n.id)
            if (producer_quant in (True, "layer_norm") and q is not None and by_id[q].op == "quantize"
                    and by_id[q].attrs.get("granularity") == "row"):
                absorbed.add(n.id)
                fused[q] = ("layer_norm_quant_rows", list(n.inputs), dict(n.attrs))
                continue
        if n.op == "matmul":
            ad = only_user(n.id)
            if ad is not None and by_id[ad].op == "add":
                a_in = by_id[ad].inputs
                if a_in[0] == n.id and _is_bias(graph, by_id, n.id, a_in[1]):
                    absorbed.add(n.id)
                    fused[ad] = ("matmul_bias", list(n.inputs) + [a_in[1]], {})
                    continue
        if n.op == "add" and n.id not in fused and len(n.inputs) == 2 and _is_bias(graph, by_id, *n.inputs):
            r = only_user(n.id)
            if r is not None and by_id[r].op == "relu":
                absorbed.add(n.id)
                fused[r] = ("fused_bias_relu", list(n.inputs), {})

    # Phase 2: emit in order.
    out, remap = Graph(), {}
    for n in graph.nodes:
        if n.id in absorbed:
            continue
        if n.id in fused:
            op, ins, attrs = fused[n.id]
            dtype = n.dtype if op.endswith(("_quant", "_quant_rows")) else "float32"
            nid = out.add(op, [remap[i] for i in ins], n.shape, dtype, **attrs)
        else:
            nid = out.add(n.op, [remap[i] for i in n.inputs], n.shape, n.dtype, **n.attrs)
        remap[n.id] = nid
    out.inputs = [remap[i] for i in graph.inputs]
    out.output = remap[graph.output]

    # Phase 3: producers of a per-tensor quantize (or of a quantize fused
    # into its int8_linear) write its absmax partials; producers of a per-row
    # quantize fused into its int8_linear write per-row partials.
    for n in out.nodes:
        if n.op == "int8_linear" and n.attrs.get("rows"):
            out.nodes[n.inputs[0]].attrs["row_absmax"] = True
        elif ((n.op == "quantize" and n.attrs.get("granularity", "tensor") == "tensor")
                or (n.op == "int8_linear" and n.attrs.get("qload"))):
            src = out.nodes[n.inputs[0]]
            if src.op in _ABSMAX_PRODUCERS:
                src.attrs["absmax"] = True
    return out


_ABSMAX_PRODUCERS = ("int8_linear", "layer_norm", "attention")
# Producers that can write per-row partials (kh_attention_rows).
_ROW_ABSMAX_PRODUCERS = ("attention",)

# quant_fusion(qload=True) fuses a quantize into its GEMM only for activations
# of at most this many columns: on MI355X the fused kernel (one workgroup
# per CU streaming 64 rows of fp32) beat the two launches at K = 384 (18.5
# against 20.7 us at M = 16384, N = 384) but not at K = 1536 (49 against 48).
_QLOAD_MAX_K = 512


# ---------------------------------------------------------------------------
# Memory planning (kir.py:884-954)
# ---------------------------------------------------------------------------

@dataclass
class MemoryPlan:
    last_use: dict
    slot_of: dict
    num_slots: int
    num_computed_nodes: int


def plan_memory(graph) -> MemoryPlan:
    """Liveness (index of each value's last reader; the output lives to the
    end) and a greedy slot assignment in node order, reusing the most
    recently freed slot; placeholders and constants own no slot.  The same
    algorithm as the reference's plan_memory (kir.py:892-954)."""
    n = len(graph.nodes)
    last_use = {}
    for idx, node in enumerate(graph.nodes):
        for i in node.inputs:
            last_use[i] = idx
    if graph.output is not None:
        last_use[graph.output] = n
    slot_of, free, busy_until, next_slot = {}, [], {}, 0
    for idx, node in enumerate(graph.nodes):
        for sid, until in busy_until.items():
            if until <= idx and sid not in free:
                free.append(sid)
        if node.op in ("placeholder", "constant"):
            continue
        if free:
            sid = free.pop()
        else:
            sid, next_slot = next_slot, next_slot + 1
        slot_of[node.id] = sid
        busy_until[sid] = last_use.get(node.id, idx)
    return MemoryPlan(last_use, slot_of, next_slot, len(slot_of))


class DevicePool:
    """Handle on the library's hipMalloc-backed caching pool: the role of
    core.StoragePool (core/include/kansai/StoragePool.hpp:15-26) for device
    memory.  Every DeviceTensor draws from it; run_hip_planned returns each
    intermediate to it right after the value's last use."""

    def stats(self) -> dict:
        return N.pool_stats()

    def num_allocated(self) -> int:
        return N.pool_stats()["driver_allocs"]

    def trim(self):
        N.call("kh_pool_trim")


# ---------------------------------------------------------------------------
# Interpreter
# ---------------------------------------------------------------------------

@dataclass
class _Acc:
    """Value of an unfused int8_matmul: int32 accumulators + operand scales."""
    acc: DeviceTensor
    sa: DeviceTensor
    sb: DeviceTensor


def _constant(node):
    from .quantize import QTensor
    v = node.attrs["value"]
    if isinstance(v, (QTensor, DeviceTensor)):
        return v
    cached = node.attrs.get("_dev")
    if cached is None or cached[0] is not v:
        cached = (v, DeviceTensor.from_host(as_host_array(v, "float32")))
        node.attrs["_dev"] = cached  # weights stay resident across calls
    return cached[1]


def _dequantize(v):
    from .quantize import QTensor
    if isinstance(v, _Acc):
        return H.dequantize_acc(v.acc, v.sa, v.sb)
    if isinstance(v, QTensor):
        return v.dequantize()
    raise TypeError(f"dequantize: unsupported operand {type(v).__name__}")


def _add(a, b):
    if list(a.shape) == list(b.shape):
        return H.add(a, b)
    if len(a.shape) >= 2 and len(b.shape) == 1 and a.shape[-1] == b.shape[0]:
        return H.add_bias(a, b)  # [..., N] + [N]: the bias over every leading axis
    raise NotImplementedError(f"run_hip: add with broadcast {a.shape} + {b.shape} has no HIP kernel")


def _quantize_node(x, node):
    from .quantize import QTensor
    if node.attrs.get("granularity", "tensor") == "row":
        q, s = H.quantize_rows(x)
        return QTensor(q, s, list(x.shape), "row", packed=False)
    parts = getattr(x, "absmax_parts", None)
    q, s = H.quantize_tensor_parts(x, parts) if parts is not None else H.quantize_tensor(x)
    return QTensor(q, s, list(x.shape), "tensor", packed=False)


def _with_parts(out, parts):
    """Attaches the absmax partials a producer wrote to its output tensor
    (read by the next per-tensor quantize, released with the tensor)."""
    if parts is not None:
        out.absmax_parts = parts
    return out


def _int8_operands(qa, qb, what):
    from .quantize import QTensor
    if not (isinstance(qa, QTensor) and isinstance(qb, QTensor)):
        raise TypeError(f"{what}: operands must be quantized")
    if qa.packed or not qb.packed:
        raise TypeError(f"{what}: expects quantized activations [M,K] and a packed weight [K,N]")
    return qa.codes.reshape(qa.shape), qb.codes, qa.scales, qb.scales


def _exec(node, vals):
    op = node.op
    ins = [vals[i] for i in node.inputs]
    if op == "matmul":
        return H.matmul(*ins)
    if op == "matmul_bias":
        return H.matmul(ins[0], ins[1], ins[2])
    if op == "add":
        return _add(*ins)
    if op == "relu":
        return H.relu(ins[0])
    if op == "fused_bias_relu":
        return H.add_bias(ins[0], ins[1], relu=True)
    if op == "quantize":
        return _quantize_node(ins[0], node)
    if op == "dequantize":
        return _dequantize(ins[0])
    if op == "int8_matmul":
        a, b, sa, sb = _int8_operands(ins[0], ins[1], "int8_matmul")
        _, acc = H.gemm_i8(a, b, want_out=False, want_acc=True)
        return _Acc(acc, sa, sb)
    if op == "int8_linear" and node.attrs.get("qload"):
        from .quantize import QTensor
        x, w = ins[0], ins[1]
        if not isinstance(w, QTensor) or not w.packed:
            raise TypeError("int8_linear: expects a packed quantized weight [K,N]")
        at = node.attrs
        bias = ins[2] if at.get("bias") else None
        residual = ins[-1] if at.get("residual") else None
        if at.get("rows"):
            rp = getattr(x, "row_parts", None)
            if rp is not None:
                return H.gemm_i8_qload_rows(x, rp, w.codes, w.scales, bias, act=at.get("act"), residual=residual)
            # No producer partials: the per-row quantize, then the GEMM.
            q, s = H.quantize_rows(x)
            out, _ = H.gemm_i8_fused(q, w.codes, s, w.scales, bias, act=at.get("act"), residual=residual)
            q.release()
            s.release()
            return out
        parts = getattr(x, "absmax_parts", None)
        if parts is None and not at.get("act") and residual is None and not at.get("absmax"):
            # No producer partials and a plain epilogue: kh_linear_i8_tensor
            # (one launch for small activations, C1's shape).
            return H.linear_i8_tensor(x, w.codes, w.scales, bias)
        if parts is None:
            q, s = H.quantize_tensor(x)
            out, oparts = H.gemm_i8_fused(q, w.codes, s, w.scales, bias, act=at.get("act"), residual=residual,
                                          absmax=bool(at.get("absmax")))
            q.release()
            s.release()
        else:
            out, oparts = H.gemm_i8_qload(x, parts, w.codes, w.scales, bias, act=at.get("act"), residual=residual,
                                          absmax=bool(at.get("absmax")))
        return _with_parts(out, oparts)
    if op == "int8_linear":
        a, b, sa, sb = _int8_operands(ins[0], ins[1], "int8_linear")
        at = node.attrs
        has_bias = at.get("bias", len(ins) > 2 and not at.get("residual"))
        bias = ins[2] if has_bias else None
        residual = ins[-1] if at.get("residual") else None
        if at.get("act") or residual is not None or at.get("absmax"):
            out, parts = H.gemm_i8_fused(a, b, sa, sb, bias, act=at.get("act"), residual=residual,
                                         absmax=bool(at.get("absmax")))
            return _with_parts(out, parts)
        out, _ = H.gemm_i8(a, b, sa, sb, bias)
        return out
    if op == "int8_linear_quant":
        from .quantize import QTensor
        a, b, sa, sb = _int8_operands(ins[0], ins[1], "int8_linear_quant")
        at = node.attrs
        bias = ins[2] if at.get("bias") else None
        residual = ins[-1] if at.get("residual") else None
        q, s = H.gemm_i8_quant(a, b, sa, sb, bias, act=at.get("act"), residual=residual)
        return QTensor(q, s, list(node.shape), "tensor", packed=False)
    if op == "int8_linear_quant_rows":
        from .quantize import QTensor
        a, b, sa, sb = _int8_operands(ins[0], ins[1], "int8_linear_quant_rows")
        bias = ins[2] if node.attrs.get("bias") else None
        q, s = H.gemm_i8_quant_rows(a, b, sa, sb, bias, act=node.attrs.get("act"))
        return QTensor(q, s, list(node.shape), "row", packed=False)
    if op == "layer_norm_quant":
        from .quantize import QTensor
        x, w, b = ins
        q, s = H.layer_norm_quant(x, w, b, node.attrs.get("eps", 1e-5))
        return QTensor(q, s, list(node.shape), "tensor", packed=False)
    if op == "layer_norm_quant_rows":
        from .quantize import QTensor
        x, w, b = ins
        q, s = H.layer_norm_quant_rows(x, w, b, node.attrs.get("eps", 1e-5))
        return QTensor(q, s, list(node.shape), "row", packed=False)
    if op == "embedding":
        ids, tok, pos = ins
        rows, D = node.shape
        out = DeviceTensor([rows, D], "float32")
        N.call("kh_embedding", ids.ptr, rows, node.attrs["seq"], tok.ptr, tok.shape[0], pos.ptr, D, out.ptr)
        return out
    if op == "layer_norm":
        x, w, b = ins
        out, parts = H.layer_norm(x, w, b, node.attrs.get("eps", 1e-5), absmax=bool(node.attrs.get("absmax")))
        return _with_parts(out, parts)
    if op == "gelu":
        out = DeviceTensor(ins[0].shape, "float32")
        N.call("kh_gelu", ins[0].ptr, out.ptr, ins[0].numel())
        return out
    if op == "attention":
        mask = ins[1] if len(ins) > 1 else None
        if node.attrs.get("row_absmax"):
            out, rp = H.attention_rows(ins[0], node.attrs["batch"], node.attrs["seq"], node.attrs["heads"],
                                       node.shape[1], causal=node.attrs["causal"], mask=mask)
            out.row_parts = rp
            return out
        out, parts = H.attention(ins[0], node.attrs["batch"], node.attrs["seq"], node.attrs["heads"], node.shape[1],
                                 causal=node.attrs["causal"], absmax=bool(node.attrs.get("absmax")), mask=mask)
        return _with_parts(out, parts)
    if op == "tuple":
        return tuple(ins)
    raise KeyError(op)


def _release(v):
    from .quantize import QTensor
    if isinstance(v, DeviceTensor):
        for parts in (getattr(v, "absmax_parts", None), getattr(v, "row_parts", None)):
            if parts is not None:
                parts.release()
        v.release()
    elif isinstance(v, _Acc):
        v.acc.release()
    elif isinstance(v, QTensor) and v.owned:
        v.codes.release()
        v.scales.release()


def _to_host(v):
    if isinstance(v, DeviceTensor):
        return v.numpy()
    if isinstance(v, tuple):
        return tuple(_to_host(x) for x in v)
    return v


def _run(graph, args, plan, to_host, observe=None, capturing=False):
    if not N.available():
        raise RuntimeError("run_hip: no gfx950 (MI355X) device available on this system")
    by_id = {n.id: n for n in graph.nodes}
    vals = {}
    for nid, a in zip(graph.inputs, args):
        dt = by_id[nid].dtype if by_id[nid].dtype in ("float32", "int32") else "float32"
        vals[nid] = a if isinstance(a, DeviceTensor) else DeviceTensor.from_host(as_host_array(a, dt))
    external = set(graph.inputs)
    for idx, node in enumerate(graph.nodes):
        if node.op == "placeholder":
            continue
        if node.op == "constant":
            vals[node.id] = _constant(node)
            if observe is not None:
                observe(node, vals[node.id])
            continue
        vals[node.id] = _exec(node, vals)
        if observe is not None:
            observe(node, vals[node.id])
        if plan is not None:
            for i in node.inputs:
                src = by_id[i]
                if src.op in ("placeholder", "constant") or i in external:
                    continue
                if plan.last_use.get(i) == idx and i in vals:
                    _release(vals.pop(i))
    out = vals[graph.output]
    if capturing:
        return out
    N.synchronize()  # reports a non-finite quantizer input as ValueError
    return _to_host(out) if to_host else out


def run_hip(graph, *args, to_host: bool = True, observe=None):
    """Runs `graph` on the GPU.  Host inputs (numpy arrays, or anything with
    .tolist() and .shape such as the reference's Tensor) are uploaded;
    DeviceTensors are used in place.  Returns the output as a numpy array
    (or a DeviceTensor with to_host=False).

    observe(node, value), if given, is called after every constant and every
    executed node with its device value (DeviceTensor, QTensor or the
    accumulator holder), before any release: per-node inspection, like the
    reference's trace printing of node results."""
    return _run(graph, args, None, to_host, observe)


def run_hip_planned(graph, plan: MemoryPlan, pool: DevicePool | None, *args, to_host: bool = True, observe=None):
    """run_planned's contract (kir.py:957-1068) on the device: every
    intermediate is returned to the device pool right after its last use, so
    repeated runs of the graph reuse the same device buffers and never call
    hipMalloc after the first run.  Placeholders and constants are never
    released; the output's ownership passes to the caller.  `observe` is
    run_hip's per-node hook."""
    return _run(graph, args, plan, to_host, observe)


class HipGraph:
    """A planned run recorded once as a HIP graph and replayed with one host
    call per run (hipGraphLaunch), where the reference re-interprets its
    cached traced graph on every call (kir.py:536-555, 957-1068): the same
    kernels on the same buffers, without the per-node Python dispatch.

    The graph owns private input buffers (filled from the capture's
    arguments) and writes one output buffer: launch(*args) copies its
    arguments into the input buffers on the library stream, replays, and
    returns the output -- a host array, or with to_host=False the output
    DeviceTensor itself, which the next launch overwrites.  The graph reads
    the constants' device copies (the model's weights) in place, so it is
    only valid while they are.  close() (or garbage collection) destroys the
    graph and returns its buffers to the pool.  Errors the kernels record
    (non-finite quantizer input, token id out of range) surface on the next
    synchronize, as for an eager run."""

    def __init__(self, graph, plan: MemoryPlan, *args):
        if not N.available():
            raise RuntimeError("HipGraph: no gfx950 (MI355X) device available on this system")
        by_id = {n.id: n for n in graph.nodes}
        self._dtypes = [by_id[nid].dtype if by_id[nid].dtype in ("float32", "int32") else "float32"
                        for nid in graph.inputs]
        self.inputs = []
        for a, dt in zip(args, self._dtypes):
            if isinstance(a, DeviceTensor):
                buf = DeviceTensor(a.shape, a.dtype)
                N.call("kh_memcpy_d2d", buf.ptr, a.ptr, a.nbytes)
            else:
                buf = DeviceTensor.from_host(as_host_array(a, dt))
            self.inputs.append(buf)
        self.handle = None
        self._graph = graph  # holds the constants' device buffers the nodes read
        # One eager run first: it uploads the constants, sizes the scratch
        # area and warms the pool, none of which can happen inside a capture.
        _release(_run(graph, self.inputs, plan, to_host=False))
        N.call("kh_graph_capture_begin")
        try:
            out = _run(graph, self.inputs, plan, to_host=False, capturing=True)
        except BaseException:
            N.lib().kh_graph_capture_end(None)
            raise
        h = ctypes.c_void_p()
        N.call("kh_graph_capture_end", ctypes.byref(h))
        self.handle = h
        self.output = out

    def launch(self, *args, to_host: bool = True):
        if self.handle is None:
            raise RuntimeError("HipGraph: the graph has been closed")
        if len(args) != len(self.inputs):
            raise ValueError(f"HipGraph: expected {len(self.inputs)} inputs, got {len(args)}")
        for buf, a, dt in zip(self.inputs, args, self._dtypes):
            if a is buf:
                continue
            if isinstance(a, DeviceTensor):
                if tuple(a.shape) != tuple(buf.shape) or a.dtype != buf.dtype:
                    raise ValueError(f"HipGraph: input {a.dtype}{list(a.shape)} does not match the captured "
                                     f"{buf.dtype}{list(buf.shape)}")
                N.call("kh_memcpy_d2d", buf.ptr, a.ptr, buf.nbytes)
            else:
                arr = np.ascontiguousarray(as_host_array(a, dt))
                if tuple(arr.shape) != tuple(buf.shape):
                    raise ValueError(f"HipGraph: input shape {list(arr.shape)} does not match the captured "
                                     f"{list(buf.shape)}")
                N.call("kh_memcpy_h2d", buf.ptr, arr.ctypes.data, buf.nbytes)
        N.call("kh_graph_launch", self.handle)
        if not to_host:
            return self.output
        N.synchronize()
        return _to_host(self.output)

    __call__ = launch

    def close(self):
        if self.handle is not None:
            h, self.handle = self.handle, None
            N.call("kh_graph_destroy", h)
            _release(self.output)
            for buf in self.inputs:
                buf.release()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def capture_hip_planned(graph, plan: MemoryPlan, *args) -> HipGraph:
    """run_hip_planned's work recorded as a HipGraph (see there)."""
    return HipGraph(graph, plan, *args)


def jit(fn):
    """Traces fn on first call per input-shape key, fuses, and replays the
    graph through run_hip (kir.py:536-555's cache, on the HIP backend)."""
    cache: dict = {}

    def wrapped(*args):
        key = tuple(tuple(getattr(a, "shape", np.shape(a))) for a in args)
        g = cache.get(key)
        if g is None:
            g = quant_fusion(trace(fn, *args))
            cache[key] = g
        return run_hip(g, *args)

    wrapped.trace = lambda *args: trace(fn, *args)
    return wrapped
