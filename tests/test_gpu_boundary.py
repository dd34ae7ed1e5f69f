"""The drop-in boundary: graphs built in the reference's own conventions run
through run_hip unchanged.

The graphs here are not built with this package's tracer.  A test-local
schema and tracer follow the reference's (python/kansai/kir.py:40-75 Node /
Graph; :115-147 TraceValue._coerce / add / matmul; :393-407 trace): constants
are float32-typed nodes whose `value` is the host object itself, and that
object exposes only `.shape` and a flat `.tolist()` (the reference's
kansai.Tensor, python/bindings.cpp:44).  The add(bias) -> relu pair is
rewritten into the reference's `fused_bias_relu` node (inputs [x, bias], no
attrs; kir.py:581-600, 630-735).  The tracer value carries the three int8
emitters a maintainer adds to the reference's TraceValue (quantize,
int8_matmul, dequantize); a second tracer without them stands for the
unpatched reference.

Every result is checked against the oracle: codes, int32 accumulators and
the dequantize epilogue bit for bit, the fp32 matmul within a K-scaled
rounding bound of the C restatement of the reference's i-k-j loop."""

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


# ---------------------------------------------------------------------------
# The reference's conventions, restated for the test
# ---------------------------------------------------------------------------

class RefTensor:
    """What a graph constant holds in the reference: a kansai.Tensor, seen
    through its binding as .shape and a flat .tolist() only."""

    def __init__(self, a):
        self._a = np.ascontiguousarray(a, np.float32)

    @property
    def shape(self):
        return list(self._a.shape)

    def tolist(self):
        return self._a.reshape(-1).tolist()


class RefNode:
    def __init__(self, id, op, inputs, shape, dtype="float32", attrs=None):
        self.id, self.op, self.inputs, self.shape, self.dtype = id, op, list(inputs), list(shape), dtype
        self.attrs = dict(attrs or {})


class RefGraph:
    def __init__(self):
        self.nodes, self.inputs, self.output = [], [], None

    def add(self, op, inputs, shape, dtype="float32", **attrs):
        self.nodes.append(RefNode(len(self.nodes), op, inputs, shape, dtype, attrs))
        return len(self.nodes) - 1

    def placeholder(self, shape, dtype="float32"):
        nid = self.add("placeholder", [], shape, dtype)
        self.inputs.append(nid)
        return nid


class RefValue:
    """The reference TraceValue's surface on the Linear path: a non-traced
    operand becomes a float32 "constant" node holding the object."""

    def __init__(self, graph, node_id, shape, dtype="float32"):
        self.graph, self.node_id, self.shape, self.dtype = graph, node_id, list(shape), dtype

    def _coerce(self, other):
        if isinstance(other, RefValue):
            return other
        nid = self.graph.add("constant", [], list(other.shape), value=other)
        return type(self)(self.graph, nid, list(other.shape))

    def _op(self, op, inputs, shape, dtype="float32", **attrs):
        nid = self.graph.add(op, [t.node_id for t in inputs], shape, dtype, **attrs)
        return type(self)(self.graph, nid, shape, dtype)

    def add(self, other):
        other = self._coerce(other)
        shape = self.shape if len(self.shape) >= len(other.shape) else other.shape
        return self._op("add", [self, other], shape)

    def relu(self):
        return self._op("relu", [self], self.shape)

    def matmul(self, other):
        other = self._coerce(other)
        assert self.shape[1] == other.shape[0]
        return self._op("matmul", [self, other], [self.shape[0], other.shape[1]])


class RefValueInt8(RefValue):
    """RefValue plus the three emitters of the reference-side patch."""

    def quantize(self, granularity="tensor"):
        if granularity not in ("tensor", "row"):
            raise ValueError(granularity)
        return self._op("quantize", [self], self.shape, "int8", granularity=granularity)

    def int8_matmul(self, other):
        if not isinstance(other, RefValue):
            nid = self.graph.add("constant", [], list(other.shape), "int8", value=other)
            other = type(self)(self.graph, nid, list(other.shape), "int8")
        assert self.dtype == "int8" and other.dtype == "int8" and self.shape[1] == other.shape[0]
        return self._op("int8_matmul", [self, other], [self.shape[0], other.shape[1]], "int32")

    def dequantize(self):
        assert self.dtype in ("int8", "int32")
        return self._op("dequantize", [self], self.shape, "float32")


def ref_trace(value_cls, fn, *examples):
    g = RefGraph()
    args = [value_cls(g, g.placeholder(list(x.shape)), list(x.shape)) for x in examples]
    g.output = fn(*args).node_id
    return g


def ref_bias_relu_fusion(g):
    """add(x, bias[N]) -> relu, the add used once, becomes fused_bias_relu(x,
    bias) in the relu's place (the reference's pattern); ids renumbered."""
    by_id = {n.id: n for n in g.nodes}
    uses = {n.id: 0 for n in g.nodes}
    for n in g.nodes:
        for i in n.inputs:
            uses[i] += 1
    fused = {}
    for n in g.nodes:
        if n.op == "relu":
            a = by_id[n.inputs[0]]
            if a.op == "add" and uses[a.id] == 1 and by_id[a.inputs[0]].shape != by_id[a.inputs[1]].shape:
                fused[n.id] = a.id
    skip = set(fused.values())
    out, remap = RefGraph(), {}
    for n in g.nodes:
        if n.id in skip:
            continue
        if n.id in fused:
            a = by_id[fused[n.id]]
            nid = out.add("fused_bias_relu", [remap[i] for i in a.inputs], n.shape, n.dtype)
        else:
            nid = out.add(n.op, [remap[i] for i in n.inputs], n.shape, n.dtype, **n.attrs)
            if n.op == "placeholder":
                out.inputs.append(nid)
        remap[n.id] = nid
    out.output = remap[g.output]
    return out


class RefLinear:
    """nn.Linear's parameters as the reference holds them (nn.py:74-81):
    weight [in, out], bias [out]."""

    def __init__(self, w, b):
        self.weight, self.bias = RefTensor(w), RefTensor(b)


# ---------------------------------------------------------------------------

@pytest.fixture(scope="module")
def env():
    from kansaiml_amd import kir, quantize
    from kansaiml_amd import hip as H
    assert H.available(), "no gfx950 device"
    return kir, quantize


def _data(seed, M=64, K=512, N1=512, N2=256):
    g = np.random.Generator(np.random.PCG64(seed))
    x = g.standard_normal((M, K), dtype=np.float32)
    w1 = g.standard_normal((K, N1), dtype=np.float32) * np.float32(0.02)
    b1 = g.standard_normal(N1, dtype=np.float32) * np.float32(0.1)
    w2 = g.standard_normal((N1, N2), dtype=np.float32) * np.float32(0.05)
    b2 = g.standard_normal(N2, dtype=np.float32)
    return x, w1, b1, w2, b2


def _matmul_bound(a, b):
    K = a.shape[1]
    return 2 * K * np.finfo(np.float32).eps * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))


def _oracle_int8_layer(x, w1, b1, act, wgran):
    """The int8 layer on the oracle: per-tensor or per-row activation codes,
    per-tensor or per-column packed weight codes, exact int32 GEMM, binary64
    dequantize, then the bias add and relu in fp32 (the fused_bias_relu
    node's arithmetic)."""
    qx, sx = O.ko_quantize_rows(x) if act == "row" else O.ko_quantize_tensor(x)
    qw, sw = O.ko_quantize_cols_packed(w1) if wgran == "col" else O.ko_quantize_tensor_packed(w1)
    acc = O.ko_gemm_i8(qx, qw)
    y = O.ko_epilogue(acc, np.atleast_1d(sx), np.atleast_1d(sw))
    return np.maximum(O.ko_add_bias(y, b1), np.float32(0))


@pytest.mark.parametrize("act,wgran", [("tensor", "tensor"), ("row", "col")])
def test_reference_style_graph_through_run_hip(env, act, wgran):
    """x -> QLinear(int8) -> relu -> matmul(W2) + b2, traced in the
    reference's conventions, bias+relu fused the reference's way.  The
    graph, its quant_fusion and its planned run all equal the oracle."""
    kir, quantize = env
    x, w1, b1, w2, b2 = _data(1)
    layer = quantize.QLinear(RefLinear(w1, b1), mode="int8", act_granularity=act, weight_granularity=wgran)
    W2, B2 = RefTensor(w2), RefTensor(b2)

    def fn(v):
        return layer(v).relu().matmul(W2).add(B2)

    g = ref_bias_relu_fusion(ref_trace(RefValueInt8, fn, x))
    ops = [n.op for n in g.nodes]
    assert ops.count("fused_bias_relu") == 1 and "relu" not in ops
    for op in ("quantize", "int8_matmul", "dequantize", "matmul", "add"):
        assert op in ops, ops
    consts = [n.attrs["value"] for n in g.nodes if n.op == "constant"]
    assert any(isinstance(v, RefTensor) for v in consts)

    h = _oracle_int8_layer(x, w1, b1, act, wgran)
    seen = {}

    def observe(node, value):
        if node.op == "fused_bias_relu":
            seen["h"] = value.numpy()

    y = kir.run_hip(g, x, observe=observe)
    np.testing.assert_array_equal(seen["h"].view(np.uint32), h.view(np.uint32))
    want = O.ko_add_bias(O.ko_matmul_f32(h, w2), b2)
    bound = _matmul_bound(h, w2) + np.float32(np.finfo(np.float32).eps) * np.abs(want)
    assert np.all(np.abs(y.astype(np.float64) - want) <= bound)

    # The same graph through this package's fusion pass and planned run.
    fused = kir.quant_fusion(g)
    y2 = kir.run_hip(fused, x)
    y3 = kir.run_hip_planned(fused, kir.plan_memory(fused), None, x)
    np.testing.assert_array_equal(y2.view(np.uint32), y3.view(np.uint32))
    assert np.all(np.abs(y2.astype(np.float64) - want) <= bound)


def test_unpatched_reference_tracer(env):
    """Without the int8 emitters: QLinear(mode='int8') refuses to trace, and
    QLinear(mode='weight_only') records what the reference's QLinear records
    (a matmul with the dequantized weight as a constant), whose run equals
    x @ dequantize(W) + b."""
    kir, quantize = env
    x, w1, b1, _, _ = _data(2)
    with pytest.raises(TypeError, match="int8_matmul"):
        ref_trace(RefValue, quantize.QLinear(RefLinear(w1, b1), mode="int8"), x)
    layer = quantize.QLinear(RefLinear(w1, b1), mode="weight_only")
    g = ref_trace(RefValue, layer, x)
    assert [n.op for n in g.nodes] == ["placeholder", "constant", "matmul", "constant", "add"]
    qw, sw = O.ko_quantize_tensor_packed(w1)
    wd = O.ko_dequantize_tensor(np.ascontiguousarray(qw.T), sw)
    np.testing.assert_array_equal(g.nodes[1].attrs["value"].numpy().view(np.uint32), wd.view(np.uint32))
    y = kir.run_hip(g, RefTensor(x))
    want = O.ko_add_bias(O.ko_matmul_f32(x, wd), b1)
    bound = _matmul_bound(x, wd) + np.float32(np.finfo(np.float32).eps) * np.abs(want)
    assert np.all(np.abs(y.astype(np.float64) - want) <= bound)


def test_reference_c1_graph_bit_exact(env):
    """C1 (x [64,512], W [512,512] ~N(0,0.02), zero bias, seed 0) traced in the
    reference's conventions: the int8 Linear's output is the oracle's bit
    for bit."""
    kir, quantize = env
    gen = np.random.Generator(np.random.PCG64(0))
    x = gen.standard_normal((64, 512), dtype=np.float32)
    w = gen.standard_normal((512, 512), dtype=np.float32) * np.float32(0.02)
    b = np.zeros(512, np.float32)
    layer = quantize.QLinear(RefLinear(w, b), mode="int8")
    g = ref_trace(RefValueInt8, layer, RefTensor(x))
    y = kir.run_hip(g, RefTensor(x))
    want = O.int8_linear(x, w, b)[0]
    np.testing.assert_array_equal(y.view(np.uint32), want.view(np.uint32))
