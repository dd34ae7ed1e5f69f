"""Host logic of the KIR layer (no GPU): tracing the int8 path, the fusion
pass and the memory planner (python/kansai/kir.py:884-954's algorithm)."""

import numpy as np
import pytest

from kansaiml_amd import kir


def _linear_int8(x, w_q, bias, gran="tensor"):
    return x.quantize(gran).int8_matmul(w_q).dequantize().add(bias)


def test_trace_int8_linear_and_fuse():
    bias = np.zeros(8, np.float32)

    def fn(x, w):
        return _linear_int8(x, w.quantize("tensor"), bias)

    g = kir.trace(fn, np.zeros((4, 16), np.float32), np.zeros((16, 8), np.float32))
    ops = [n.op for n in g.nodes]
    assert ops == ["placeholder", "placeholder", "quantize", "quantize", "int8_matmul", "dequantize", "constant",
                   "add"]
    assert g.nodes[4].dtype == "int32" and g.nodes[4].shape == [4, 8]
    f = kir.quant_fusion(g)
    fops = [n.op for n in f.nodes]
    assert "int8_linear" in fops and "int8_matmul" not in fops and "dequantize" not in fops
    lin = [n for n in f.nodes if n.op == "int8_linear"][0]
    assert len(lin.inputs) == 3 and f.output == lin.id
    assert f.inputs == [0, 1]


def test_fusion_keeps_shared_intermediates():
    """An intermediate read twice must not be fused away."""
    def fn(x, w):
        acc = x.quantize().int8_matmul(w.quantize())
        d = acc.dequantize()
        return d.add(d)

    g = kir.trace(fn, np.zeros((4, 16), np.float32), np.zeros((16, 8), np.float32))
    f = kir.quant_fusion(g)
    ops = [n.op for n in f.nodes]
    assert "int8_linear" in ops  # int8_matmul -> dequantize fused; the add reads it twice
    assert ops[-1] == "add"
    assert f.nodes[-1].inputs[0] == f.nodes[-1].inputs[1]


def test_matmul_bias_and_bias_relu_fusion():
    b1 = np.zeros(8, np.float32)
    w1 = np.zeros((16, 8), np.float32)

    def fn(x):
        return x.matmul(w1).add(b1).relu()

    g = kir.trace(fn, np.zeros((4, 16), np.float32))
    f = kir.quant_fusion(g)
    assert [n.op for n in f.nodes if n.op not in ("placeholder", "constant")] == ["matmul_bias", "relu"]


def test_trace_shape_errors():
    with pytest.raises(ValueError):
        kir.trace(lambda x: x.matmul(np.zeros((3, 2), np.float32)), np.zeros((4, 5), np.float32))
    with pytest.raises(ValueError):
        kir.trace(lambda x: x.int8_matmul(x), np.zeros((4, 4), np.float32))
    with pytest.raises(ValueError):
        kir.trace(lambda x: x.quantize("col"), np.zeros((4, 4), np.float32))


def test_trace_rank3_activations():
    """[batch, seq, d] activations (nn.py:80-81, 412-414): Tensor::matmul's
    batched shapes (kir.py:164-181), the per-token quantize over the last
    axis, [B, T, N] + [N] as a bias, and the int8 chain still fusing into one
    int8_linear of the rank-3 shape."""
    bias = np.zeros(8, np.float32)
    w = np.zeros((16, 8), np.float32)
    x3 = np.zeros((2, 5, 16), np.float32)

    g = kir.trace(lambda x: x.matmul(w).add(bias), x3)
    assert [n.shape for n in g.nodes if n.op in ("matmul", "add")] == [[2, 5, 8], [2, 5, 8]]
    f = kir.quant_fusion(g)
    assert [n.op for n in f.nodes if n.op not in ("placeholder", "constant")] == ["matmul_bias"]

    for gran in ("tensor", "row"):
        g = kir.trace(lambda x, wq: _linear_int8(x, wq.quantize("tensor"), bias, gran), x3, w)
        mm = [n for n in g.nodes if n.op == "int8_matmul"][0]
        assert mm.shape == [2, 5, 8] and mm.dtype == "int32"
        f = kir.quant_fusion(g)
        lin = [n for n in f.nodes if n.op == "int8_linear"]
        assert len(lin) == 1 and lin[0].shape == [2, 5, 8] and lin[0].attrs["bias"] and f.output == lin[0].id

    # batched right operands trace with the reference's broadcast shapes
    g = kir.trace(lambda a, b: a.matmul(b), np.zeros((3, 1, 4, 6), np.float32), np.zeros((5, 6, 7), np.float32))
    assert g.nodes[-1].shape == [3, 5, 4, 7]
    g = kir.trace(lambda x: x.layer_norm(np.ones(16, np.float32), np.zeros(16, np.float32)), x3)
    assert g.nodes[-1].shape == [2, 5, 16]
    with pytest.raises(ValueError):
        kir.trace(lambda x: x.matmul(np.zeros((15, 8), np.float32)), x3)
    with pytest.raises(ValueError):
        kir.trace(lambda x: x.matmul(np.zeros((8,), np.float32)), x3)
    with pytest.raises(ValueError):  # the int8 weight must be 2-D
        kir.trace(lambda x, wq: x.quantize().int8_matmul(wq.quantize()), x3, np.zeros((2, 16, 8), np.float32))


def test_plan_memory_chain_reuses_slots():
    """A 6-deep chain of computed nodes: each op's input dies at that op, so
    (as in the reference's planner, which releases inputs after the op runs)
    the whole chain fits in one slot."""
    g = kir.Graph()
    x = g.placeholder([4, 4])
    cur = x
    for _ in range(6):
        cur = g.add("relu", [cur], [4, 4])
    g.output = cur
    plan = kir.plan_memory(g)
    assert plan.num_computed_nodes == 6
    assert plan.num_slots == 1
    assert plan.last_use[g.output] == len(g.nodes)
    assert x not in plan.slot_of


def test_plan_memory_matches_liveness_brute_force():
    """Slots never overlap in time: brute-force interval check on a random DAG."""
    rng = np.random.default_rng(0)
    for trial in range(20):
        g = kir.Graph()
        ids = [g.placeholder([2, 2])]
        ids.append(g.add("constant", [], [2, 2]))
        for _ in range(15):
            k = int(rng.integers(1, 3))
            ins = [int(v) for v in rng.choice(ids, size=k)]
            ids.append(g.add("add" if k == 2 else "relu", ins, [2, 2]))
        g.output = ids[-1]
        plan = kir.plan_memory(g)
        live = {}
        for nid, sid in plan.slot_of.items():
            live.setdefault(sid, []).append((nid, plan.last_use.get(nid, nid)))
        for sid, iv in live.items():
            iv.sort()
            for (a0, a1), (b0, b1) in zip(iv, iv[1:]):
                assert a1 <= b0, f"slot {sid} reused while live (trial {trial})"


def test_quantize_producers_fuse_into_quant_nodes():
    """A per-tensor quantize whose input is only read by it absorbs its
    producer: layer_norm -> layer_norm_quant, an int8 Linear chain (here with
    GELU) -> int8_linear_quant; a per-row one too: layer_norm_quant_rows,
    int8_linear_quant_rows.  A producer with a second reader keeps the fp32
    tensor."""
    w1 = np.zeros((16, 32), np.float32)
    w2 = np.zeros((32, 16), np.float32)
    g1, b1 = np.ones(16, np.float32), np.zeros(16, np.float32)
    bias = np.zeros(32, np.float32)

    def fn(x):
        h = x.layer_norm(g1, b1)
        f = h.quantize().int8_matmul(x._coerce(w1).quantize()).dequantize().add(bias).gelu()
        return f.quantize().int8_matmul(x._coerce(w2).quantize()).dequantize()

    g = kir.trace(fn, np.zeros((4, 16), np.float32))
    assert "layer_norm_quant" not in [n.op for n in kir.quant_fusion(g).nodes]  # off by default
    f = kir.quant_fusion(g, producer_quant=True)
    ops = [n.op for n in f.nodes if n.op not in ("placeholder", "constant")]
    assert "layer_norm_quant" in ops and "int8_linear_quant" in ops
    assert "layer_norm" not in ops and "gelu" not in ops
    lq = [n for n in f.nodes if n.op == "int8_linear_quant"][0]
    assert lq.dtype == "int8" and lq.attrs["act"] == "gelu" and lq.attrs["bias"]
    assert [n for n in f.nodes if n.op == "layer_norm_quant"][0].dtype == "int8"
    # "layer_norm": the LayerNorm emits codes, the GEMM chain keeps its fp32
    # output (and absmax partials for the separate quantize).
    fl = kir.quant_fusion(g, producer_quant="layer_norm")
    opsl = [n.op for n in fl.nodes if n.op not in ("placeholder", "constant")]
    assert "layer_norm_quant" in opsl and "int8_linear_quant" not in opsl and "layer_norm" not in opsl
    assert [n for n in fl.nodes if n.op == "int8_linear" and n.attrs.get("act") == "gelu"][0].attrs["absmax"]
    with pytest.raises(ValueError, match="producer_quant"):
        kir.quant_fusion(g, producer_quant="gelu")

    def shared(x):
        h = x.layer_norm(g1, b1)
        y = h.quantize().int8_matmul(x._coerce(np.zeros((16, 16), np.float32)).quantize()).dequantize()
        return y.add(h)

    f2 = kir.quant_fusion(kir.trace(shared, np.zeros((4, 16), np.float32)), producer_quant=True)
    ops2 = [n.op for n in f2.nodes]
    assert "layer_norm" in ops2 and "layer_norm_quant" not in ops2

    def per_row(x):
        return x.layer_norm(g1, b1).quantize("row").int8_matmul(x._coerce(w1).quantize()).dequantize()

    # a per-row quantize of a LayerNorm fuses into one pass (codes and
    # per-row scales), under either producer option, and not when it is off
    gr = kir.trace(per_row, np.zeros((4, 16), np.float32))
    for opt in (True, "layer_norm"):
        fr = kir.quant_fusion(gr, producer_quant=opt)
        ops3 = [n.op for n in fr.nodes]
        assert "layer_norm_quant_rows" in ops3 and "layer_norm" not in ops3 and "layer_norm_quant" not in ops3
        assert [n for n in fr.nodes if n.op == "layer_norm_quant_rows"][0].dtype == "int8"
    ops4 = [n.op for n in kir.quant_fusion(gr).nodes]
    assert "layer_norm" in ops4 and "layer_norm_quant_rows" not in ops4

    # an int8 Linear (-> bias -> GELU) whose only user is a per-row quantize
    # quantizes its own rows (int8_linear_quant_rows) under either producer
    # option; not with a residual add in the chain, nor when fusion is off
    def ffn_rows(x):
        h = x.layer_norm(g1, b1).quantize("row")
        f = h.int8_matmul(x._coerce(w1).quantize()).dequantize().add(bias).gelu()
        return f.quantize("row").int8_matmul(x._coerce(w2).quantize()).dequantize()

    gf = kir.trace(ffn_rows, np.zeros((4, 16), np.float32))
    for opt in (True, "layer_norm"):
        ff = kir.quant_fusion(gf, producer_quant=opt)
        opsf = [n.op for n in ff.nodes if n.op not in ("placeholder", "constant")]
        # (the two quantizes left are the weights')
        assert [o for o in opsf if o != "quantize"] == ["layer_norm_quant_rows", "int8_linear_quant_rows",
                                                        "int8_linear"], opsf
        assert all(ff.nodes[n.inputs[0]].op == "constant" for n in ff.nodes if n.op == "quantize")
        fq = [n for n in ff.nodes if n.op == "int8_linear_quant_rows"][0]
        assert fq.dtype == "int8" and fq.attrs["act"] == "gelu" and fq.attrs["bias"] and not fq.attrs["residual"]
        assert ff.nodes[fq.inputs[0]].op == "layer_norm_quant_rows"
    assert "int8_linear_quant_rows" not in [n.op for n in kir.quant_fusion(gf).nodes]

    def resid_rows(x):
        h = x.layer_norm(g1, b1)
        y = h.quantize("row").int8_matmul(x._coerce(np.zeros((16, 16), np.float32)).quantize()).dequantize()
        return y.add(x).quantize("row").int8_matmul(x._coerce(np.zeros((16, 8), np.float32)).quantize())

    fres = kir.quant_fusion(kir.trace(resid_rows, np.zeros((4, 16), np.float32)), producer_quant=True)
    assert "int8_linear_quant_rows" not in [n.op for n in fres.nodes]
    assert [n.attrs["residual"] for n in fres.nodes if n.op == "int8_linear"] == [True]


def test_quantize_fuses_into_its_int8_linear_with_qload():
    """qload=True: a per-tensor quantize whose only reader is an int8 Linear
    becomes part of it (operand 0 is then the fp32 activation) and the
    activation's producer writes absmax partials for it; a per-row quantize,
    a quantize with a second reader, or a quantize a producer already
    absorbed (producer_quant) is left alone.  Off by default."""
    w1 = np.zeros((16, 32), np.float32)
    w2 = np.zeros((32, 16), np.float32)
    g1, b1 = np.ones(16, np.float32), np.zeros(16, np.float32)
    bias = np.zeros(32, np.float32)

    def fn(x):
        h = x.layer_norm(g1, b1)
        f = h.quantize().int8_matmul(x._coerce(w1).quantize()).dequantize().add(bias).gelu()
        return f.quantize().int8_matmul(x._coerce(w2).quantize()).dequantize().add(x)

    g = kir.trace(fn, np.zeros((4, 16), np.float32))
    assert not any(n.attrs.get("qload") for n in kir.quant_fusion(g).nodes)  # off by default
    f = kir.quant_fusion(g, qload=True)
    lin = [n for n in f.nodes if n.op == "int8_linear"]
    assert [bool(n.attrs.get("qload")) for n in lin] == [True, True]
    assert not [n for n in f.nodes if n.op == "quantize" and f.nodes[n.inputs[0]].op != "constant"]
    # operand 0 is the fp32 producer, marked to write absmax partials
    assert [f.nodes[n.inputs[0]].op for n in lin] == ["layer_norm", "int8_linear"]
    assert all(f.nodes[n.inputs[0]].attrs.get("absmax") for n in lin)
    assert lin[1].attrs["residual"] and not lin[1].attrs["bias"]
    # with the LayerNorm emitting its codes, only the second quantize fuses
    fl = kir.quant_fusion(g, producer_quant="layer_norm", qload=True)
    assert [bool(n.attrs.get("qload")) for n in fl.nodes if n.op == "int8_linear"] == [False, True]
    assert "layer_norm_quant" in [n.op for n in fl.nodes]

    def per_row_and_shared(x):
        q = x.quantize("row").int8_matmul(x._coerce(w1).quantize()).dequantize()
        t = q.quantize()  # two readers
        a = t.int8_matmul(x._coerce(w2).quantize()).dequantize()
        return a.add(t.int8_matmul(x._coerce(np.ones((32, 16), np.float32)).quantize()).dequantize())

    f2 = kir.quant_fusion(kir.trace(per_row_and_shared, np.zeros((4, 16), np.float32)), qload=True)
    assert not any(n.attrs.get("qload") for n in f2.nodes)
    assert sum(n.op == "quantize" for n in f2.nodes if n.attrs.get("granularity") == "row") == 1


def test_masked_attention_trace_and_row_qload_fusion():
    """attention(mask=...) records the additive mask as its second input for
    every shape that broadcasts to [batch, heads, seq, seq] (nn.py:421-422),
    rejects the rest, and a per-row quantize of its output fused into the
    next int8 Linear (qload) makes the masked attention write row maxima."""
    batch, seq, heads, d = 2, 8, 2, 128
    qkv = np.zeros((batch * seq, 3 * d), np.float32)
    w = np.zeros((d, 16), np.float32)

    def model(mask):
        def fn(x):
            a = x.attention(batch, seq, heads, causal=True, mask=mask)
            return a.quantize("row").int8_matmul(x._coerce(w).quantize()).dequantize()
        return fn

    for shape in [(seq,), (seq, seq), (batch, 1, seq, seq), (1, heads, seq, seq), (batch, heads, seq, seq),
                  (batch, 1, 1, seq)]:
        g = kir.trace(model(np.zeros(shape, np.float32)), qkv)
        att = next(n for n in g.nodes if n.op == "attention")
        assert len(att.inputs) == 2 and g.nodes[att.inputs[1]].op == "constant"
        assert list(g.nodes[att.inputs[1]].shape) == list(shape)
        f = kir.quant_fusion(g, qload=True)
        assert next(n for n in f.nodes if n.op == "attention").attrs.get("row_absmax")
        lin = [n for n in f.nodes if n.op == "int8_linear"]
        assert len(lin) == 1 and lin[0].attrs.get("qload") and lin[0].attrs.get("rows")
    for bad in [(seq, seq + 1), (3, 1, seq, seq), (1, 3, seq, seq), (2, batch, heads, seq, seq), (seq + 1,)]:
        with pytest.raises(ValueError, match="broadcast"):
            kir.trace(model(np.zeros(bad, np.float32)), qkv)


@pytest.mark.parametrize("values,shape", [([1.0, 2.0, 3.0], [2, 2]), ([], [1]), ([1.0], [-1]), ([1.0, 2.0], [1])])
def test_from_flat_length_mismatch_raises(values, shape):
    """kansai.from_flat throws runtime_error("from_flat: data length does not
    match shape") (core/src/Tensor.cpp:96-97); the check runs before any
    device allocation, so it needs no GPU."""
    from kansaiml_amd.device import DeviceTensor
    with pytest.raises(RuntimeError, match="data length does not match shape"):
        DeviceTensor.from_flat(values, shape)
