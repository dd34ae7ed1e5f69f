"""GPU parity of the drop-in surface: the reference's quantize.py API and KIR
graphs run through run_hip, checked against the CPU oracle.

Mirrors the reference's own tests: tests/test_quantize.py (known-answer
quantize, 4.00x footprint, a trained XOR model still classifying after
quantization), tests/test_metal_backend.py:53-71 (run_<backend> of a traced
Linear-ReLU-Linear vs run()), tests/test_kir_memory_planner.py:54,72,94
(pooled == unpooled exactly; the pool stops growing)."""

import numpy as np
import pytest

from conftest import load_golden
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def K():
    from kansaiml_amd import kir, quantize
    from kansaiml_amd import _native as N
    assert N.available(), "no gfx950 device"
    return kir, quantize, N


class Linear:
    """The reference's nn.Linear layout (python/kansai/nn.py:74-81): weight
    [in, out], bias [out]."""

    def __init__(self, w, b):
        self.weight, self.bias = w, b


def bits32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_quantize_symmetric_reference_api(K):
    kir, Q, N = K
    g = load_golden("ref_test_quantize_1000")
    q, scale, shape = Q.quantize_symmetric(g["x"])
    assert shape == [1000] and isinstance(scale, float) and isinstance(q, list)
    assert q == g["q"].tolist() and scale == g["scale"][0]
    rec = Q.dequantize(q, scale, shape)
    np.testing.assert_array_equal(bits32(rec), bits32(g["deq"]))
    assert float(np.max(np.abs(g["x"].astype(np.float64) - rec))) <= scale / 2 + 1e-6
    qz, _, _ = Q.quantize_symmetric(np.array([0.0, 1.0, -1.0], np.float32))
    assert qz[0] == 0
    big = np.random.Generator(np.random.PCG64(1)).standard_normal((256, 256)).astype(np.float32)
    qt = Q.QTensor.from_tensor(big)
    assert (4 * big.size) / qt.nbytes() == 4.0
    with pytest.raises(ValueError):
        Q.quantize_symmetric(np.array([1.0, np.nan], np.float32))


def _c1(seed=0):
    gen = np.random.Generator(np.random.PCG64(seed))
    x = gen.standard_normal((64, 512), dtype=np.float32)
    w = gen.standard_normal((512, 512), dtype=np.float32) * np.float32(0.02)
    b = np.zeros(512, np.float32)
    return x, w, b


def test_c1_int8_linear_through_run_hip(K):
    """Config C1: per-tensor x and W, int8 GEMM, fused dequantize; bit-exact."""
    kir, Q, N = K
    x, w, b = _c1()
    layer = Q.QLinear(Linear(w, b), mode="int8", act_granularity="tensor", weight_granularity="tensor")
    g = kir.quant_fusion(kir.trace(layer, x))
    assert any(n.op == "int8_linear" for n in g.nodes)
    y = kir.run_hip(g, x)
    ey = O.int8_linear(x, w, b)[0]
    np.testing.assert_array_equal(bits32(y), bits32(ey))
    # eager call, unfused graph and fused graph agree exactly
    np.testing.assert_array_equal(bits32(layer(x).numpy()), bits32(ey))
    y_unfused = kir.run_hip(kir.trace(layer, x), x)
    np.testing.assert_array_equal(bits32(y_unfused), bits32(ey))
    # with the quantize fused into the GEMM too (quant_fusion(qload=True):
    # one launch, kh_linear_i8_tensor, for an activation with no producer)
    gq = kir.quant_fusion(kir.trace(layer, x), qload=True)
    assert [n.op for n in gq.nodes if n.attrs.get("qload")] == ["int8_linear"]
    np.testing.assert_array_equal(bits32(kir.run_hip(gq, x)), bits32(ey))
    # and stays within quantization error of the fp32 reference x @ W + b
    ref = O.ref_add_bias(O.ref_matmul(x, w), b) if O.ref_available() else x @ w + b
    assert np.abs(y - ref).max() < 0.05 * np.abs(ref).max()


@pytest.mark.parametrize("act,wg", [("row", "col"), ("tensor", "col"), ("row", "tensor")])
def test_int8_linear_granularities(K, act, wg):
    kir, Q, N = K
    gen = np.random.Generator(np.random.PCG64(5))
    x = gen.standard_normal((96, 384), dtype=np.float32)
    w = gen.standard_normal((384, 200), dtype=np.float32) * np.float32(0.02)
    b = gen.standard_normal(200).astype(np.float32)
    layer = Q.QLinear(Linear(w, b), mode="int8", act_granularity=act, weight_granularity=wg)
    y = kir.run_hip(kir.quant_fusion(kir.trace(layer, x)), x)
    ey = O.int8_linear(x, w, b, x_gran=act, w_gran=wg)[0]
    np.testing.assert_array_equal(bits32(y), bits32(ey))
    np.testing.assert_array_equal(bits32(layer(x).numpy()), bits32(ey))


def test_weight_only_qlinear_matches_reference_semantics(K):
    """quantize.py:115-122: x @ dequantize(W) + b, W per-tensor; the
    dequantized weight is bit-exact and the fp32 GEMM within rounding of the
    reference's own compiled i-k-j loop."""
    kir, Q, N = K
    x, w, b = _c1(1)
    b = np.random.Generator(np.random.PCG64(2)).standard_normal(512).astype(np.float32)
    layer = Q.QLinear(Linear(w, b))
    qw, sw = O.ko_quantize_tensor(w)
    wdeq = O.ko_dequantize_tensor(qw, sw)
    np.testing.assert_array_equal(bits32(layer.qweight.dequantize().numpy()), bits32(wdeq))
    assert layer.qweight.q == qw.reshape(-1).tolist() and layer.qweight.scale == sw
    ref = O.ref_add_bias(O.ref_matmul(x, wdeq), b) if O.ref_available() else O.ko_add_bias(O.ko_matmul_f32(x, wdeq), b)
    y = layer(x).numpy()
    bound = 2 * 512 * np.finfo(np.float32).eps * (np.abs(x) @ np.abs(wdeq) + np.abs(b))
    assert (np.abs(y - ref) <= bound).all()
    g = kir.quant_fusion(kir.trace(layer, x))
    assert any(n.op == "matmul_bias" for n in g.nodes)
    np.testing.assert_array_equal(bits32(kir.run_hip(g, x)), bits32(y))


@pytest.mark.parametrize("act,wg", [("row", "col"), ("tensor", "col"), ("tensor", "tensor")])
def test_qlinear_int8_rank3_activations(K, act, wg):
    """A [batch, seq, d] = [4, 64, 384] activation (the reference applies its
    Linears to such tensors, nn.py:80-81, 412-414) through QLinear(mode="int8"),
    eager, traced, traced and fused, and planned: output [4, 64, N],
    bit-exact against the oracle's int8 Linear of the flattened [256, 384]
    rows (per-token scales are per row of the last axis)."""
    kir, Q, N = K
    gen = np.random.Generator(np.random.PCG64(31))
    x = gen.standard_normal((4, 64, 384), dtype=np.float32)
    w = gen.standard_normal((384, 1152), dtype=np.float32) * np.float32(0.02)
    b = gen.standard_normal(1152).astype(np.float32)
    layer = Q.QLinear(Linear(w, b), mode="int8", act_granularity=act, weight_granularity=wg)
    ey = O.int8_linear(x.reshape(256, 384), w, b, x_gran=act, w_gran=wg)[0].reshape(4, 64, 1152)
    y = layer(x).numpy()
    assert y.shape == (4, 64, 1152)
    np.testing.assert_array_equal(bits32(y), bits32(ey))
    g = kir.trace(layer, x)
    assert g.nodes[g.output].shape == [4, 64, 1152]
    np.testing.assert_array_equal(bits32(kir.run_hip(g, x)), bits32(ey))
    f = kir.quant_fusion(g)
    assert [n.op for n in f.nodes if n.op == "int8_linear"] == ["int8_linear"]
    np.testing.assert_array_equal(bits32(kir.run_hip(f, x)), bits32(ey))
    plan = kir.plan_memory(f)
    np.testing.assert_array_equal(bits32(kir.run_hip_planned(f, plan, None, x)), bits32(ey))


def test_qlinear_weight_only_rank3_matches_reference_build(K):
    """quantize.py:115-122 on a [4, 64, 384] activation: x.matmul(dequantize(W))
    .add(bias) through the reference's batched path (Tensor.cpp:364-393) and
    general broadcast add (Tensor.cpp:158-166), compiled from its Ops.cpp,
    against the HIP path eager and traced: within the fp32 matmul's rounding
    bound, and the rank-3 call bit-identical to the same rows as a 2-D call."""
    kir, Q, N = K
    gen = np.random.Generator(np.random.PCG64(32))
    x = gen.standard_normal((4, 64, 384), dtype=np.float32)
    w = gen.standard_normal((384, 384), dtype=np.float32) * np.float32(0.02)
    b = gen.standard_normal(384).astype(np.float32)
    layer = Q.QLinear(Linear(w, b))
    y = layer(x).numpy()
    assert y.shape == (4, 64, 384)
    np.testing.assert_array_equal(bits32(y), bits32(layer(x.reshape(256, 384)).numpy().reshape(4, 64, 384)))
    f = kir.quant_fusion(kir.trace(layer, x))
    np.testing.assert_array_equal(bits32(kir.run_hip(f, x)), bits32(y))
    qw, sw = O.ko_quantize_tensor(w)
    wdeq = O.ko_dequantize_tensor(qw, sw)
    if O.ref_available():
        ref = O.ref_add_broadcast(O.ref_batched_matmul(x, wdeq), b)
    else:
        ref = O.ko_add_bias(O.ko_matmul_f32(x.reshape(256, 384), wdeq), b).reshape(4, 64, 384)
    bound = 2 * 384 * np.finfo(np.float32).eps * (np.abs(x) @ np.abs(wdeq) + np.abs(b))
    assert (np.abs(y - ref) <= bound).all()


def test_planned_equals_unplanned_and_pool_converges(K):
    kir, Q, N = K
    gen = np.random.Generator(np.random.PCG64(7))
    dims = [256, 512, 512, 256]
    params = [(gen.standard_normal((a, c), dtype=np.float32) * np.float32(0.05), gen.standard_normal(c).astype(np.float32))
              for a, c in zip(dims, dims[1:])]
    layers = [Q.QLinear(Linear(w, b), mode="int8", act_granularity="row", weight_granularity="col") for w, b in params]

    def mlp(x):
        for i, l in enumerate(layers):
            x = l(x)
            if i + 1 < len(layers):
                x = x.relu()
        return x

    x = gen.standard_normal((128, 256), dtype=np.float32)
    g = kir.quant_fusion(kir.trace(mlp, x))
    plan = kir.plan_memory(g)
    assert plan.num_slots < plan.num_computed_nodes
    pool = kir.DevicePool()
    ref = kir.run_hip(g, x)
    first = kir.run_hip_planned(g, plan, pool, x)
    np.testing.assert_array_equal(bits32(first), bits32(ref))
    allocs = pool.num_allocated()
    for _ in range(5):
        again = kir.run_hip_planned(g, plan, pool, x)
        np.testing.assert_array_equal(bits32(again), bits32(ref))
    assert pool.num_allocated() == allocs, "the device pool kept growing across identical runs"
    # the same network through the oracle: per-token quantize, int8 GEMM,
    # epilogue, relu (Ops.cpp:197-199: v > 0 ? v : 0)
    h = x
    for i, (w, b) in enumerate(params):
        h = O.int8_linear(h, w, b, x_gran="row", w_gran="col")[0]
        if i + 1 < len(params):
            h = np.where(h > 0, h, np.float32(0)).astype(np.float32)
    np.testing.assert_array_equal(bits32(ref), bits32(h))


def test_xor_still_classifies_after_quantization(K):
    """tests/test_quantize.py:81-124 of the reference: a trained 2-8-1 ReLU
    XOR model (trained here in numpy: SGD lr 0.1 on MSE, 3000 steps) keeps
    its predictions within 0.1 and still rounds to [0, 1, 1, 0] once both
    Linears are quantized."""
    kir, Q, N = K
    X = np.array([[0, 0], [0, 1], [1, 0], [1, 1]], np.float32)
    Y = np.array([[0], [1], [1], [0]], np.float32)
    rng = np.random.Generator(np.random.PCG64(3))
    w1 = rng.standard_normal((2, 8)).astype(np.float32) / np.sqrt(2)
    b1 = np.zeros(8, np.float32)
    w2 = rng.standard_normal((8, 1)).astype(np.float32) / np.sqrt(8)
    b2 = np.zeros(1, np.float32)
    for _ in range(3000):
        h = X @ w1 + b1
        a = np.maximum(h, 0)
        p = a @ w2 + b2
        d = 2 * (p - Y) / 4
        gw2, gb2 = a.T @ d, d.sum(0)
        da = d @ w2.T * (h > 0)
        gw1, gb1 = X.T @ da, da.sum(0)
        w1 -= 0.1 * gw1; b1 -= 0.1 * gb1; w2 -= 0.1 * gw2; b2 -= 0.1 * gb2
    float_pred = np.maximum(X @ w1 + b1, 0) @ w2 + b2
    if not (np.round(float_pred).ravel() == [0, 1, 1, 0]).all():
        pytest.skip("numpy XOR training did not converge for this seed")
    for mode in ("weight_only", "int8"):
        l1 = Q.QLinear(Linear(w1, b1), mode=mode)
        l2 = Q.QLinear(Linear(w2, b2), mode=mode)
        pred = kir.run_hip(kir.quant_fusion(kir.trace(lambda x: l2(l1(x).relu()), X)), X)
        assert np.abs(pred - float_pred).max() < 0.1, mode
        assert np.round(pred).ravel().tolist() == [0, 1, 1, 0], mode
