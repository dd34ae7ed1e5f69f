"""HIP graph capture and replay of a planned KIR run (kh_graph_* through
kir.HipGraph / CharLM.capture): every replay must equal the eager forward of
the same ids bit for bit, with eager work, other allocations and host
synchronisations between the replays; memory the graph writes must never be
handed to other work; loads into the model's buffers are seen by the next
replay; errors the kernels record surface as for an eager run."""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SMALL = dict(vocab=20, d_model=128, heads=2, layers=2, d_ff=256, seq=64)  # head dimension 64


@pytest.fixture(scope="module")
def G():
    from kansaiml_amd import _native as N
    from kansaiml_amd.device import DeviceTensor as D
    assert N.available(), "no gfx950 device"
    return N, D


def _ids(batch, seq, vocab, seed):
    return np.random.Generator(np.random.PCG64(seed)).integers(0, vocab, (batch, seq)).astype(np.int32)


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.mark.parametrize("producer_quant", [False, "layer_norm", True])
def test_replays_equal_eager_runs(G, producer_quant):
    N, D = G
    from kansaiml_amd.charlm import CharLM, CharLMWeights
    from kansaiml_amd import hip as H
    m = CharLM(CharLMWeights(**SMALL, seed=11, bias_std=0.05), producer_quant=producer_quant)
    g = m.capture(3, 40)
    first = None
    for k in range(4):
        ids = _ids(3, 40, 20, 100 + k)
        want = m(ids)  # eager, through the same planned graph
        # Unrelated eager work and allocations between the replays.
        x = np.random.Generator(np.random.PCG64(k)).standard_normal((257, 300)).astype(np.float32)
        codes, scale = H.quantize_tensor(D.from_host(x))
        N.synchronize()
        got = g(D.from_host(ids), to_host=False)
        first = got if first is None else first
        assert got is first  # one output buffer, overwritten by each replay
        np.testing.assert_array_equal(_bits(got.numpy()), _bits(want))
        # A host array input is uploaded into the graph's input buffer.
        np.testing.assert_array_equal(_bits(g(ids)), _bits(want))
        del codes, scale
    g.close()
    with pytest.raises(RuntimeError, match="closed"):
        g(ids)


def test_graph_memory_is_not_handed_to_other_work(G):
    N, D = G
    from kansaiml_amd.charlm import CharLM, CharLMWeights
    m = CharLM(CharLMWeights(**SMALL, seed=12, bias_std=0.05))
    g = m.capture(2, 64)
    # Eager outputs held across replays keep their values: none of their
    # buffers is one the graph writes.
    held = []
    for k in range(3):
        ids = _ids(2, 64, 20, 200 + k)
        out = m.forward(ids, to_host=False)
        held.append((out, out.numpy().copy()))
        g(_ids(2, 64, 20, 300 + k))
    for out, before in held:
        np.testing.assert_array_equal(_bits(out.numpy()), _bits(before))
    # The graph's own output, freed by the caller while the graph lives,
    # is not reused by later allocations either.
    out = g(_ids(2, 64, 20, 7), to_host=False)
    snap = out.numpy().copy()
    tmp = [D.from_host(np.full(out.shape, 3.0, np.float32)) for _ in range(4)]
    np.testing.assert_array_equal(_bits(out.numpy()), _bits(snap))
    assert all(t.ptr.value != out.ptr.value for t in tmp)
    stats_open = N.pool_stats()
    g.close()
    stats_closed = N.pool_stats()
    assert stats_closed["in_use"] <= stats_open["in_use"]


def test_loaded_weights_are_seen_by_the_next_replay(G, tmp_path):
    from kansaiml_amd import serialize
    from kansaiml_amd.charlm import CharLM, CharLMWeights
    src = CharLM(CharLMWeights(**SMALL, seed=13, bias_std=0.05))
    p = str(tmp_path / "m.kan")
    serialize.save(src, p)
    dst = CharLM(CharLMWeights(**SMALL, seed=14, bias_std=0.05))
    g = dst.capture(2, 32)
    ids = _ids(2, 32, 20, 5)
    before = g(ids)
    serialize.load(dst, p)
    after = g(ids)
    assert not np.array_equal(before, after)
    np.testing.assert_array_equal(_bits(after), _bits(src(ids)))
    g.close()


def test_capture_rules_and_recorded_errors(G):
    N, D = G
    from kansaiml_amd.charlm import CharLM, CharLMWeights
    # Host-synchronous calls are refused inside a capture; a discarded
    # capture leaves the stream usable.
    N.call("kh_graph_capture_begin")
    with pytest.raises(RuntimeError, match="captured"):
        N.synchronize()
    with pytest.raises(RuntimeError, match="already in progress"):
        N.call("kh_graph_capture_begin")
    N.call("kh_graph_capture_end", None)
    with pytest.raises(RuntimeError, match="no capture"):
        N.call("kh_graph_capture_end", ctypes.byref(ctypes.c_void_p()))
    m = CharLM(CharLMWeights(**SMALL, seed=15, bias_std=0.05))
    g = m.capture(1, 16)
    good = _ids(1, 16, 20, 9)
    want = m(good)
    bad = good.copy()
    bad[0, 3] = 20  # token id out of range: the embedding kernel records it
    g(bad, to_host=False)
    with pytest.raises(RuntimeError, match="out of range"):
        N.synchronize()
    np.testing.assert_array_equal(_bits(g(good)), _bits(want))
    with pytest.raises(ValueError, match="does not match"):
        g(_ids(1, 8, 20, 1))
    g.close()


def test_any_planned_graph_replays(G):
    """kir.HipGraph on a graph other than the char-LM: the fused C1 Linear
    (per-tensor quantize of x, int8 GEMM with dequantize and bias), replayed
    on new inputs with eager work between the replays, equals run_hip bit for
    bit each time."""
    N, D = G
    from kansaiml_amd import kir
    from kansaiml_amd.quantize import QLinear

    class _Lin:
        def __init__(self, w, b):
            self.weight, self.bias = w, b

    gen = np.random.Generator(np.random.PCG64(21))
    w = gen.standard_normal((512, 384), dtype=np.float32) * np.float32(0.02)
    b = gen.standard_normal(384).astype(np.float32)
    layer = QLinear(_Lin(w, b), mode="int8", act_granularity="tensor", weight_granularity="col")
    x0 = gen.standard_normal((64, 512), dtype=np.float32)
    g = kir.quant_fusion(kir.trace(layer, x0))
    hg = kir.HipGraph(g, kir.plan_memory(g), x0)
    for k in range(3):
        x = gen.standard_normal((64, 512), dtype=np.float32) * np.float32(1 + k)
        want = kir.run_hip(g, x)
        N.synchronize()
        np.testing.assert_array_equal(_bits(hg(x)), _bits(want))
    hg.close()
