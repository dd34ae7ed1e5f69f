"""int8 KAN1 checkpoints on the GPU: a quantized model saves its codes and
scales and a fresh model loads them straight to the device (no
requantization), a float32 checkpoint in the reference's layout loads into
the int8 model (quantized per output channel on the way, the same
arithmetic as at construction), and an int8 checkpoint loads into a float32
model through the reference's dequantize (quantize.py:73-77).  The codes in
the file are checked against the oracle's per-column quantizer
(quantize.py:66-70 per output channel) and the dequantized values against
the oracle's dequantize.
"""

import json
import struct

import numpy as np
import pytest

from kansaiml_amd import serialize
from kansaiml_amd.charlm import CharLM, CharLMWeights
from kansaiml_amd.quantize import QLinear
from oracle import oracle as O

pytestmark = pytest.mark.gpu

SMALL = dict(vocab=20, d_model=128, heads=2, layers=2, d_ff=256, seq=16)  # head dimension 64


def _ids(batch, seq, vocab, seed):
    return np.random.Generator(np.random.PCG64(seed)).integers(0, vocab, (batch, seq)).astype(np.int32)


def test_charlm_int8_checkpoint_round_trip(tmp_path):
    w1 = CharLMWeights(**SMALL, seed=1, bias_std=0.05)
    m1 = CharLM(w1)
    p = str(tmp_path / "m.kan")
    serialize.save(m1, p)

    header = serialize.read_header(p)
    q = header["blocks.1.attn.w_k"]
    assert (q["dtype"], q["layout"], q["granularity"], q["shape"]) == ("int8", "packed", "col", [128, 128])
    assert header["blocks.0.ln1.weight"]["dtype"] == "float32"
    # The codes in the file are the oracle's per-output-channel codes of the
    # fp32 weight (packed [out, in]), the scales its binary64 scales.
    raw = open(p, "rb").read()
    start = 12 + struct.unpack("<Q", raw[4:12])[0]
    codes = np.frombuffer(raw, np.int8, 128 * 128, start + q["offset"]).reshape(128, 128)
    scales = np.frombuffer(raw, "<f8", 128, start + q["scales"]["offset"])
    oc, os_ = O.ko_quantize_cols_packed(w1.blocks[1]["w_k"])
    assert np.array_equal(codes, oc) and np.array_equal(scales, os_)
    # Size: 1 byte per int8 weight element + 8 per scale + 4 per fp32 element.
    size = 12 + struct.unpack("<Q", raw[4:12])[0]
    for meta in header.values():
        size += meta["nbytes"] + (meta["scales"]["nbytes"] if "scales" in meta else 0)
    assert size == len(raw)

    m2 = CharLM(CharLMWeights(**SMALL, seed=2, bias_std=0.05))
    ids = _ids(3, 16, 20, 7)
    before = m2(ids)  # traces and caches m2's graph with its own weights
    serialize.load(m2, p)
    ref = m1(ids)
    assert not np.array_equal(before, ref)
    got = m2(ids)  # the cached graph, now reading the loaded buffers
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_fp32_checkpoint_loads_into_the_int8_model(tmp_path):
    w = CharLMWeights(**SMALL, seed=3, bias_std=0.05)
    p = str(tmp_path / "fp32.kan")
    serialize.save(w, p)  # the reference's float32 layout
    m = CharLM(CharLMWeights(**SMALL, seed=4, bias_std=0.05))
    serialize.load(m, p)
    ids = _ids(2, 16, 20, 8)
    assert np.array_equal(m(ids).view(np.uint32), CharLM(w)(ids).view(np.uint32))


def test_int8_checkpoint_loads_into_a_float32_model(tmp_path):
    w = CharLMWeights(**SMALL, seed=5, bias_std=0.05)
    p = str(tmp_path / "m.kan")
    serialize.save(CharLM(w), p)
    host = CharLMWeights(**SMALL, seed=6, bias_std=0.05)
    serialize.load(host, p)
    oc, os_ = O.ko_quantize_cols_packed(w.blocks[0]["fc1_w"])
    want = O.ko_dequantize_rows(oc, os_).T  # packed [out, in] rows -> [in, out]
    got = host.blocks[0]["fc1_w"]
    assert got.dtype == np.float32 and np.array_equal(got.view(np.uint32), np.ascontiguousarray(want).view(np.uint32))
    assert np.array_equal(host.blocks[0]["fc1_b"], w.blocks[0]["fc1_b"])  # float32 entries unchanged


class _Lin:
    def __init__(self, i, o, seed):
        g = np.random.Generator(np.random.PCG64(seed))
        self.weight = (g.standard_normal((i, o)) * 0.05).astype(np.float32)
        self.bias = g.standard_normal(o).astype(np.float32)


def test_qlinear_round_trip_and_granularity_mismatch(tmp_path):
    a = QLinear(_Lin(256, 96, 1), mode="int8", weight_granularity="col")
    p = str(tmp_path / "l.kan")
    serialize.save(a, p)
    b = QLinear(_Lin(256, 96, 2), mode="int8", weight_granularity="col")
    serialize.load(b, p)
    assert np.array_equal(b.qweight.codes.numpy(), a.qweight.codes.numpy())
    assert np.array_equal(b.qweight.scales.numpy(), a.qweight.scales.numpy())
    x = np.random.Generator(np.random.PCG64(3)).standard_normal((8, 256)).astype(np.float32)
    assert np.array_equal(b(x).numpy().view(np.uint32), a(x).numpy().view(np.uint32))

    c = QLinear(_Lin(256, 96, 2), mode="int8", weight_granularity="tensor")
    with pytest.raises(ValueError, match="'col' int8 codes"):
        serialize.load(c, p)
    hdr = serialize.read_header(p)
    assert json.loads(json.dumps(hdr))["weight"]["granularity"] == "col"
