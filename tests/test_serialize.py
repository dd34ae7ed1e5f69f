"""KAN1 checkpoints on the host (no GPU): the byte layout of the reference's
format (python/kansai/serialize.py:17-30, 117-143), the round trip, and the
reference's failure modes (tests/test_serialize.py:189-256), plus the int8
entry checks that run before anything reaches the device.

The expected bytes are built here independently of kansaiml_amd.serialize:
the parameter names in the reference BigGPT's named_parameters() order
(train_shakespeare_large.py:61-79, nn.py:19-39, 384-390, 466-472), typed out
below, each tensor's float32 bytes concatenated, and the header written as
json.dumps of {name: {"dtype", "shape", "offset", "nbytes"}}.
"""

import json
import os
import struct

import numpy as np
import pytest

from kansaiml_amd import serialize
from kansaiml_amd.charlm import CharLMWeights

SMALL = dict(vocab=20, d_model=16, heads=2, layers=2, d_ff=32, seq=6)


def _reference_names(layers):
    names = ["tok_embed.weight", "pos_embed.weight"]
    for i in range(layers):
        names += [f"blocks.{i}.{n}" for n in ("ln1.weight", "ln1.bias", "attn.w_q", "attn.w_k", "attn.w_v",
                                             "attn.w_o", "ln2.weight", "ln2.bias", "fc1.weight", "fc1.bias",
                                             "fc2.weight", "fc2.bias")]
    return names + ["ln_f.weight", "ln_f.bias", "head.weight", "head.bias"]


def _expected_arrays(w):
    arrays = [w.tok, w.pos]
    for b in w.blocks:
        arrays += [b["ln1_w"], b["ln1_b"], b["w_q"], b["w_k"], b["w_v"], b["w_o"], b["ln2_w"], b["ln2_b"],
                   b["fc1_w"], b["fc1_b"], b["fc2_w"], b["fc2_b"]]
    return arrays + [w.lnf_w, w.lnf_b, w.head_w, w.head_b]


def test_fp32_checkpoint_bytes_are_the_reference_layout(tmp_path):
    w = CharLMWeights(**SMALL, seed=1, bias_std=0.1)
    p = tmp_path / "w.kan"
    serialize.save(w, str(p))

    header, blob, offset = {}, b"", 0
    for name, a in zip(_reference_names(SMALL["layers"]), _expected_arrays(w)):
        data = np.asarray(a, np.float32).tobytes()
        header[name] = {"dtype": "float32", "shape": list(a.shape), "offset": offset, "nbytes": len(data)}
        blob += data
        offset += len(data)
    hb = json.dumps(header).encode("utf-8")
    expected = b"KAN1" + struct.pack("<Q", len(hb)) + hb + blob
    got = p.read_bytes()
    assert got == expected
    # tests/test_serialize.py:243-256: the size is the 12-byte prefix, the
    # header and 4 bytes per parameter element.
    n = sum(a.size for a in _expected_arrays(w))
    assert os.path.getsize(p) == 4 + 8 + len(hb) + 4 * n


def test_fp32_round_trip_is_bit_exact(tmp_path):
    src = CharLMWeights(**SMALL, seed=1, bias_std=0.1)
    dst = CharLMWeights(**SMALL, seed=999, bias_std=0.1)
    assert not np.array_equal(src.blocks[0]["w_q"], dst.blocks[0]["w_q"])  # setup: they differ before
    p = str(tmp_path / "w.kan")
    serialize.save(src, p)
    serialize.load(dst, p)
    for (n1, a), (n2, b) in zip(src.named_parameters(), dst.named_parameters()):
        assert n1 == n2
        assert a.dtype == b.dtype == np.float32 and np.array_equal(a.view(np.uint32), b.view(np.uint32)), n1


class _Linear:
    """A reference-style Linear: attributes named as nn.py:77-78, no
    set_parameter (so load() assigns by attribute path)."""

    def __init__(self, i, o, seed):
        g = np.random.Generator(np.random.PCG64(seed))
        self.weight = g.standard_normal((i, o)).astype(np.float32)
        self.bias = g.standard_normal(o).astype(np.float32)

    def named_parameters(self, prefix=""):
        yield f"{prefix}weight", self.weight
        yield f"{prefix}bias", self.bias


class _Seq:
    def __init__(self, layers):
        self.layers = layers

    def named_parameters(self):
        for i, l in enumerate(self.layers):
            yield from l.named_parameters(f"layers.{i}.")


def test_attribute_path_load_like_the_reference(tmp_path):
    p = str(tmp_path / "s.kan")
    a = _Seq([_Linear(2, 8, 3), _Linear(8, 1, 4)])
    serialize.save(a, p)
    b = _Seq([_Linear(2, 8, 99), _Linear(8, 1, 100)])
    serialize.load(b, p)
    assert np.array_equal(a.layers[0].weight, b.layers[0].weight)
    assert np.array_equal(a.layers[1].bias, b.layers[1].bias)


def _expect(module, path, fragment):
    with pytest.raises(ValueError) as e:
        serialize.load(module, path)
    assert fragment in str(e.value), str(e.value)


def test_reference_failure_modes(tmp_path):
    p = str(tmp_path / "xor.kan")
    serialize.save(_Seq([_Linear(2, 8, 3), _Linear(8, 1, 4)]), p)
    # tests/test_serialize.py:189-204 (shape), 206-219 (missing), 221-228
    # (unexpected), 230-241 (magic).
    _expect(_Seq([_Linear(2, 16, 1), _Linear(16, 1, 2)]), p, "shape mismatch")
    _expect(_Seq([_Linear(2, 8, 3), _Linear(8, 1, 4), _Linear(1, 1, 6)]), p, "missing parameter")
    _expect(_Seq([_Linear(2, 8, 3)]), p, "doesn't expect")
    data = open(p, "rb").read()
    bad = str(tmp_path / "bad.kan")
    open(bad, "wb").write(b"NOPE" + data[4:])
    _expect(_Seq([_Linear(2, 8, 3), _Linear(8, 1, 4)]), bad, "not a Kansai checkpoint")
    # serialize.py:180-196: a byte count that disagrees with the shape, and a
    # range past the end of the file.
    open(bad, "wb").write(data[:-4])
    _expect(_Seq([_Linear(2, 8, 3), _Linear(8, 1, 4)]), bad, "runs past the end")
    hlen = struct.unpack("<Q", data[4:12])[0]
    header = json.loads(data[12:12 + hlen])
    header["layers.0.bias"]["nbytes"] = 28
    hb = json.dumps(header).encode()
    open(bad, "wb").write(b"KAN1" + struct.pack("<Q", len(hb)) + hb + data[12 + hlen:])
    _expect(_Seq([_Linear(2, 8, 3), _Linear(8, 1, 4)]), bad, "inconsistent header")
    open(bad, "wb").write(b"KAN1" + struct.pack("<Q", 5) + b"{oops" + data[12 + hlen:])
    _expect(_Seq([_Linear(2, 8, 3), _Linear(8, 1, 4)]), bad, "unparseable header")


def _write(path, entries):
    """A KAN1 file from (name, meta, payload bytes) with offsets filled in;
    meta may hold a "scales" dict whose payload follows."""
    header, blob = {}, b""
    for name, meta, payload, spayload in entries:
        meta = dict(meta, offset=len(blob), nbytes=len(payload))
        blob += payload
        if spayload is not None:
            meta["scales"] = dict(meta["scales"], offset=len(blob), nbytes=len(spayload))
            blob += spayload
        header[name] = meta
    hb = json.dumps(header).encode()
    open(path, "wb").write(b"KAN1" + struct.pack("<Q", len(hb)) + hb + blob)


def test_int8_entries_are_checked_before_upload(tmp_path):
    p = str(tmp_path / "q.kan")
    lin = _Linear(4, 3, 0)
    bias = lin.bias.tobytes()
    good_codes = np.arange(-6, 6, dtype=np.int8).tobytes()
    cases = [
        (dict(dtype="int8", shape=[4, 3], layout="packed", granularity="col",
              scales=dict(dtype="float64", shape=[3])), np.full(12, -128, np.int8).tobytes(),
         np.ones(3).tobytes(), "code -128"),
        (dict(dtype="int8", shape=[4, 3], layout="packed", granularity="col",
              scales=dict(dtype="float64", shape=[3])), good_codes, np.array([1.0, 0.0, 1.0]).tobytes(),
         "non-positive scale"),
        (dict(dtype="int8", shape=[4, 3], layout="packed", granularity="col",
              scales=dict(dtype="float64", shape=[1])), good_codes, np.ones(1).tobytes(), "needs 3 scales"),
        (dict(dtype="int8", shape=[4, 3], layout="sideways", granularity="col",
              scales=dict(dtype="float64", shape=[3])), good_codes, np.ones(3).tobytes(), "layout"),
        (dict(dtype="int8", shape=[4, 3], layout="packed", granularity="row",
              scales=dict(dtype="float64", shape=[4])), good_codes, np.ones(4).tobytes(), "packed codes"),
        (dict(dtype="int8", shape=[4, 3], layout="packed", granularity="col",
              scales=dict(dtype="float64", shape=[3])), good_codes[:-1], np.ones(3).tobytes(), "inconsistent"),
        (dict(dtype="bfloat16", shape=[4, 3]), good_codes, None, "unsupported dtype"),
    ]
    for meta, codes, scales, fragment in cases:
        _write(p, [("weight", meta, codes, scales),
                   ("bias", dict(dtype="float32", shape=[3]), bias, None)])
        before = lin.weight.copy()
        _expect(lin, p, fragment)
        assert np.array_equal(lin.weight, before)  # nothing assigned on a bad file


def test_truncated_scales_are_rejected(tmp_path):
    p = str(tmp_path / "q.kan")
    _write(p, [("weight", dict(dtype="int8", shape=[4, 3], layout="packed", granularity="col",
                               scales=dict(dtype="float64", shape=[3])),
                np.zeros(12, np.int8).tobytes(), np.ones(3).tobytes())])
    data = open(p, "rb").read()
    open(p, "wb").write(data[:-8])

    class _W:
        weight = np.zeros((4, 3), np.float32)

        def named_parameters(self):
            yield "weight", self.weight

    _expect(_W(), p, "scales byte range runs past the end")
