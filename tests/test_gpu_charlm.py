"""GPU parity for config C4 (the int8 char-LM forward): each fp32 kernel
against numpy, then the whole model against the CPU restatement
(oracle/charlm_ref.py, whose int8 steps are the C oracle's)."""

import numpy as np
import pytest
from scipy.special import erf

from oracle import charlm_ref as R

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def G():
    from kansaiml_amd import _native as N
    from kansaiml_amd.device import DeviceTensor as D
    assert N.available(), "no gfx950 device"
    return N, D


@pytest.mark.parametrize("rows,d", [(1, 384), (37, 384), (256, 64), (5, 1000), (8, 1024)])
def test_layernorm(G, rows, d):
    N, D = G
    gen = np.random.Generator(np.random.PCG64(rows * 31 + d))
    x = (gen.standard_normal((rows, d)) * 3 + 1).astype(np.float32)
    w = gen.standard_normal(d).astype(np.float32)
    b = gen.standard_normal(d).astype(np.float32)
    out = D([rows, d])
    xd, wd, bd = D.from_host(x), D.from_host(w), D.from_host(b)  # keep the buffers alive across the call
    N.call("kh_layernorm", xd.ptr, rows, d, wd.ptr, bd.ptr, 1e-5, out.ptr)
    x64 = x.astype(np.float64)
    m = x64.mean(-1, keepdims=True)
    ref = (x64 - m) / np.sqrt(((x64 - m) ** 2).mean(-1, keepdims=True) + 1e-5) * w + b
    assert np.abs(out.numpy() - ref).max() < 2e-5 * (1 + np.abs(ref).max())


def test_gelu(G):
    """kh_gelu (the GELU the fused GEMM epilogues share) against binary64
    x * 0.5 * (1 + erf(x / sqrt(2))): within 2e-7 * max(1, |x|) everywhere
    (the binary32 formula's bound, tests/test_gelu_formula.py, plus the
    hardware reciprocal's and exp2's ulp), the special values as the
    reference's binary32 formula gives them."""
    N, D = G
    x = np.concatenate([np.linspace(-12, 12, 400_001, dtype=np.float32),
                        (10.0 ** np.linspace(-30, 30, 2001)).astype(np.float32),
                        -(10.0 ** np.linspace(-30, 30, 2001)).astype(np.float32),
                        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 3e38, -3e38], np.float32)])
    out = D([x.size])
    xd = D.from_host(x)
    N.call("kh_gelu", xd.ptr, out.ptr, x.size)
    got = out.numpy()
    fin = np.isfinite(x)
    x64 = x[fin].astype(np.float64)
    ref = x64 * 0.5 * (1 + erf(x64 / np.sqrt(2)))
    err = np.abs(got[fin].astype(np.float64) - ref) / np.maximum(1.0, np.abs(x64))
    assert err.max() < 2e-7, (err.max(), x[fin][np.argmax(err)])
    sp = got[-7:]
    assert sp[0] == 0 and not np.signbit(sp[0]) and sp[1] == 0 and np.signbit(sp[1])
    assert sp[2] == np.inf and np.isnan(sp[3]) and np.isnan(sp[4])  # -inf * 0, as the reference formula
    assert sp[5] == np.float32(3e38) and sp[6] == 0


def test_gelu_order_over_every_binary32_value(G):
    """The absmax pass of a GELU epilogue (gelu_absmax_bits in
    kansaiml_amd/csrc/kh_gemm_i8.hip) takes max |GELU| over values whose
    largest is >= 0.3 as the GELU of that largest value.  Exact when the
    GPU's kh::gelu is non-decreasing over every non-negative binary32 value
    (+0 to +inf) and |GELU(x)| < GELU(0.3) for every negative finite x:
    both checked here value by value, all 2^32 - 2^24 + 1 of them, against
    the kernel's own threshold constant."""
    import os
    import re
    N, D = G
    src = open(os.path.join(os.path.dirname(__file__), "..", "kansaiml_amd", "csrc", "kh_gemm_i8.hip")).read()
    thr = int(re.search(r"constexpr int kGeluMonoBits = (0x[0-9A-Fa-f]+);", src).group(1), 16)
    assert thr == int(np.array([0.3], np.float32).view(np.uint32)[0])
    chunk = 1 << 27
    xd, od = D([chunk]), D([chunk])

    def gelu_bits(lo, hi):  # GELU of the binary32 values with bit patterns lo .. hi - 1
        n = hi - lo
        xd.view(0, [n]).copy_from(np.arange(lo, hi, dtype=np.uint32).view(np.float32))
        N.call("kh_gelu", xd.ptr, od.ptr, n)
        return od.view(0, [n]).numpy()

    prev = np.float32(-1.0)
    for lo in range(0, 0x7F800001, chunk):  # +0 .. +inf
        y = gelu_bits(lo, min(lo + chunk, 0x7F800001))
        assert not np.isnan(y).any(), lo
        assert y[0] >= prev and not (y[1:] < y[:-1]).any(), hex(lo)
        prev = y[-1]
    assert prev == np.inf
    g_thr = gelu_bits(thr, thr + 1)[0]
    neg_max = np.float32(0.0)
    for lo in range(0x80000000, 0xFF800000, chunk):  # -0 .. the most negative finite value
        y = gelu_bits(lo, min(lo + chunk, 0xFF800000))
        assert not np.isnan(y).any(), hex(lo)
        neg_max = max(neg_max, np.abs(y).max())
    assert 0.169 < neg_max < g_thr, (neg_max, g_thr)


@pytest.mark.parametrize("d", [48, 50, 384, 256])  # float4 path, scalar path, half-wave rows (C4's 384)
def test_embedding_exact_and_bad_id(G, d):
    N, D = G
    gen = np.random.Generator(np.random.PCG64(3))
    tok = gen.standard_normal((65, d)).astype(np.float32)
    pos = gen.standard_normal((20, d)).astype(np.float32)
    ids = gen.integers(0, 65, (3, 20)).astype(np.int32)
    out = D([60, d])
    idd, td, pd = D.from_host(ids), D.from_host(tok), D.from_host(pos)
    N.call("kh_embedding", idd.ptr, 60, 20, td.ptr, 65, pd.ptr, d, out.ptr)
    ref = tok[ids.reshape(-1)] + np.tile(pos, (3, 1))
    np.testing.assert_array_equal(out.numpy().view(np.uint32), ref.astype(np.float32).view(np.uint32))
    ids[1, 4] = 65
    idd = D.from_host(ids)
    N.call("kh_embedding", idd.ptr, 60, 20, td.ptr, 65, pd.ptr, d, out.ptr)
    with pytest.raises(RuntimeError):
        N.synchronize()
    N.synchronize()
    got = out.numpy()
    np.testing.assert_array_equal(got[24], np.zeros(d, np.float32))  # the bad id's row is zeros
    ok = np.arange(60) != 24
    np.testing.assert_array_equal(got[ok].view(np.uint32), ref[ok].astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("batch,seq,heads", [(2, 1, 2), (2, 5, 3), (1, 64, 2), (2, 100, 2), (2, 256, 6), (4, 200, 2),
                                             (8, 130, 3)])
@pytest.mark.parametrize("causal", [True, False])
def test_attention(G, batch, seq, heads, causal):
    N, D = G
    gen = np.random.Generator(np.random.PCG64(batch * 1000 + seq * 10 + heads))
    dm = heads * 64
    qkv = (gen.standard_normal((batch * seq, 3 * dm)) * 1.5).astype(np.float32)
    out = D([batch * seq, dm])
    qd = D.from_host(qkv)
    if causal:
        N.call("kh_causal_attention", qd.ptr, batch, seq, heads, 64, out.ptr)
    else:
        N.call("kh_attention_ex", qd.ptr, batch, seq, heads, 64, 0, out.ptr, None, 0, None)
    ref = R.attention(qkv.astype(np.float64), batch, seq, heads, causal=causal)
    assert np.abs(out.numpy() - ref).max() < 2e-5


MASK_SHAPES = {"TT": lambda b, h, t: (t, t), "B1TT": lambda b, h, t: (b, 1, t, t),
               "1HTT": lambda b, h, t: (1, h, t, t), "BHTT": lambda b, h, t: (b, h, t, t),
               "B11T": lambda b, h, t: (b, 1, 1, t)}


def _mask(gen, kind, batch, heads, seq):
    """A random additive mask of the named broadcast shape; the [B,1,1,T]
    kind is a key-padding mask (0, or -inf on each sequence's last keys,
    never key 0)."""
    shape = MASK_SHAPES[kind](batch, heads, seq)
    if kind == "B11T":
        m = np.zeros(shape, np.float32)
        for b in range(batch):
            pad = int(gen.integers(0, seq))  # 0 .. seq-1 padded keys
            m[b, 0, 0, seq - pad:] = -np.inf
        return m
    return (gen.standard_normal(shape) * 2).astype(np.float32)


@pytest.mark.parametrize("batch,seq,heads", [(2, 5, 3), (2, 100, 2), (1, 130, 2), (3, 64, 2)])
@pytest.mark.parametrize("kind", list(MASK_SHAPES))
@pytest.mark.parametrize("causal", [True, False])
def test_attention_additive_mask(G, batch, seq, heads, kind, causal):
    """scores.add(mask) before the softmax (nn.py:421-422) for every way a
    mask broadcasts to [batch, heads, seq, seq], with the causal mask on top
    or not, against the restatement; the per-(row, head) output maxima the
    masked kernel writes for a following per-token quantize are exact."""
    from kansaiml_amd import hip as H
    N, D = G
    gen = np.random.Generator(np.random.PCG64(batch * 7919 + seq * 31 + heads))
    dm = heads * 64
    qkv = (gen.standard_normal((batch * seq, 3 * dm)) * 1.5).astype(np.float32)
    m = _mask(gen, kind, batch, heads, seq)
    print(f"masked attention {kind} {m.shape} batch={batch} seq={seq} heads={heads} causal={causal}", flush=True)
    qd, md = D.from_host(qkv), D.from_host(m)
    out, _ = H.attention(qd, batch, seq, heads, dm, causal=causal, mask=md)
    got = out.numpy()
    ref = R.attention(qkv.astype(np.float64), batch, seq, heads, causal=causal, mask=m.astype(np.float64))
    assert np.isfinite(ref).all()
    assert np.abs(got - ref).max() < 3e-5
    out2, rp = H.attention_rows(qd, batch, seq, heads, dm, causal=causal, mask=md)
    N.synchronize()
    np.testing.assert_array_equal(out2.numpy().view(np.uint32), got.view(np.uint32))
    want = np.abs(got).reshape(batch * seq, heads, 64).max(axis=2).view(np.uint32)
    np.testing.assert_array_equal(rp.buf.numpy().view(np.uint32).reshape(-1)[:batch * seq * heads],
                                  want.reshape(-1))


@pytest.mark.parametrize("batch,seq,heads", [(2, 100, 2), (1, 256, 6)])
def test_attention_zero_mask_and_reference_causal_mask(G, batch, seq, heads):
    """A zero mask changes nothing (bit-exact against the unmasked kernel,
    causal or not), and the reference model's own causal mask (a [1, 1, T, T]
    tensor, 0 on and below the diagonal, -1e9 above) without the causal flag
    gives the causal kernel's output bit for bit: every masked probability
    is exactly 0 either way."""
    from kansaiml_amd import hip as H
    N, D = G
    gen = np.random.Generator(np.random.PCG64(seq + heads))
    dm = heads * 64
    qd = D.from_host((gen.standard_normal((batch * seq, 3 * dm)) * 1.5).astype(np.float32))
    zero = D.from_host(np.zeros((seq, seq), np.float32))
    for causal in (True, False):
        plain, _ = H.attention(qd, batch, seq, heads, dm, causal=causal)
        masked, _ = H.attention(qd, batch, seq, heads, dm, causal=causal, mask=zero)
        np.testing.assert_array_equal(masked.numpy().view(np.uint32), plain.numpy().view(np.uint32))
    tri = np.where(np.arange(seq)[None, :] <= np.arange(seq)[:, None], 0.0, -1e9).astype(np.float32)
    causal_out, _ = H.attention(qd, batch, seq, heads, dm, causal=True)
    ref_mask, _ = H.attention(qd, batch, seq, heads, dm, causal=False, mask=D.from_host(tri[None, None]))
    np.testing.assert_array_equal(ref_mask.numpy().view(np.uint32), causal_out.numpy().view(np.uint32))


def test_attention_fully_masked_row_is_nan(G):
    """A query whose every visible key the mask sets to -inf has no score
    left: NaN, as the reference states for a literal -inf mask that masks a
    whole row (nn.py:355-360; its softmax, Tensor.cpp:906-913, takes -inf -
    -inf).  The causal flag excludes later keys exactly, so under it a row
    whose keys up to the query are all -inf is NaN too (the restatement's
    additive -1e9 there leaves scores s - 1e9, which keep nothing of s in
    binary32: an artifact of rounding, not compared).  Every other row
    matches the restatement."""
    from kansaiml_amd import hip as H
    N, D = G
    batch, seq, heads = 1, 70, 2
    gen = np.random.Generator(np.random.PCG64(70))
    qkv = (gen.standard_normal((seq, 3 * 128))).astype(np.float32)
    m = np.zeros((seq, seq), np.float32)
    m[3, :] = -np.inf     # query 3 sees nothing
    m[66, :67] = -np.inf  # query 66: keys 0..66 masked; only keys 67..69 (later ones) left
    for causal in (True, False):
        out, _ = H.attention(D.from_host(qkv), batch, seq, heads, 128, causal=causal, mask=D.from_host(m))
        got = out.numpy()
        with np.errstate(invalid="ignore"):
            ref = R.attention(qkv.astype(np.float64), batch, seq, heads, causal=causal, mask=m.astype(np.float64))
        nan_rows = [3, 66] if causal else [3]
        assert np.isnan(got[nan_rows]).all() and np.isnan(ref[3]).all()
        ok = np.ones(seq, bool)
        ok[nan_rows] = False
        assert not np.isnan(got[ok]).any()
        assert np.abs(got[ok] - ref[ok]).max() < 2e-5


def test_attention_mask_shapes_rejected(G):
    from kansaiml_amd import hip as H
    N, D = G
    qd = D.from_host(np.zeros((2 * 8, 3 * 128), np.float32))
    for bad in [(8, 7), (3, 1, 8, 8), (1, 3, 8, 8), (2, 2, 2, 8, 8), (8, 8, 8)]:
        with pytest.raises(RuntimeError, match="broadcast"):
            H.attention(qd, 2, 8, 2, 128, mask=D.from_host(np.zeros(bad, np.float32)))
    with pytest.raises(TypeError, match="float32"):
        H.attention(qd, 2, 8, 2, 128, mask=D.from_host(np.zeros((8, 8), np.float64)))


def test_attention_mask_traced_and_fused(G):
    """A traced model with a mask constant: attention(mask) -> per-token
    QLinear.  run_hip's unfused graph matches the eager masked kernel and
    the oracle's int8 Linear of its output bit for bit; quant_fusion's
    (masked attention writing row maxima -> quantize-on-load GEMM) gives the
    same bits."""
    from kansaiml_amd import hip as H
    from kansaiml_amd import kir
    from kansaiml_amd import quantize as Q
    from oracle import oracle as O
    N, D = G
    batch, seq, heads = 2, 96, 3
    dm = heads * 64
    gen = np.random.Generator(np.random.PCG64(96))
    qkv = (gen.standard_normal((batch * seq, 3 * dm)) * 1.5).astype(np.float32)
    m = _mask(gen, "B11T", batch, heads, seq)
    w = (gen.standard_normal((dm, 256)) * 0.05).astype(np.float32)
    b = gen.standard_normal(256).astype(np.float32)

    class Lin:
        weight, bias = w, b

    proj = Q.QLinear(Lin(), mode="int8", act_granularity="row", weight_granularity="col")
    g = kir.trace(lambda x: proj(x.attention(batch, seq, heads, causal=True, mask=m)), qkv)
    f = kir.quant_fusion(g, qload=True)
    att = [n for n in f.nodes if n.op == "attention"]
    assert len(att) == 1 and att[0].attrs.get("row_absmax"), "the masked attention did not take the row partials"
    unfused = kir.run_hip(g, qkv)
    fused = kir.run_hip(f, qkv)
    eager, _ = H.attention(D.from_host(qkv), batch, seq, heads, dm, causal=True, mask=D.from_host(m))
    want = O.int8_linear(eager.numpy(), w, b, x_gran="row", w_gran="col")[0]
    np.testing.assert_array_equal(np.asarray(unfused, np.float32).view(np.uint32), want.view(np.uint32))
    np.testing.assert_array_equal(np.asarray(fused, np.float32).view(np.uint32), want.view(np.uint32))


def _host(v):
    """Host copy of a node value: arrays, or (codes, scales) for a QTensor
    (packed codes in their [out, in] storage order)."""
    from kansaiml_amd.quantize import QTensor
    if isinstance(v, QTensor):
        c = v.codes.numpy()
        c = c.reshape(v.shape[::-1] if v.packed else v.shape)
        return c, v.scales.numpy()
    return v.numpy()


def _check_node(node, got, ins):
    """One graph node against the restatement fed with the GPU's own inputs:
    bit-exact for embedding, add, quantize and the int8 Linear; the fp32
    kernels within their own unit tests' bounds."""
    from oracle import oracle as O
    op = node.op
    if op == "embedding":
        ids, tok, pos = ins
        seq = node.attrs["seq"]
        ref = (tok[ids.reshape(-1)] + np.tile(pos[:seq], (ids.size // seq, 1))).astype(np.float32)
        np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    elif op == "add":
        a, b = ins
        np.testing.assert_array_equal(got.view(np.uint32), (a + b).astype(np.float32).view(np.uint32))
    elif op == "quantize" and node.attrs.get("granularity") == "row":
        q, s = O.ko_quantize_rows(ins[0])
        np.testing.assert_array_equal(got[0], q)
        np.testing.assert_array_equal(got[1], s)
    elif op == "quantize":
        q, s = O.ko_quantize_tensor(ins[0])
        np.testing.assert_array_equal(got[0], q.reshape(got[0].shape))
        assert got[1][0] == s
    elif op == "int8_linear":
        if node.attrs.get("qload") and node.attrs.get("rows"):
            # the activation's per-row quantize ran inside the GEMM
            q, s = O.ko_quantize_rows(ins[0])
            ins = [(q, s)] + list(ins[1:])
        elif node.attrs.get("qload"):
            # the activation's per-tensor quantize ran inside the GEMM: the
            # oracle's quantize of the same fp32 input
            q, s = O.ko_quantize_tensor(ins[0])
            ins = [(q.reshape(ins[0].shape), np.array([s]))] + list(ins[1:])
        (qa, sa), (qw, sw) = ins[0], ins[1]
        at = node.attrs
        bias = ins[2] if at.get("bias") else None
        ref = O.ko_epilogue(O.ko_gemm_i8(qa, qw), sa, sw, bias)
        if at.get("act") == "gelu":
            # the fused epilogue applies the GELU kernel's binary32 arithmetic
            # to the bit-exact linear output
            x = ref.astype(np.float64)
            gref = x * 0.5 * (1 + erf(x / np.sqrt(2)))
            assert np.abs(got - gref).max() < 4e-6 * max(1.0, np.abs(gref).max())
        elif at.get("residual"):
            ref = (ins[-1] + ref).astype(np.float32)  # x.add(linear(..)): one fp32 add
            np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
        else:
            np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    elif op == "layer_norm_quant":
        # the unfused composition on the same input: kh_layernorm (checked
        # against the restatement as the layer_norm node is), then the
        # oracle's per-tensor quantize -- bit for bit
        from kansaiml_amd import hip as H
        from kansaiml_amd.device import DeviceTensor as D
        x, w, b = ins
        y, _ = H.layer_norm(D.from_host(x), D.from_host(w), D.from_host(b), node.attrs.get("eps", 1e-5))
        yh = y.numpy()
        ref = R.layer_norm(x.astype(np.float64), w, b, node.attrs.get("eps", 1e-5))
        assert np.abs(yh - ref).max() < 2e-5 * max(1.0, np.abs(ref).max())
        q, s = O.ko_quantize_tensor(yh)
        np.testing.assert_array_equal(got[0], q.reshape(got[0].shape))
        assert got[1][0] == s
    elif op == "layer_norm_quant_rows":
        # kh_layernorm on the same input, then the oracle's per-row quantize
        from kansaiml_amd import hip as H
        from kansaiml_amd.device import DeviceTensor as D
        x, w, b = ins
        y, _ = H.layer_norm(D.from_host(x), D.from_host(w), D.from_host(b), node.attrs.get("eps", 1e-5))
        q, s = O.ko_quantize_rows(y.numpy())
        np.testing.assert_array_equal(got[0], q)
        np.testing.assert_array_equal(got[1], s)
    elif op == "int8_linear_quant":
        # the unfused int8_linear on the same inputs (checked against the
        # oracle as the int8_linear node is), then the oracle's quantize
        from kansaiml_amd import hip as H
        from kansaiml_amd.device import DeviceTensor as D
        (qa, sa), (qw, sw) = ins[0], ins[1]
        at = node.attrs
        bias = ins[2] if at.get("bias") else None
        residual = ins[-1] if at.get("residual") else None
        y, _ = H.gemm_i8_fused(D.from_host(qa), D.from_host(qw), D.from_host(sa), D.from_host(sw),
                               D.from_host(bias) if bias is not None else None, act=at.get("act"),
                               residual=D.from_host(residual) if residual is not None else None)
        yh = y.numpy()
        _check_node(type("N", (), {"op": "int8_linear", "attrs": at})(), yh, ins)
        q, s = O.ko_quantize_tensor(yh)
        np.testing.assert_array_equal(got[0], q.reshape(got[0].shape))
        assert got[1][0] == s
    elif op == "int8_linear_quant_rows":
        # the unfused int8_linear on the same inputs (checked against the
        # oracle as the int8_linear node is), then the oracle's per-row
        # quantize: codes and binary64 row scales bit for bit
        from kansaiml_amd import hip as H
        from kansaiml_amd.device import DeviceTensor as D
        (qa, sa), (qw, sw) = ins[0], ins[1]
        at = node.attrs
        bias = ins[2] if at.get("bias") else None
        y, _ = H.gemm_i8_fused(D.from_host(qa), D.from_host(qw), D.from_host(sa), D.from_host(sw),
                               D.from_host(bias) if bias is not None else None, act=at.get("act"))
        yh = y.numpy()
        _check_node(type("N", (), {"op": "int8_linear", "attrs": at})(), yh, ins)
        q, s = O.ko_quantize_rows(yh.reshape(-1, yh.shape[-1]))
        np.testing.assert_array_equal(got[0].reshape(q.shape), q)
        np.testing.assert_array_equal(got[1], s)
    elif op == "layer_norm":
        x, w, b = ins
        ref = R.layer_norm(x.astype(np.float64), w, b, node.attrs.get("eps", 1e-5))
        assert np.abs(got - ref).max() < 2e-5 * max(1.0, np.abs(ref).max())
    elif op == "gelu":
        x = ins[0].astype(np.float64)
        ref = x * 0.5 * (1 + erf(x / np.sqrt(2)))
        assert np.abs(got - ref).max() < 4e-6 * max(1.0, np.abs(ref).max())
    elif op == "attention":
        ref = R.attention(ins[0].astype(np.float64), node.attrs["batch"], node.attrs["seq"], node.attrs["heads"],
                          causal=node.attrs["causal"])
        assert np.abs(got - ref).max() < 2e-5
    else:
        raise AssertionError(f"unchecked node kind {op}")


@pytest.mark.parametrize("seq,producer_quant", [(64, False), (100, False), (128, False), (100, True), (128, True),
                                                (128, "layer_norm")])
def test_small_model_matches_restatement(G, seq, producer_quant):
    """Two layers of the C4 architecture (d 384, 6 heads, FFN 1536, vocab 65)
    with nonzero biases, checked node by node: every node's GPU output
    against the restatement of that node applied to the GPU's own inputs.

    End to end the int8 model is discontinuous: one activation tensor's
    per-tensor scale is set by its largest element, and a one-ulp change of
    the attention output (below any fp32 kernel's rounding bound) re-rounds
    enough codes downstream to move logits by 2.5e-2 at seq 100.  So the
    whole-model comparison is against the fp32 model, at the quantization
    error's scale, and exactness is asserted per node.  The position table
    holds 128 rows: seq 128 runs under the causal mask, shorter sequences
    without it (BigGPT.forward, train_shakespeare_large.py:86)."""
    from kansaiml_amd.charlm import CharLM, CharLMWeights
    w = CharLMWeights(layers=2, seq=128, seed=1, bias_std=0.02)
    ids = np.random.Generator(np.random.PCG64(2)).integers(0, 65, (2, seq)).astype(np.int32)
    model = CharLM(w, producer_quant=producer_quant, qload=True)
    seen = {}
    y = model(ids, observe=lambda node, v: seen.__setitem__(node.id, (node, _host(v))))
    assert y.shape == (2 * seq, 65)
    g, _ = model.graph(2, seq)
    assert {n.attrs["causal"] for n in g.nodes if n.op == "attention"} == {seq == 128}
    by_id = {n.id: n for n in g.nodes}
    checked = set()
    for nid, (node, got) in seen.items():
        if node.op == "constant":
            continue
        ins = [ids if by_id[i].op == "placeholder" else seen[i][1] for i in node.inputs]
        _check_node(node, got, ins)
        checked.add(node.op)
    # GELU and the residual adds are fused into the int8_linear epilogues;
    # per-tensor quantizes read absmax partials their producers wrote.  With
    # producer_quant, every LayerNorm and fc1 (-> GELU) output feeds only a
    # per-tensor quantize, so those producers emit the codes themselves
    # ("layer_norm": the LayerNorms only).
    acts = {(n.op, n.attrs.get("act"), bool(n.attrs.get("residual"))) for n in g.nodes
            if n.op in ("int8_linear", "int8_linear_quant")}
    # With qload the quantizes of activations of at most 512 columns run
    # inside the consuming GEMM: the attention output's (and without
    # producer_quant the LayerNorms'), not fc1's 1536-column output.
    qloads = {by_id[n.inputs[0]].op for n in g.nodes if n.attrs.get("qload")}
    if producer_quant == "layer_norm":
        assert checked == {"embedding", "layer_norm_quant", "quantize", "int8_linear", "attention"}
        assert qloads == {"attention"}
        assert acts == {("int8_linear", None, False), ("int8_linear", "gelu", False), ("int8_linear", None, True)}
        assert all(n.attrs.get("absmax") for n in g.nodes
                   if n.op == "attention" or (n.op == "int8_linear" and n.attrs.get("act")))
    elif producer_quant:
        assert checked == {"embedding", "layer_norm_quant", "int8_linear", "int8_linear_quant", "attention"}
        assert qloads == {"attention"}
        assert acts == {("int8_linear", None, False), ("int8_linear_quant", "gelu", False),
                        ("int8_linear", None, True)}
        assert all(n.attrs.get("absmax") for n in g.nodes if n.op == "attention")
    else:
        assert checked == {"embedding", "layer_norm", "quantize", "int8_linear", "attention"}
        assert qloads == {"attention", "layer_norm"}
        assert acts == {("int8_linear", None, False), ("int8_linear", "gelu", False), ("int8_linear", None, True)}
        assert all(n.attrs.get("absmax") for n in g.nodes
                   if n.op in ("layer_norm", "attention") or (n.op == "int8_linear" and n.attrs.get("act")))
    np.testing.assert_array_equal(seen[g.output][1].view(np.uint32), y.view(np.uint32))
    # and the int8 model stays near the fp32 one (quantization error)
    fp = R.forward(w, ids, quantized=False)
    assert np.abs(y - fp).max() < 0.1 * np.abs(fp).max()
    # repeated forwards through the memory plan are identical
    np.testing.assert_array_equal(model(ids).view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("rows,D", [(1, 384), (17, 384), (1000, 384), (64, 1024), (33, 48), (40, 50), (5, 700)])
def test_layernorm_quant_rows(G, rows, D):
    """One-pass LayerNorm + per-row quantize against kh_layernorm's fp32
    output quantized per row by the oracle: codes and binary64 scales bit for
    bit.  Row 0 is constant (its output is the bias; with a zero bias an
    all-zero row, scale 1.0); D = 50 takes the unvectorized fallback."""
    from oracle import oracle as O
    from kansaiml_amd import hip as H
    N, D_ = G
    gen = np.random.Generator(np.random.PCG64(rows * 7 + D))
    x = (gen.standard_normal((rows, D)) * gen.uniform(0.1, 30, (rows, 1))).astype(np.float32)
    x[0] = 2.5
    w = gen.standard_normal(D).astype(np.float32)
    b = np.zeros(D, np.float32) if D == 48 else (gen.standard_normal(D) * 0.1).astype(np.float32)
    xd, wd, bd = D_.from_host(x), D_.from_host(w), D_.from_host(b)
    q, s = H.layer_norm_quant_rows(xd, wd, bd)
    y, _ = H.layer_norm(xd, wd, bd)
    rq, rs = O.ko_quantize_rows(y.numpy())
    np.testing.assert_array_equal(q.numpy(), rq)
    np.testing.assert_array_equal(s.numpy(), rs)
    if D == 48:
        assert s.numpy()[0] == 1.0 and not q.numpy()[0].any()


@pytest.mark.parametrize("producer_quant", [False, "layer_norm"])
def test_small_model_per_token(G, producer_quant):
    """The C4 architecture with per-token activation scales (every Linear's
    input quantized per row), node by node against the restatement on the
    GPU's own inputs; with producer fusion each LayerNorm emits its codes and
    scales in one pass."""
    from kansaiml_amd.charlm import CharLM, CharLMWeights
    w = CharLMWeights(layers=2, seq=128, seed=3, bias_std=0.02)
    ids = np.random.Generator(np.random.PCG64(4)).integers(0, 65, (2, 128)).astype(np.int32)
    model = CharLM(w, producer_quant=producer_quant, act_granularity="row")
    seen = {}
    y = model(ids, observe=lambda node, v: seen.__setitem__(node.id, (node, _host(v))))
    g, _ = model.graph(2, 128)
    by_id = {n.id: n for n in g.nodes}
    checked = set()
    for nid, (node, got) in seen.items():
        if node.op == "constant":
            continue
        ins = [ids if by_id[i].op == "placeholder" else seen[i][1] for i in node.inputs]
        _check_node(node, got, ins)
        checked.add(node.op)
    # With producer fusion the LayerNorms emit codes and scales and fc1
    # (-> GELU) quantizes its rows inside the GEMM; the attention output is
    # quantized inside the O GEMM (qload): no quantize node is left.
    if producer_quant:
        assert checked == {"embedding", "layer_norm_quant_rows", "int8_linear", "int8_linear_quant_rows", "attention"}
        assert [n.attrs.get("act") for n in g.nodes if n.op == "int8_linear_quant_rows"] == ["gelu"] * 2
    else:
        assert checked == {"embedding", "layer_norm", "quantize", "int8_linear", "attention"}
    assert all(n.attrs.get("granularity") == "row" for n in g.nodes if n.op == "quantize")
    fp = R.forward(w, ids, quantized=False)
    assert np.abs(y - fp).max() < 0.1 * np.abs(fp).max()
    np.testing.assert_array_equal(model(ids).view(np.uint32), y.view(np.uint32))


class _Sliced:
    """A node seen through a subset of its rows (attrs overridden)."""

    def __init__(self, node, **attrs):
        self.op, self.attrs = node.op, {**node.attrs, **attrs}


def _check_node_sampled(node, got, ins, gen, nrows=64, nbatches=3):
    """_check_node at full size: quantizes and embeddings in full; each
    int8 Linear on `nrows` sampled rows (its rows depend only on their own
    input rows and, per tensor, on the scale the GPU used); attention on
    `nbatches` sampled sequences (each sequence's outputs depend on its own
    rows only); LayerNorm on sampled rows."""
    op = node.op
    if op == "int8_linear":
        from oracle import oracle as O
        rows = np.sort(gen.choice(got.shape[0], nrows, replace=False))
        if node.attrs.get("qload") and node.attrs.get("rows"):
            # per-row scales: each row's own absmax (the oracle's per-row quantize)
            q, s = O.ko_quantize_rows(ins[0])
            ins = [(q, s)] + list(ins[1:])
            node = type("N", (), {"op": "int8_linear",
                                  "attrs": {k: v for k, v in node.attrs.items() if k not in ("qload", "rows")}})()
        elif node.attrs.get("qload"):
            # the per-tensor scale depends on the whole input: quantize it all
            q, s = O.ko_quantize_tensor(ins[0])
            ins = [(q.reshape(ins[0].shape), np.array([s]))] + list(ins[1:])
            node = type("N", (), {"op": "int8_linear",
                                  "attrs": {k: v for k, v in node.attrs.items() if k != "qload"}})()
        (qa, sa), w = ins[0], ins[1]
        sub = [(qa[rows], sa[rows] if sa.size > 1 else sa), w] + [
            (v[rows] if (k == len(ins) - 1 and node.attrs.get("residual")) else v) for k, v in enumerate(ins[2:], 2)]
        _check_node(node, got[rows], sub)
    elif op == "int8_linear_quant_rows":
        # the unfused GEMM (GPU) and per-row quantize in full, bit for bit;
        # the GEMM's rows against the oracle, and their per-row quantize, on
        # sampled rows
        from oracle import oracle as O
        from kansaiml_amd import hip as H
        from kansaiml_amd.device import DeviceTensor as D
        (qa, sa), (qw, sw) = ins[0], ins[1]
        at = node.attrs
        bias = ins[2] if at.get("bias") else None
        y, _ = H.gemm_i8_fused(D.from_host(qa), D.from_host(qw), D.from_host(sa), D.from_host(sw),
                               D.from_host(bias) if bias is not None else None, act=at.get("act"))
        q2, s2 = H.quantize_rows(y)
        np.testing.assert_array_equal(got[0].reshape(q2.shape), q2.numpy())
        np.testing.assert_array_equal(got[1], s2.numpy())
        rows = np.sort(gen.choice(got[0].shape[0], nrows, replace=False))
        yh = y.numpy()[rows]
        lin = type("N", (), {"op": "int8_linear", "attrs": at})()
        _check_node(lin, yh, [(qa[rows], sa[rows] if sa.size > 1 else sa), ins[1]] + list(ins[2:]))
        q, s = O.ko_quantize_rows(yh)
        np.testing.assert_array_equal(got[0][rows], q)
        np.testing.assert_array_equal(got[1][rows], s)
    elif op == "layer_norm":
        rows = np.sort(gen.choice(got.shape[0], nrows, replace=False))
        _check_node(node, got[rows], [ins[0][rows], ins[1], ins[2]])
    elif op == "attention":
        T = node.attrs["seq"]
        for b in gen.choice(node.attrs["batch"], nbatches, replace=False):
            r = slice(b * T, (b + 1) * T)
            _check_node(_Sliced(node, batch=1), got[r], [ins[0][r]])
    else:
        _check_node(node, got, ins)


@pytest.mark.parametrize("act_granularity,qload", [("tensor", False), ("tensor", True), ("row", False), ("row", True)])
def test_full_c4_forward(G, act_granularity, qload):
    """Config C4 at full size (vocab 65, d 384, 6 heads, 6 layers, FFN 1536,
    seq 256, batch 64), node by node on the GPU's own inputs: every
    quantize / layer_norm_quant(_rows) node exactly and in full against the
    oracle (codes and binary64 scales), every int8 Linear exactly on 64
    sampled rows (the oracle's int32 GEMM and binary64 epilogue; GELU to its
    fp32 bound), attention on 3 sampled sequences within 2e-5 of float64,
    the embedding exactly.  Then the whole model: deterministic, and near
    the fp32 model (max and mean deviation within 10 % of the logits' max
    and mean magnitude, the quantization error of 6 layers)."""
    from kansaiml_amd.charlm import CharLM, CharLMWeights
    w = CharLMWeights(seed=0)
    B, T = 64, 256
    ids = np.random.Generator(np.random.PCG64(9)).integers(0, 65, (B, T)).astype(np.int32)
    model = CharLM(w, act_granularity=act_granularity, qload=qload)
    seen = {}
    y = model(ids, observe=lambda node, v: seen.__setitem__(node.id, (node, _host(v))))
    assert y.shape == (B * T, 65) and np.isfinite(y).all()
    g, _ = model.graph(B, T)
    by_id = {n.id: n for n in g.nodes}
    gen = np.random.Generator(np.random.PCG64(17))
    counts = {}
    for nid, (node, got) in sorted(seen.items()):
        if node.op == "constant":
            continue
        ins = [ids if by_id[i].op == "placeholder" else seen[i][1] for i in node.inputs]
        _check_node_sampled(node, got, ins, gen)
        counts[node.op] = counts.get(node.op, 0) + 1
    ln = "layer_norm_quant_rows" if act_granularity == "row" else "layer_norm_quant"
    # 6 blocks: 2 LayerNorms, 4 Linears, attention; then the final LayerNorm
    # and the head.  The LayerNorms emit their own codes; the attention and
    # fc1 outputs are quantized by a quantize node, or with qload the
    # attention output inside the O GEMM (per tensor from the attention's
    # partials, or per row from its per-(row, head) partials).
    # Per row, fc1 (-> GELU) quantizes its own rows (int8_linear_quant_rows).
    lin = {"int8_linear": 25} if act_granularity == "tensor" else {"int8_linear": 19, "int8_linear_quant_rows": 6}
    nq = 12 if act_granularity == "tensor" else 6
    if not qload:
        assert counts == {"embedding": 1, ln: 13, **lin, "attention": 6, "quantize": nq}, counts
    else:
        assert counts == {"embedding": 1, ln: 13, **lin, "attention": 6, **({"quantize": nq - 6} if nq > 6 else {})}, counts
        assert sum(bool(n.attrs.get("qload")) for n in g.nodes) == 6
    np.testing.assert_array_equal(seen[g.output][1].view(np.uint32), y.view(np.uint32))
    del seen
    fp = R.forward(w, ids, quantized=False)
    assert np.abs(y - fp).max() < 0.1 * np.abs(fp).max()
    assert np.abs(y - fp).mean() < 0.1 * np.abs(fp).mean()
    np.testing.assert_array_equal(model(ids).view(np.uint32), y.view(np.uint32))
