"""Pins the CPU restatement of the C4 forward (oracle/charlm_ref.py) before the
GPU char-LM tests are checked against it.

Each check is chosen so a plausible mistake in the restatement fails it:
  * the reference tests' own known answers: LayerNorm of [1..4], [5..8]
    against their manual per-row normalization
    (tests/test_normalization.py:53-71 of the reference), GELU against
    x * 0.5 * (1 + erf(x / sqrt 2)) in binary64 (tests/test_activations.py:
    52-61), and the causal mask giving zero weight to every future position
    with each row of weights summing to 1
    (tests/test_multihead_attention.py:172-195);
  * closed forms: a constant row normalizes to the bias, gelu(x) - gelu(-x)
    = x, zero queries give the running mean of the values, the first
    position's output is its own value row;
  * brute force in binary64: attention as explicit per-(batch, head, query)
    loops over the reference's head split (python/kansai/nn.py:393-402),
    and the whole forward composed from the reference's module definitions
    (nn.py:308-331, 381-427, 466-478, 624-646 and BigGPT,
    examples/tinyshakespeare/train_shakespeare_large.py:79-89);
  * invariants: causality and batch independence (perturbing future or other
    batches' keys and values leaves an output row bit-identical);
  * mutation checks: deliberately wrong copies (planted here, on the CPU)
    must fail the checks above.
"""

import math

import numpy as np
import pytest

from oracle import charlm_ref as R

f32, f64 = np.float32, np.float64


def _gen(seed):
    return np.random.Generator(np.random.PCG64(seed))


# ---------------------------------------------------------------------------
# binary64 restatements built from the reference's module definitions
# ---------------------------------------------------------------------------

def _manual_normalize(row, eps=1e-5):
    """The reference test's own per-row normalization (pure Python floats)."""
    m = sum(row) / len(row)
    var = sum((v - m) ** 2 for v in row) / len(row)
    return [(v - m) / math.sqrt(var + eps) for v in row]


def _ln64(x, w, b, eps=1e-5):
    x = np.asarray(x, f64)
    out = np.empty_like(x)
    for i, row in enumerate(x):
        out[i] = np.asarray(_manual_normalize(list(row), eps)) * w.astype(f64) + b.astype(f64)
    return out


def _gelu64(x):
    return np.vectorize(lambda v: v * 0.5 * (1.0 + math.erf(v / math.sqrt(2.0))))(np.asarray(x, f64))


def _attn64(q, k, v, batch, seq, heads, causal=True, mask=None):
    """softmax(q k^T / sqrt(dk) + causal mask) v, one (batch, head, query) at a
    time; head h owns columns h*dk .. h*dk+dk-1 (a row-major reshape of
    d_model into (heads, dk), nn.py:393-402).  Unmasked: every query sees all
    seq keys.  mask: an additive mask broadcast to [batch, heads, seq, seq]
    added to the scaled scores (nn.py:421-422)."""
    D = q.shape[1]
    dk = D // heads
    mk = np.broadcast_to(np.asarray(mask, f64), (batch, heads, seq, seq)) if mask is not None else None
    out = np.zeros((batch * seq, D), f64)
    for b in range(batch):
        for h in range(heads):
            cols = slice(h * dk, (h + 1) * dk)
            for i in range(seq):
                qi = q[b * seq + i, cols].astype(f64)
                keys = i + 1 if causal else seq
                s = [float(qi @ k[b * seq + j, cols].astype(f64)) / math.sqrt(dk) for j in range(keys)]
                if mk is not None:
                    s = [t + float(mk[b, h, i, j]) for j, t in enumerate(s)]
                m = max(s)
                e = [math.exp(t - m) for t in s]
                tot = sum(e)
                for j in range(keys):
                    out[b * seq + i, cols] += (e[j] / tot) * v[b * seq + j, cols].astype(f64)
    return out


def _forward64(w, ids):
    """BigGPT's forward in binary64: token + position embedding, pre-LN
    blocks (x + attn(LN1 x); x + fc2(GELU(fc1(LN2 x)))), final LN, head;
    the causal mask only when seq fills the position table
    (train_shakespeare_large.py:86)."""
    batch, seq = ids.shape
    causal = seq == w.seq
    x = np.stack([w.tok[ids[b, t]].astype(f64) + w.pos[t].astype(f64) for b in range(batch) for t in range(seq)])
    for p in w.blocks:
        h = _ln64(x, p["ln1_w"], p["ln1_b"])
        q, k, v = (h @ p[n].astype(f64) for n in ("w_q", "w_k", "w_v"))
        x = x + _attn64(q, k, v, batch, seq, w.heads, causal) @ p["w_o"].astype(f64)
        h = _ln64(x, p["ln2_w"], p["ln2_b"])
        f = _gelu64(h @ p["fc1_w"].astype(f64) + p["fc1_b"].astype(f64))
        x = x + f @ p["fc2_w"].astype(f64) + p["fc2_b"].astype(f64)
    x = _ln64(x, w.lnf_w, w.lnf_b)
    return x @ w.head_w.astype(f64) + w.head_b.astype(f64)


def _qkv(batch, seq, heads, dk, seed):
    return _gen(seed).standard_normal((batch * seq, 3 * heads * dk)).astype(f32)


# ---------------------------------------------------------------------------
# LayerNorm
# ---------------------------------------------------------------------------

def test_layer_norm_reference_known_answer():
    x = np.array([[1, 2, 3, 4], [5, 6, 7, 8]], f32)
    got = R.layer_norm(x, np.ones(4, f32), np.zeros(4, f32))
    want = _manual_normalize([1, 2, 3, 4]) + _manual_normalize([5, 6, 7, 8])
    np.testing.assert_allclose(got.reshape(-1), want, rtol=0, atol=1e-6)


@pytest.mark.parametrize("offset,spread", [(0.0, 1.0), (3.0, 0.1), (-50.0, 4.0)])
def test_layer_norm_vs_binary64(offset, spread):
    g = _gen(7)
    x = (offset + spread * g.standard_normal((48, 192))).astype(f32)
    w = g.standard_normal(192).astype(f32)
    b = g.standard_normal(192).astype(f32)
    got = R.layer_norm(x, w, b)
    want = _ln64(x, w, b)
    # float32 centring loses ~|offset| * 2^-24 per element, relative to spread
    tol = 4e-6 * (1.0 + abs(offset) / spread) * (np.abs(w) + 1.0)
    assert np.all(np.abs(got - want) <= tol)
    # with the identity affine the rows have mean 0 and mean square var/(var+eps)
    n = R.layer_norm(x, np.ones(192, f32), np.zeros(192, f32)).astype(f64)
    assert np.all(np.abs(n.mean(axis=1)) < 1e-4)
    var = x.astype(f64).var(axis=1)
    np.testing.assert_allclose((n * n).mean(axis=1), var / (var + 1e-5), rtol=1e-4)


def test_layer_norm_constant_and_tiny_variance_rows():
    g = _gen(8)
    w = g.standard_normal(192).astype(f32)
    b = g.standard_normal(192).astype(f32)
    # a constant row centres to exact zeros: the output is the bias itself
    const = np.full((2, 192), 1.5, f32)
    np.testing.assert_array_equal(R.layer_norm(const, w, b), np.broadcast_to(b, (2, 192)))
    # variance far below eps: eps sits inside the square root
    tiny = np.zeros((1, 192), f32)
    tiny[0, 5] = 1e-3
    got = R.layer_norm(tiny, w, b)
    np.testing.assert_allclose(got, _ln64(tiny, w, b), rtol=1e-5, atol=1e-6)


def _ln_mutant(x, w, b, variant, eps=1e-5):
    x = x.astype(f64)
    c = x - x.mean(axis=-1, keepdims=True)
    n = x.shape[-1]
    if variant == "unbiased_var":
        d = np.sqrt((c * c).sum(axis=-1, keepdims=True) / (n - 1) + eps)
    elif variant == "eps_outside_sqrt":
        d = np.sqrt((c * c).mean(axis=-1, keepdims=True)) + eps
    elif variant == "no_eps":
        d = np.sqrt((c * c).mean(axis=-1, keepdims=True))
    return (c / d * w + b).astype(f32)


@pytest.mark.parametrize("variant", ["unbiased_var", "eps_outside_sqrt", "no_eps"])
def test_layer_norm_mutants_are_caught(variant):
    known = _ln_mutant(np.array([[1, 2, 3, 4], [5, 6, 7, 8]], f32), 1, 0, variant).reshape(-1)
    want = _manual_normalize([1, 2, 3, 4]) + _manual_normalize([5, 6, 7, 8])
    tiny = np.zeros((1, 192), f32)
    tiny[0, 5] = 1e-3
    caught_known = np.max(np.abs(known - want)) > 1e-6
    caught_tiny = not np.allclose(_ln_mutant(tiny, 1, 0, variant), _ln64(tiny, np.ones(192, f32), np.zeros(192, f32)),
                                  rtol=1e-5, atol=1e-6)
    assert caught_known or caught_tiny, f"mutant {variant} passed"


# ---------------------------------------------------------------------------
# GELU (exact erf form, backend/cpu/src/Ops.cpp:250-256 of the reference)
# ---------------------------------------------------------------------------

def _gelu_inputs():
    rng = _gen(9)
    ref_test = rng.uniform(0.3, 2.5, 5)  # the reference test's positive range
    grid = np.linspace(-12.0, 12.0, 24001)
    return np.concatenate([ref_test, grid, [0.0, -0.0, 1e-30, -1e-30, 40.0, -40.0]]).astype(f32)


def test_gelu_vs_binary64_erf():
    x = _gelu_inputs()
    got = R.gelu(x).astype(f64)
    want = _gelu64(x)
    # float32 erf, 1 + erf and the two products each round once
    tol = 3e-7 * np.abs(x.astype(f64)) + 1e-37
    assert np.all(np.abs(got - want) <= tol)


def test_gelu_closed_forms():
    x = _gelu_inputs()
    g = R.gelu(x)
    assert R.gelu(np.array([0.0], f32))[0] == 0.0
    big = np.array([10.0, 20.0, 40.0], f32)
    np.testing.assert_array_equal(R.gelu(big), big)  # erf saturates to 1 in float32
    np.testing.assert_array_equal(R.gelu(-big), np.zeros(3, f32))
    # gelu(x) - gelu(-x) = x * (cdf(x) + cdf(-x)) = x
    odd = g.astype(f64) - R.gelu(-x).astype(f64)
    assert np.all(np.abs(odd - x) <= 4e-7 * np.abs(x.astype(f64)) + 1e-37)


@pytest.mark.parametrize("variant", ["tanh_approx", "sigmoid_approx", "one_minus_erf"])
def test_gelu_mutants_are_caught(variant):
    x = _gelu_inputs().astype(f64)
    if variant == "tanh_approx":
        m = 0.5 * x * (1 + np.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))
    elif variant == "sigmoid_approx":
        m = x / (1 + np.exp(-1.702 * x))
    else:
        m = x * 0.5 * (1 - np.vectorize(math.erf)(x / math.sqrt(2)))
    m = m.astype(f32).astype(f64)
    assert np.any(np.abs(m - _gelu64(x)) > 3e-7 * np.abs(x) + 1e-37)


# ---------------------------------------------------------------------------
# Causal attention (nn.py:381-427 under BigGPT's additive -1e9 mask)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("batch,seq,heads,dk", [(1, 1, 1, 4), (2, 7, 3, 4), (1, 33, 2, 16), (3, 5, 6, 8)])
def test_attention_vs_binary64_loops(batch, seq, heads, dk):
    qkv = _qkv(batch, seq, heads, dk, seed=seq * 31 + heads)
    D = heads * dk
    got = R.causal_attention(qkv, batch, seq, heads)
    want = _attn64(qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:], batch, seq, heads)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6)


@pytest.mark.parametrize("batch,seq,heads,dk", [(1, 1, 1, 4), (2, 7, 3, 4), (1, 33, 2, 16)])
def test_unmasked_attention_vs_binary64_loops(batch, seq, heads, dk):
    qkv = _qkv(batch, seq, heads, dk, seed=seq * 37 + heads)
    D = heads * dk
    got = R.attention(qkv, batch, seq, heads, causal=False)
    want = _attn64(qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:], batch, seq, heads, causal=False)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6)
    # zero queries: every position gets the mean of all its sequence's values
    z = qkv.copy()
    z[:, :D] = 0
    v = z[:, 2 * D:].astype(f64).reshape(batch, seq, D)
    mean = np.broadcast_to(v.mean(axis=1, keepdims=True), v.shape).reshape(batch * seq, D)
    np.testing.assert_allclose(R.attention(z, batch, seq, heads, causal=False), mean, rtol=0, atol=1e-6)
    # and the unmasked form is not the causal one
    if seq > 1:
        assert not np.allclose(got, R.causal_attention(qkv, batch, seq, heads), rtol=0, atol=2e-6)


@pytest.mark.parametrize("mshape", [(7, 7), (2, 1, 7, 7), (1, 3, 7, 7), (2, 3, 7, 7), (2, 1, 1, 7)])
@pytest.mark.parametrize("causal", [False, True])
def test_masked_attention_vs_binary64_loops(mshape, causal):
    """The caller's additive mask (nn.py:421-422) in the restatement against
    the binary64 loops, for every broadcast shape the kernel takes."""
    batch, seq, heads, dk = 2, 7, 3, 8
    D = heads * dk
    qkv = _qkv(batch, seq, heads, dk, seed=77)
    mask = (_gen(len(mshape) * 13 + sum(mshape)).standard_normal(mshape) * 2).astype(f32)
    got = R.attention(qkv, batch, seq, heads, causal=causal, mask=mask)
    want = _attn64(qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:], batch, seq, heads, causal=causal, mask=mask)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6)
    # a mask matters: the unmasked result differs
    assert not np.allclose(got, R.attention(qkv, batch, seq, heads, causal=causal), rtol=0, atol=1e-4)


def test_masked_attention_closed_forms():
    """Zero mask = no mask; BigGPT's own [1, 1, T, T] -1e9 mask
    (train_shakespeare_large.py:74-75) = the causal form; a -inf mask on key
    j for every query = attention without key j; a constant added to a
    query's whole mask row changes nothing (softmax shift invariance)."""
    batch, seq, heads, dk = 2, 9, 3, 8
    D = heads * dk
    qkv = _qkv(batch, seq, heads, dk, seed=91)
    plain = R.attention(qkv, batch, seq, heads, causal=False)
    np.testing.assert_array_equal(R.attention(qkv, batch, seq, heads, causal=False,
                                              mask=np.zeros((seq, seq), f32)), plain)
    big = np.array([[0.0 if j <= i else -1e9 for j in range(seq)] for i in range(seq)], f32).reshape(1, 1, seq, seq)
    np.testing.assert_array_equal(R.attention(qkv, batch, seq, heads, causal=False, mask=big),
                                  R.causal_attention(qkv, batch, seq, heads))
    j = 4
    drop = np.zeros((1, 1, 1, seq), f32)
    drop[..., j] = -np.inf
    keep = [t for t in range(seq) if t != j]
    q, k, v = qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:]
    got = R.attention(qkv, batch, seq, heads, causal=False, mask=drop)
    for b in range(batch):
        rows = [b * seq + t for t in keep]
        sub = np.concatenate([q[rows], k[rows], v[rows]], axis=1)
        want = _attn64(sub[:, :D], sub[:, D:2 * D], sub[:, 2 * D:], 1, seq - 1, heads, causal=False)
        # queries other than j see the same keys; compare their rows
        np.testing.assert_allclose(got[rows], want, rtol=0, atol=2e-6)
    shift = (_gen(3).standard_normal((1, 1, seq, 1)) * 5).astype(f64)
    np.testing.assert_allclose(R.attention(qkv, batch, seq, heads, causal=False, mask=shift),
                               plain, rtol=0, atol=2e-6)


def test_attention_closed_forms():
    batch, seq, heads, dk = 2, 9, 3, 8
    D = heads * dk
    qkv = _qkv(batch, seq, heads, dk, seed=5)
    # each query's first position attends only to itself
    out = R.causal_attention(qkv, batch, seq, heads)
    for b in range(batch):
        np.testing.assert_array_equal(out[b * seq], qkv[b * seq, 2 * D:])
    # zero queries: uniform weights over positions 0..i (future weights 0,
    # every row of weights sums to 1) -> the running mean of the values
    z = qkv.copy()
    z[:, :D] = 0
    out = R.causal_attention(z, batch, seq, heads).astype(f64)
    v = z[:, 2 * D:].astype(f64).reshape(batch, seq, D)
    running = np.cumsum(v, axis=1) / np.arange(1, seq + 1)[None, :, None]
    np.testing.assert_allclose(out, running.reshape(batch * seq, D), rtol=0, atol=1e-6)
    # scores of several hundred: the max-subtracted softmax stays finite
    hot = qkv.copy()
    hot[:, :2 * D] *= f32(12.0)
    got = R.causal_attention(hot, batch, seq, heads)
    assert np.all(np.isfinite(got))
    np.testing.assert_allclose(got, _attn64(hot[:, :D], hot[:, D:2 * D], hot[:, 2 * D:], batch, seq, heads),
                               rtol=0, atol=5e-4)


def test_attention_causality_and_batch_independence():
    batch, seq, heads, dk = 2, 12, 2, 8
    D = heads * dk
    qkv = _qkv(batch, seq, heads, dk, seed=10)
    base = R.causal_attention(qkv, batch, seq, heads)
    cut = 5
    fut = qkv.copy()
    g = _gen(11)
    for b in range(batch):
        fut[b * seq + cut + 1:(b + 1) * seq, D:] = g.standard_normal(((seq - cut - 1), 2 * D)) * 5
    got = R.causal_attention(fut, batch, seq, heads)
    for b in range(batch):
        rows = slice(b * seq, b * seq + cut + 1)
        np.testing.assert_array_equal(got[rows], base[rows])
        assert not np.array_equal(got[b * seq + cut + 1:(b + 1) * seq], base[b * seq + cut + 1:(b + 1) * seq])
    other = qkv.copy()
    other[seq:] = g.standard_normal((seq, 3 * D))
    np.testing.assert_array_equal(R.causal_attention(other, batch, seq, heads)[:seq], base[:seq])


def _attn_mutant(qkv, batch, seq, heads, variant):
    D = qkv.shape[1] // 3
    dk = D // heads
    split = (batch, seq, dk, heads) if variant == "heads_interleaved" else (batch, seq, heads, dk)

    def heads_of(cols):
        t = qkv[:, cols].astype(f64).reshape(split)
        return t.transpose(0, 3, 1, 2) if variant == "heads_interleaved" else t.transpose(0, 2, 1, 3)

    q, k, v = heads_of(slice(0, D)), heads_of(slice(D, 2 * D)), heads_of(slice(2 * D, 3 * D))
    scale = 1.0 / dk if variant == "scale_dk" else 1.0 / math.sqrt(dk)
    s = q @ k.transpose(0, 1, 3, 2) * scale
    i, j = np.arange(seq)[:, None], np.arange(seq)[None, :]
    allowed = (j < i) | ((i == 0) & (j == 0)) if variant == "strict_mask" else (j <= i)
    s = s + np.where(allowed, 0.0, -1e9)
    axis = -2 if variant == "softmax_over_queries" else -1
    e = np.exp(s - s.max(axis=axis, keepdims=True))
    p = e / e.sum(axis=axis, keepdims=True)
    o = p @ v
    o = o.transpose(0, 2, 3, 1) if variant == "heads_interleaved" else o.transpose(0, 2, 1, 3)
    return o.reshape(batch * seq, D).astype(f32)


@pytest.mark.parametrize("variant", ["scale_dk", "strict_mask", "heads_interleaved", "softmax_over_queries"])
def test_attention_mutants_are_caught(variant):
    batch, seq, heads, dk = 2, 7, 3, 4
    D = heads * dk
    qkv = _qkv(batch, seq, heads, dk, seed=seq * 31 + heads)
    want = _attn64(qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:], batch, seq, heads)
    assert not np.allclose(_attn_mutant(qkv, batch, seq, heads, variant), want, rtol=0, atol=2e-6)
    # the unmutated copy passes the same check, so the check itself is sound
    np.testing.assert_allclose(_attn_mutant(qkv, batch, seq, heads, "none"), want, rtol=0, atol=2e-6)


# ---------------------------------------------------------------------------
# The whole forward, and the fused QKV Linear
# ---------------------------------------------------------------------------

def _tiny_weights(seed):
    from kansaiml_amd.charlm import CharLMWeights
    w = CharLMWeights(vocab=11, d_model=12, heads=3, layers=2, d_ff=20, seq=6, seed=seed, std=0.3, bias_std=0.1)
    g = _gen(seed + 1)
    for p in w.blocks:  # non-trivial LayerNorm affines
        for n in ("ln1_w", "ln1_b", "ln2_w", "ln2_b"):
            p[n] = (p[n] + 0.2 * g.standard_normal(12)).astype(f32)
    w.lnf_w = (w.lnf_w + 0.2 * g.standard_normal(12)).astype(f32)
    w.lnf_b = (w.lnf_b + 0.2 * g.standard_normal(12)).astype(f32)
    return w


@pytest.mark.parametrize("seq", [6, 4])
def test_fp32_forward_vs_binary64_composition(seq):
    """seq 6 fills the position table (causal mask); seq 4 runs unmasked."""
    w = _tiny_weights(3)
    ids = _gen(4).integers(0, 11, (2, seq))
    got = R.forward(w, ids, quantized=False).astype(f64)
    want = _forward64(w, ids)
    assert np.max(np.abs(got - want)) <= 2e-5 * (1.0 + np.max(np.abs(want)))


@pytest.mark.parametrize("mutant", ["gelu_tanh", "attention_scale_dk", "ln_affine_dropped", "no_position"])
def test_forward_mutants_are_caught(mutant, monkeypatch):
    w = _tiny_weights(3)
    ids = _gen(4).integers(0, 11, (2, 6))
    if mutant == "gelu_tanh":
        monkeypatch.setattr(R, "gelu", lambda x: (0.5 * x * (1 + np.tanh(math.sqrt(2 / math.pi) *
                                                                          (x + 0.044715 * x ** 3)))).astype(f32))
    elif mutant == "attention_scale_dk":
        monkeypatch.setattr(R, "attention", lambda qkv, b, s, h, causal=True: _attn_mutant(qkv, b, s, h, "scale_dk"))
    elif mutant == "ln_affine_dropped":
        ln = R.layer_norm
        monkeypatch.setattr(R, "layer_norm", lambda x, a, b: ln(x, np.ones_like(a), np.zeros_like(b)))
    elif mutant == "no_position":
        w.pos = np.zeros_like(w.pos)
    got = R.forward(w, ids, quantized=False).astype(f64)
    if mutant == "no_position":
        want = _forward64(_tiny_weights(3), ids)
    else:
        want = _forward64(w, ids)
    assert np.max(np.abs(got - want)) > 2e-5 * (1.0 + np.max(np.abs(want)))


def test_fused_qkv_linear_equals_three_linears():
    """One int8 Linear over [w_q | w_k | w_v] is bit-identical to three: the
    activation scale is per tensor and the weight scales per output column."""
    g = _gen(12)
    h = g.standard_normal((40, 48)).astype(f32)
    ws = [(g.standard_normal((48, 48)) * 0.05).astype(f32) for _ in range(3)]
    fused = R.linear(h, np.concatenate(ws, axis=1), None, True)
    split = np.concatenate([R.linear(h, wi, None, True) for wi in ws], axis=1)
    np.testing.assert_array_equal(fused.view(np.uint32), split.view(np.uint32))


@pytest.mark.parametrize("act_granularity", ["tensor", "row"])
def test_quantized_forward_tracks_fp32(act_granularity):
    """The int8 forward differs from the fp32 one only by quantization error:
    close, but not identical (so the quantized Linears are really used)."""
    w = _tiny_weights(5)
    ids = _gen(6).integers(0, 11, (2, 6))
    q = R.forward(w, ids, quantized=True, act_granularity=act_granularity).astype(f64)
    f = R.forward(w, ids, quantized=False).astype(f64)
    err = np.max(np.abs(q - f)) / np.max(np.abs(f))
    assert 0 < err < 0.1


def test_per_token_linear_is_row_by_row():
    """A per-row activation scale makes each output row depend on its own
    input row only: the Linear of a stack equals the stack of each row's
    Linear, bit for bit, and differs from the per-tensor Linear."""
    g = _gen(13)
    x = (g.standard_normal((6, 32)) * g.uniform(0.1, 10, (6, 1))).astype(f32)
    wt = (g.standard_normal((32, 24)) * 0.1).astype(f32)
    b = g.standard_normal(24).astype(f32)
    whole = R.linear(x, wt, b, True, "row")
    rows = np.concatenate([R.linear(x[i:i + 1], wt, b, True, "tensor") for i in range(6)])
    np.testing.assert_array_equal(whole.view(np.uint32), rows.view(np.uint32))
    assert not np.array_equal(whole, R.linear(x, wt, b, True, "tensor"))
