"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each check is chosen so a plausible mistake in the oracle fails it:
  * golden fixtures computed by CPython's own round()/binary64 floats
    (tests/golden/make_golden.py), including exact ties -> even;
  * the reference test's own known answers (tests/test_quantize.py:41-59,
    66-72 of the reference): range, error <= scale/2 + 1e-6, zero -> 0,
    exactly 4.00x smaller;
  * brute force against the pure-Python restatement on random tiny inputs;
  * independent library routines: numpy int64 matmul for the int8 GEMM,
    numpy float64 for the epilogue, the reference's own compiled
    backend/cpu/src/Ops.cpp (oracle/_ref) for the fp32 i-k-j loop;
  * mutation checks: deliberately wrong oracles (planted here, on the CPU)
    must fail the same fixtures.
"""

import math
import random

import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

from conftest import golden_names, load_golden

from oracle import oracle as O


# ---------------------------------------------------------------------------
# Quantize / dequantize against the golden fixtures
# ---------------------------------------------------------------------------

PER_TENSOR = ["ref_test_quantize_1000", "zero_maps_to_zero", "ties_scale_one", "ties_scale_half", "near_ties",
              "all_zero"] + golden_names("per_tensor_n")


@pytest.mark.parametrize("name", PER_TENSOR)
def test_per_tensor_matches_golden(name):
    g = load_golden(name)
    q, s = O.ko_quantize_tensor(g["x"])
    assert s == g["scale"][0]
    np.testing.assert_array_equal(q, g["q"])
    d = O.ko_dequantize_tensor(q, s)
    np.testing.assert_array_equal(d.view(np.uint32), g["deq"].view(np.uint32))


@pytest.mark.parametrize("name", golden_names("per_row_"))
def test_per_row_matches_golden(name):
    g = load_golden(name)
    q, s = O.ko_quantize_rows(g["x"])
    np.testing.assert_array_equal(s, g["scale"])
    np.testing.assert_array_equal(q, g["q"])
    d = O.ko_dequantize_rows(q, s)
    np.testing.assert_array_equal(d.view(np.uint32), g["deq"].view(np.uint32))


@pytest.mark.parametrize("name", golden_names("per_col_"))
def test_per_col_packed_matches_golden(name):
    g = load_golden(name)
    q, s = O.ko_quantize_cols_packed(g["w"])
    np.testing.assert_array_equal(s, g["scale"])
    np.testing.assert_array_equal(q, g["q_packed"])


@pytest.mark.parametrize("name", ["ref_test_quantize_1000"] + golden_names("per_col_"))
def test_per_tensor_packed_is_transposed_per_tensor(name):
    """ko_quantize_tensor_packed is its own loop: pin it to the per-tensor
    quantize (itself pinned by the fixtures above) of the same [k, n] weight,
    transposed into the packed [n, k] layout -- codes and scale."""
    g = load_golden(name)
    w = g["w"] if "w" in g else g["x"].reshape(40, 25)
    q, s = O.ko_quantize_tensor_packed(w)
    qt, st_ = O.ko_quantize_tensor(w)
    assert s == st_
    np.testing.assert_array_equal(q, qt.T)


def test_ties_go_to_even():
    g = load_golden("ties_scale_one")
    q, s = O.ko_quantize_tensor(g["x"])
    assert s == 1.0
    expect = {0.5: 0, 1.5: 2, 2.5: 2, -0.5: 0, -1.5: -2, -2.5: -2, 3.5: 4, 126.5: 126, -126.5: -126, 100.5: 100}
    for v, e in expect.items():
        assert q[list(g["x"]).index(np.float32(v))] == e, v


# ---------------------------------------------------------------------------
# The reference test's own checks (tests/test_quantize.py:41-72)
# ---------------------------------------------------------------------------

def test_reference_known_answers():
    rng = random.Random(0)
    vals = np.array([rng.uniform(-3.0, 3.0) for _ in range(1000)], np.float32)
    q, scale = O.ko_quantize_tensor(vals)
    assert q.min() >= -127 and q.max() <= 127
    rec = O.ko_dequantize_tensor(q, scale)
    max_err = float(np.max(np.abs(vals.astype(np.float64) - rec.astype(np.float64))))
    assert max_err <= scale / 2 + 1e-6
    qz, _ = O.ko_quantize_tensor(np.array([0.0, 1.0, -1.0], np.float32))
    assert qz[0] == 0
    big = np.random.Generator(np.random.PCG64(1)).standard_normal((256, 256)).astype(np.float32)
    qb, _ = O.ko_quantize_tensor(big)
    assert (4 * big.size) / qb.nbytes == 4.0


def test_nonfinite_rejected():
    for bad in (np.nan, np.inf, -np.inf):
        x = np.array([1.0, bad, 2.0], np.float32)
        with pytest.raises(O.NonFiniteError):
            O.ko_quantize_tensor(x)
        with pytest.raises(O.NonFiniteError):
            O.ko_quantize_rows(x.reshape(1, 3))


def test_never_minus_128():
    x = np.array([-1.0, 1.0, -0.99999994], np.float32)
    q, _ = O.ko_quantize_tensor(x)
    assert q.min() == -127


# ---------------------------------------------------------------------------
# Brute force against the pure-Python restatement (CPython round())
# ---------------------------------------------------------------------------

@settings(max_examples=200, deadline=None)
@given(st.lists(st.floats(min_value=-1e6, max_value=1e6, allow_nan=False, width=32), min_size=1, max_size=40))
def test_c_oracle_equals_python_round(vals):
    x = np.array(vals, np.float32)
    q, s = O.ko_quantize_tensor(x)
    pq, ps = O.py_quantize_symmetric([float(v) for v in x])
    assert s == ps
    assert q.tolist() == pq
    d = O.ko_dequantize_tensor(q, s)
    assert d.tolist() == O.py_dequantize(pq, ps)


@settings(max_examples=100, deadline=None)
@given(st.integers(1, 127), st.integers(-127, 127), st.integers(0, 3))
def test_exact_multiples_of_scale(m_int, k, shift):
    """v = k*s / 2**shift hits exact quotients (and exact halves when
    shift = 1): the quotient is exact in binary64, so round() decides."""
    m = float(m_int) / (1 << shift)
    s = m / 127.0
    vals = [m] + [float(np.float32(k * s / 2))]
    x = np.array(vals, np.float32)
    q, sc = O.ko_quantize_tensor(x)
    pq, ps = O.py_quantize_symmetric([float(v) for v in x])
    assert sc == ps and q.tolist() == pq


# ---------------------------------------------------------------------------
# int8 GEMM and epilogue
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name", golden_names("gemm_i8_"))
def test_gemm_and_epilogue_match_golden(name):
    g = load_golden(name)
    acc = O.ko_gemm_i8(g["a"], g["bt"])
    np.testing.assert_array_equal(acc, g["acc"])
    out = O.ko_epilogue(acc, g["sa"], g["sb"], g["bias"])
    np.testing.assert_array_equal(out.view(np.uint32), g["out"].view(np.uint32))


def test_gemm_vs_numpy_int64():
    gen = np.random.Generator(np.random.PCG64(3))
    for M, N, K in ((64, 96, 256), (7, 13, 1000), (128, 128, 4096)):
        a = gen.integers(-127, 128, (M, K), dtype=np.int8)
        b = gen.integers(-127, 128, (N, K), dtype=np.int8)
        ref = a.astype(np.int64) @ b.astype(np.int64).T
        np.testing.assert_array_equal(O.ko_gemm_i8(a, b).astype(np.int64), ref)


def test_gemm_extreme_accumulator():
    # all -127 * -127 at K = 8192: 132,128,768 < 2**31, exact.
    K = 8192
    a = np.full((2, K), -127, np.int8)
    b = np.full((3, K), -127, np.int8)
    acc = O.ko_gemm_i8(a, b)
    assert (acc == 127 * 127 * K).all()


def test_epilogue_vs_numpy_f64():
    gen = np.random.Generator(np.random.PCG64(4))
    M, N = 37, 53
    acc = gen.integers(-2_000_000, 2_000_000, (M, N), dtype=np.int32)
    sa = gen.uniform(1e-4, 1e-1, M)
    sb = gen.uniform(1e-4, 1e-1, N)
    bias = gen.standard_normal(N).astype(np.float32)
    out = O.ko_epilogue(acc, sa, sb, bias)
    ref = (acc.astype(np.float64) * (sa[:, None] * sb[None, :])).astype(np.float32) + bias[None, :]
    np.testing.assert_array_equal(out.view(np.uint32), ref.view(np.uint32))
    # the 1e-5 relative bar against the exact real value
    exact = acc.astype(np.float64) * sa[:, None] * sb[None, :] + bias.astype(np.float64)[None, :]
    bound = 1e-5 * (np.abs(acc) * sa[:, None] * sb[None, :] + np.abs(bias)[None, :]) + 1e-30
    assert (np.abs(out - exact) <= bound).all()


# ---------------------------------------------------------------------------
# fp32 matmul: the restated i-k-j loop against the reference's own compiled
# Ops.cpp, and against numpy float64
# ---------------------------------------------------------------------------

@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("shape", [(17, 19, 15), (100, 77, 50), (1, 1, 1), (64, 512, 512)])
def test_matmul_f32_equals_reference_build(shape):
    M, K, N = shape
    gen = np.random.Generator(np.random.PCG64(9))
    a = gen.standard_normal((M, K)).astype(np.float32)
    b = gen.standard_normal((K, N)).astype(np.float32)
    mine = O.ko_matmul_f32(a, b)
    theirs = O.ref_matmul(a, b)
    np.testing.assert_array_equal(mine.view(np.uint32), theirs.view(np.uint32))
    bias = gen.standard_normal(N).astype(np.float32)
    np.testing.assert_array_equal(O.ko_add_bias(mine, bias), O.ref_add_bias(theirs, bias))
    ref64 = a.astype(np.float64) @ b.astype(np.float64)
    tol = 4 * K * np.finfo(np.float32).eps * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
    assert (np.abs(mine - ref64) <= tol + 1e-30).all()


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
def test_reference_batched_matmul_is_the_2d_matmul_of_its_rows():
    """The reference's batched matmul with a shared 2-D right operand
    (Tensor.cpp:364-393 -> Ops.cpp:427-437) and its general broadcast add of
    a bias (Ops.cpp:121-125) equal, bit for bit, the 2-D matmul and bias add
    of the flattened [batch * M, K] rows: what the HIP path computes for a
    [batch, seq, d] activation."""
    gen = np.random.Generator(np.random.PCG64(21))
    a = gen.standard_normal((4, 16, 96)).astype(np.float32)
    b = gen.standard_normal((96, 40)).astype(np.float32)
    bias = gen.standard_normal(40).astype(np.float32)
    batched = O.ref_batched_matmul(a, b)
    flat = O.ref_matmul(a.reshape(-1, 96), b).reshape(4, 16, 40)
    np.testing.assert_array_equal(batched.view(np.uint32), flat.view(np.uint32))
    np.testing.assert_array_equal(O.ref_add_broadcast(batched, bias).view(np.uint32),
                                  O.ref_add_bias(flat.reshape(-1, 40), bias).reshape(4, 16, 40).view(np.uint32))
    # the shim passes the batch axis through: a batch of distinct matrices
    # is not the first matrix repeated
    assert not np.array_equal(batched[1], batched[0])


# ---------------------------------------------------------------------------
# Mutation checks: a plausible mistake planted in a copy of the oracle must
# fail the fixtures above.
# ---------------------------------------------------------------------------

def _mut_quantize(flat, variant):
    m = max((abs(v) for v in flat), default=0.0)
    if variant == "scale_128":
        scale = m / 128.0 if m > 0 else 1.0
    else:
        scale = m / 127.0 if m > 0 else 1.0
    out = []
    for v in flat:
        if variant == "half_away":
            r = math.floor(abs(v / scale) + 0.5) * (1 if v >= 0 else -1)
        elif variant == "fp32_divide":
            r = round(float(np.float32(np.float32(v) / np.float32(scale))))
        elif variant == "fp32_reciprocal":
            r = round(float(np.float32(v) * np.float32(1.0 / scale)))
        elif variant == "clamp_128":
            r = round(v / scale)
            out.append(max(-128, min(127, r)))
            continue
        else:
            r = round(v / scale)
        out.append(max(-127, min(127, r)))
    return out, scale


@pytest.mark.parametrize("variant", ["half_away", "scale_128", "fp32_divide", "fp32_reciprocal"])
def test_mutants_are_caught(variant):
    caught = False
    for name in PER_TENSOR + ["per_tensor_n100000"]:
        g = load_golden(name)
        q, s = _mut_quantize([float(v) for v in g["x"]], variant)
        if q != g["q"].tolist() or s != g["scale"][0]:
            caught = True
            break
    assert caught, f"mutant {variant} passed every fixture"


def test_mutant_transposed_pack_caught():
    g = load_golden("per_col_19x15")
    q, s = O.ko_quantize_cols_packed(g["w"])
    assert not np.array_equal(q.reshape(-1), g["q_packed"].T.reshape(-1))


def test_mutant_epilogue_order_caught():
    """Applying the scales one at a time (acc*sa then *sb) instead of
    acc*(sa*sb) is a different rounding; the golden epilogue must notice."""
    diffs = 0
    for name in golden_names("gemm_i8_"):
        g = load_golden(name)
        sa = np.broadcast_to(g["sa"][:, None] if g["sa"].size > 1 else g["sa"], g["acc"].shape)
        sb = np.broadcast_to(g["sb"][None, :] if g["sb"].size > 1 else g["sb"], g["acc"].shape)
        wrong = ((g["acc"].astype(np.float64) * sa) * sb).astype(np.float32) + g["bias"][None, :]
        diffs += int((wrong.view(np.uint32) != g["out"].view(np.uint32)).sum())
    assert diffs > 0
