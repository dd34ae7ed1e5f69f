"""The GELU arithmetic of the HIP kernels (kh::gelu, kansaiml_amd/csrc/kh_act.h),
pinned on the CPU.

The kernels evaluate GELU(x) = x * Phi(x) (the reference's cpu::gelu,
backend/cpu/src/Ops.cpp:250-256: x * 0.5 * (1 + erf(x / sqrt(2)))) through a
fitted erfc.  These tests (1) regenerate the fit with gen_gelu_coeffs.py and
check that the header carries exactly its binary32 coefficients, and (2)
evaluate the header's formula operation by operation in binary32 (numpy,
each operation rounded) against binary64 GELU from scipy's erfc, which the
formula shares nothing with: a wrong coefficient, a dropped term or a wrong
sign fails the bound.  The GPU tests check the kernels themselves against
binary64 (tests/test_gpu_charlm.py::test_gelu)."""

import os
import re
import sys

import numpy as np
import pytest
from scipy.special import erfc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "kansaiml_amd", "csrc")
f32 = np.float32


def _header_constants():
    src = open(os.path.join(CSRC, "kh_act.h")).read()
    body = src[src.index("float gelu(float x)"):]
    body = body[:body.index("\n}\n")]
    coef = [float(v) for v in re.findall(r"fmaf\(e, s, (-?[0-9.]+)f\)", body)]
    first = float(re.search(r"float e = (-?[0-9.]+)f;", body).group(1))
    mid = float(re.search(r"h - ([0-9.]+)f;", body).group(1))
    inv_sqrt2 = float(re.search(r"fmaf\(a, ([0-9.]+)f, 2\.0f\)", body).group(1))
    half_log2e = float(re.search(r"fmaf\(-a, a \* ([0-9.]+)f, e\)", body).group(1))
    return [first] + coef, mid, inv_sqrt2, half_log2e


def _fma(a, b, c):
    # binary64 product and sum, then one rounding: exact for these operands
    # except on double-rounding ties (far below the bounds checked here)
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(f32)


def _gelu_binary32(x):
    """kh::gelu evaluated as the kernel does, one rounding per operation
    (reciprocal and exp2 correctly rounded; the hardware's are within 1 ulp)."""
    coef, mid, inv_sqrt2, half_log2e = _header_constants()
    x = np.asarray(x, f32)
    with np.errstate(all="ignore"):
        a = np.abs(x)
        h = (1.0 / _fma(a, np.full_like(a, inv_sqrt2), np.full_like(a, 2.0)).astype(np.float64)).astype(f32)
        s = (h - f32(mid)).astype(f32)
        e = np.full_like(a, f32(coef[0]))
        for c in coef[1:]:
            e = _fma(e, s, np.full_like(a, f32(c)))
        e = _fma(-a, (a * f32(half_log2e)).astype(f32), e)
        p = np.exp2(e.astype(np.float64)).astype(f32)
        cdf = np.where(x >= 0, _fma(-h, p, np.ones_like(a)), (h * p).astype(f32))
        return (x * cdf).astype(f32)


def _gelu64(x):
    x = np.asarray(x, np.float64)
    return x * 0.5 * erfc(-x / np.sqrt(2.0))


def test_header_coefficients_are_the_fit():
    sys.path.insert(0, CSRC)
    try:
        import gen_gelu_coeffs as G
    finally:
        sys.path.remove(CSRC)
    q, err = G.coefficients()
    assert err < 2e-8
    coef, mid, inv_sqrt2, half_log2e = _header_constants()
    assert coef == [float(q[i]) for i in range(G.DEGREE, -1, -1)]
    assert mid == G.H_MID
    assert f32(inv_sqrt2) == f32(1 / np.sqrt(2.0))
    assert f32(half_log2e) == f32(np.log2(np.e) / 2)


def test_binary32_formula_against_binary64():
    x = np.concatenate([np.linspace(-12, 12, 1_200_001, dtype=f32),
                        (10.0 ** np.linspace(-30, 30, 4001)).astype(f32),
                        -(10.0 ** np.linspace(-30, 30, 4001)).astype(f32)])
    got = _gelu_binary32(x).astype(np.float64)
    want = _gelu64(x)
    err = np.abs(got - want) / np.maximum(1.0, np.abs(x.astype(np.float64)))
    assert err.max() < 1.2e-7, (err.max(), x[np.argmax(err)])
    # relative accuracy where the value is not tiny (the negative tail keeps
    # the relative error that 1 + erf would lose)
    big = np.abs(want) > 1e-6
    assert (np.abs(got - want)[big] / np.abs(want[big])).max() < 5e-6


def test_binary32_formula_special_values():
    x = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e30, -1e30, 3e38, -3e38], f32)
    g = _gelu_binary32(x)
    assert g[0] == 0 and not np.signbit(g[0]) and g[1] == 0 and np.signbit(g[1])
    assert g[2] == np.inf and np.isnan(g[3]) and np.isnan(g[4])  # -inf * 0, as the reference formula
    assert g[5] == f32(1e30) and g[7] == f32(3e38)
    assert g[6] == 0 and g[8] == 0


@pytest.mark.parametrize("mutant", ["coef", "dropped", "sign", "mid"])
def test_formula_mutants_fail(mutant, monkeypatch):
    """A coefficient 1 % off, a dropped term, the a^2 term's sign and a
    shifted centre each break the bound the formula meets."""
    coef, mid, inv_sqrt2, half_log2e = _header_constants()
    coef = list(coef)
    if mutant == "coef":
        coef[4] *= 1.01
    elif mutant == "dropped":
        coef[7] = 0.0
    elif mutant == "sign":
        half_log2e = -half_log2e
    else:
        mid = mid + 1e-3
    monkeypatch.setattr(sys.modules[__name__], "_header_constants", lambda: (coef, mid, inv_sqrt2, half_log2e))
    x = np.linspace(-6, 6, 20001, dtype=f32)
    with np.errstate(all="ignore"):
        err = np.abs(_gelu_binary32(x).astype(np.float64) - _gelu64(x)) / np.maximum(1.0, np.abs(x))
    assert np.nan_to_num(err, nan=1.0).max() > 1.2e-7
