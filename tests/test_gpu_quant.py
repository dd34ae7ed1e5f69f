"""GPU parity: quantize / dequantize kernels vs the golden fixtures and the
CPU oracle.  Bar: bit-exact int8 codes, bit-exact binary64 scales and
bit-exact dequantized binary32 values (python/kansai/quantize.py:66-76 of
the reference; the reference test's own inputs are in the fixtures)."""

import numpy as np
import pytest

from conftest import golden_names, load_golden
from oracle import oracle as O

pytestmark = pytest.mark.gpu

PER_TENSOR = ["ref_test_quantize_1000", "zero_maps_to_zero", "ties_scale_one", "ties_scale_half", "near_ties",
              "all_zero"] + golden_names("per_tensor_n")


@pytest.fixture(scope="module")
def hip():
    from kansaiml_amd import hip as H
    from kansaiml_amd.device import DeviceTensor
    assert H.available(), "no gfx950 device"
    return H, DeviceTensor


def bits32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("name", PER_TENSOR)
def test_quantize_tensor_golden(hip, name):
    H, D = hip
    g = load_golden(name)
    x = D.from_host(g["x"])
    q, s = H.quantize_tensor(x)
    np.testing.assert_array_equal(q.numpy(), g["q"])
    assert s.numpy()[0] == g["scale"][0]
    d = H.dequantize_tensor(q, s)
    np.testing.assert_array_equal(bits32(d.numpy()), bits32(g["deq"]))


@pytest.mark.parametrize("name", golden_names("per_row_"))
def test_quantize_rows_golden(hip, name):
    H, D = hip
    g = load_golden(name)
    x = D.from_host(g["x"])
    q, s = H.quantize_rows(x)
    np.testing.assert_array_equal(q.numpy(), g["q"])
    np.testing.assert_array_equal(s.numpy(), g["scale"])
    d = H.dequantize_rows(q, s)
    np.testing.assert_array_equal(bits32(d.numpy()), bits32(g["deq"]))


@pytest.mark.parametrize("name", golden_names("per_col_"))
def test_quantize_cols_packed_golden(hip, name):
    H, D = hip
    g = load_golden(name)
    w = D.from_host(g["w"])
    q, s = H.quantize_cols_packed(w)
    np.testing.assert_array_equal(q.numpy(), g["q_packed"])
    np.testing.assert_array_equal(s.numpy(), g["scale"])


def _outlier_matrix(rows, cols, seed, frac=0.001):
    gen = np.random.Generator(np.random.PCG64(seed))
    x = gen.standard_normal((rows, cols), dtype=np.float32)
    n_out = max(1, int(rows * cols * frac))
    idx = gen.choice(rows * cols, size=n_out, replace=False)
    x.reshape(-1)[idx] = np.where(gen.random(n_out) < 0.5, -50.0, 50.0).astype(np.float32)
    return x


# Row lengths covering every per-row kernel variant: register-resident for
# cols <= 256, 1024, 4096, 16384, 32768 (multiples of 4) and the two-pass
# kernel for cols % 4 != 0 and cols > 32768.
@pytest.mark.parametrize("rows,cols", [(7, 8), (33, 256), (9, 1000), (64, 1024), (5, 3000), (16, 4096),
                                       (3, 16384), (2, 32768), (2, 40000), (11, 33), (4, 4099),
                                       (5, 384), (6, 512), (7, 1536), (3, 1028), (9, 2048), (1, 1200)])
def test_quantize_rows_vs_oracle(hip, rows, cols):
    H, D = hip
    x = _outlier_matrix(rows, cols, seed=rows * 7919 + cols)
    x[0, :] = 0.0  # an all-zero row: scale 1.0
    eq, es = O.ko_quantize_rows(x)
    q, s = H.quantize_rows(D.from_host(x))
    np.testing.assert_array_equal(q.numpy(), eq)
    np.testing.assert_array_equal(s.numpy(), es)
    np.testing.assert_array_equal(bits32(H.dequantize_rows(q, s).numpy()), bits32(O.ko_dequantize_rows(eq, es)))


# n <= 65536 (float4-aligned buffers) takes the one-launch kernel, larger n the
# two-pass path.
@pytest.mark.parametrize("n", [1, 3, 4, 5, 1023, 32768, 65535, 65536, 65537, 1_000_003, 16_777_216])
def test_quantize_tensor_vs_oracle(hip, n):
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(n))
    x = gen.standard_normal(n, dtype=np.float32) * np.float32(3.0)
    eq, es = O.ko_quantize_tensor(x)
    q, s = H.quantize_tensor(D.from_host(x))
    np.testing.assert_array_equal(q.numpy(), eq)
    assert s.numpy()[0] == es
    np.testing.assert_array_equal(bits32(H.dequantize_tensor(q, s).numpy()), bits32(O.ko_dequantize_tensor(eq, es)))


@pytest.mark.parametrize("count", [1, 3, 255, 2049, 5000])
def test_quantize_tensor_parts_any_partial_count(hip, count):
    """kh_quantize_tensor_parts takes the tensor's scale from any number of
    producer partials: one, fewer than a workgroup has threads, and several
    rounds of eight loads per thread, with the largest partial first, in the
    middle or last.  Every other partial is |0.25|, below the tensor's
    absmax, so a partial left out of the maximum changes the scale and every
    code."""
    from kansaiml_amd import _native as Nn
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(count + 17))
    x = gen.standard_normal(70001, dtype=np.float32)
    eq, es = O.ko_quantize_tensor(x)
    top = np.abs(x).max().astype(np.float32).view(np.uint32)
    xd = D.from_host(x)
    for pos in sorted({0, count // 2, count - 1}):
        print(f"partials count={count} max at {pos}", flush=True)
        parts = np.full(count, np.float32(0.25).view(np.uint32), np.uint32)
        parts[pos] = top
        pd = D.from_host(parts.view(np.int32))
        q, sc = D([x.size], "int8"), D([1], "float64")
        Nn.call("kh_quantize_tensor_parts", xd.ptr, x.size, pd.ptr, count, q.ptr, sc.ptr)
        np.testing.assert_array_equal(q.numpy(), eq)
        assert sc.numpy()[0] == es


@pytest.mark.parametrize("k,n", [(512, 512), (4096, 4096), (384, 1536), (1536, 384), (19, 15), (100, 65)])
def test_quantize_weight_packed_vs_oracle(hip, k, n):
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(k * 31 + n))
    w = (gen.standard_normal((k, n), dtype=np.float32) * np.float32(0.02))
    cols = gen.choice(n, size=max(1, n // 200), replace=False)
    w[:, cols] *= np.float32(20.0)
    wd = D.from_host(w)
    eq, es = O.ko_quantize_cols_packed(w)
    q, s = H.quantize_cols_packed(wd)
    np.testing.assert_array_equal(q.numpy(), eq)
    np.testing.assert_array_equal(s.numpy(), es)
    deq = H.dequantize_packed(q, s).numpy()
    expect = (eq.T.astype(np.float64) * es[None, :]).astype(np.float32)
    np.testing.assert_array_equal(bits32(deq), bits32(expect))
    eq1, es1 = O.ko_quantize_tensor_packed(w)
    q1, s1 = H.quantize_tensor_packed(wd)
    np.testing.assert_array_equal(q1.numpy(), eq1)
    assert s1.numpy()[0] == es1


def test_misaligned_pointers_take_exact_generic_path(hip):
    """Offsets that break 16-byte alignment route to the scalar kernels."""
    H, D = hip
    x = _outlier_matrix(6, 260, seed=5)
    buf = D.from_host(np.concatenate([np.zeros(1, np.float32), x.reshape(-1)]))
    view = D.__new__(D)
    import ctypes
    view.ptr = ctypes.c_void_p(buf.addr + 4)
    view.shape, view.dtype, view.nbytes, view._owned = [6, 260], "float32", 6 * 260 * 4, False
    eq, es = O.ko_quantize_rows(x)
    q, s = H.quantize_rows(view)
    np.testing.assert_array_equal(q.numpy(), eq)
    np.testing.assert_array_equal(s.numpy(), es)
    q1, s1 = H.quantize_tensor(view)
    eq1, es1 = O.ko_quantize_tensor(x)
    np.testing.assert_array_equal(q1.numpy(), eq1)
    assert s1.numpy()[0] == es1
    del buf


def test_tiny_and_subnormal_rows(hip):
    """Rows whose max is below 2^-64 take the exact path throughout;
    subnormal fp32 inputs must not be flushed."""
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(77))
    x = gen.standard_normal((4, 64), dtype=np.float32)
    x[0] *= np.float32(1e-30)
    x[1] *= np.float32(1e-39)      # subnormal
    x[2, :] = np.float32(1.4e-45)   # smallest subnormal
    x[2, ::2] = np.float32(-1.4e-45)
    x[3] *= np.float32(2.0 ** -70)
    eq, es = O.ko_quantize_rows(x)
    q, s = H.quantize_rows(D.from_host(x))
    np.testing.assert_array_equal(q.numpy(), eq)
    np.testing.assert_array_equal(s.numpy(), es)


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_nonfinite_raises_value_error(hip, bad):
    H, D = hip
    from kansaiml_amd import _native as N
    x = np.ones((3, 8), np.float32)
    x[1, 5] = bad
    xd = D.from_host(x)
    q, s = H.quantize_rows(xd)
    with pytest.raises(ValueError):
        N.synchronize()
    sc = s.numpy()
    assert np.isnan(sc[1]) and sc[0] == 1.0 / 127.0
    assert (q.numpy()[1] == 0).all()
    H.quantize_tensor(xd)
    with pytest.raises(ValueError):
        N.synchronize()
    N.synchronize()  # the fault word was cleared


def test_c2_full_size_roundtrip(hip):
    """Config C2 at full size: [16384, 16384] fp32 (1 GiB) ~N(0,1), 0.1% of
    entries +-50, per-row scales.  Every row's codes, scale and dequantized
    values bit-exact against the oracle (in slabs of 2048 rows), plus the
    size-independent properties."""
    H, D = hip
    rows = cols = 16384
    x = _outlier_matrix(rows, cols, seed=2024)
    xd = D.from_host(x)
    q, s = H.quantize_rows(xd)
    d = H.dequantize_rows(q, s)
    qh, sh, dh = q.numpy(), s.numpy(), d.numpy()
    for r0 in range(0, rows, 2048):
        sl = slice(r0, r0 + 2048)
        eq, es = O.ko_quantize_rows(x[sl])
        np.testing.assert_array_equal(qh[sl], eq, err_msg=f"codes, rows {r0}..")
        np.testing.assert_array_equal(sh[sl], es, err_msg=f"scales, rows {r0}..")
        np.testing.assert_array_equal(bits32(dh[sl]), bits32(O.ko_dequantize_rows(eq, es)),
                                      err_msg=f"dequantized, rows {r0}..")
        del eq, es
    # properties over every row
    m = np.abs(x).max(axis=1).astype(np.float64)
    np.testing.assert_array_equal(sh, m / 127.0)
    assert qh.min() >= -127 and qh.max() <= 127
    assert (np.abs(qh).max(axis=1) == 127).all()
    # tests/test_quantize.py:53 of the reference: error <= scale/2 (+ the
    # binary32 rounding of the dequantized value, at most 1e-5 here).
    err = np.abs(x.astype(np.float64) - dh.astype(np.float64))
    assert (err <= sh[:, None] / 2 + 1e-5).all()
