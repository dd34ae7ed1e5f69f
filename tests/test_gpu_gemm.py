"""GPU parity: int8 GEMM (exact int32 accumulators, bit-exact fused
dequantize + bias epilogue) and the fp32 matmul (rounding-bound agreement
with the reference's own compiled i-k-j loop and with float64)."""

import numpy as np
import pytest

from conftest import golden_names, load_golden
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    from kansaiml_amd import hip as H
    from kansaiml_amd.device import DeviceTensor
    assert H.available(), "no gfx950 device"
    return H, DeviceTensor


def bits32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def run_gemm(H, D, a, bt, sa, sb, bias):
    out, acc = H.gemm_i8(D.from_host(a), D.from_host(bt), D.from_host(np.asarray(sa, np.float64)),
                         D.from_host(np.asarray(sb, np.float64)), D.from_host(bias) if bias is not None else None,
                         want_out=True, want_acc=True)
    return out.numpy(), acc.numpy()


@pytest.mark.parametrize("name", golden_names("gemm_i8_"))
def test_gemm_i8_golden(hip, name):
    H, D = hip
    g = load_golden(name)
    out, acc = run_gemm(H, D, g["a"], g["bt"], g["sa"], g["sb"], g["bias"])
    np.testing.assert_array_equal(acc, g["acc"])
    np.testing.assert_array_equal(bits32(out), bits32(g["out"]))


SHAPES = [
    (64, 512, 512),      # C1's int8 Linear
    (1, 1, 16), (1, 4096, 4096), (8, 4096, 4096), (32, 11008, 4096),  # C5 decode shapes
    (16384, 65, 384),    # C4 vocab head: the narrow-N kernel (N=65: a 1-column last tile)
    (2048, 1, 64), (2049, 16, 128), (4000, 100, 448), (3000, 128, 448), (2100, 17, 512),  # narrow-N kernel
    (256, 1536, 384), (256, 384, 1536),
    (129, 257, 80), (300, 200, 48), (2048, 2048, 512), (2304, 2176, 1024),
    (33, 40, 130), (100, 50, 77), (5, 7, 3),  # K % 16 != 0: byte-gather path
    (2, 100, 512), (17, 4096, 4096), (31, 64, 1024), (16, 16, 512), (5, 11008, 4096), (32, 40, 512),  # skinny
    (30, 8200, 2048), (20, 8216, 4096),  # skinny, 32 columns per workgroup, partial last workgroup
    (9, 40, 8192), (2, 33, 1536),       # skinny: a 16-step slice; a 3-step slice (chunk loop)
    (512, 768, 64), (768, 512, 192), (1024, 256, 4160),  # full-tile kernel: K % 64 == 0, K % 128 != 0
    (1000, 1000, 128), (257, 129, 64), (33, 300, 640),    # ping-pong kernel, partial tiles in M and N
    (16384, 1152, 384), (16384, 384, 1536),               # C4 QKV and fc2 shapes
    (8, 1024, 8192), (32, 512, 16384), (5, 100, 8192),    # skinny with K split over 4, 8, 8 workgroups
    (64, 2048, 8192), (17, 40, 12288),                    # split over 2; over 8 with 3 steps per wave
]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_gemm_i8_vs_oracle(hip, M, N, K):
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(M * 1_000_003 + N * 1009 + K))
    a = gen.integers(-127, 128, (M, K), dtype=np.int8)
    bt = gen.integers(-127, 128, (N, K), dtype=np.int8)
    sa = gen.uniform(1e-3, 5e-2, M)
    sb = gen.uniform(1e-3, 5e-2, N)
    bias = gen.standard_normal(N).astype(np.float32)
    out, acc = run_gemm(H, D, a, bt, sa, sb, bias)
    # check a row sample against the oracle when the full product is large
    rows = np.arange(M) if M * N * K <= 2 ** 31 else gen.choice(M, size=64, replace=False)
    eacc = O.ko_gemm_i8(a[rows], bt)
    np.testing.assert_array_equal(acc[rows], eacc)
    eout = O.ko_epilogue(eacc, sa[rows], sb, bias)
    np.testing.assert_array_equal(bits32(out[rows]), bits32(eout))


def test_gemm_i8_per_tensor_scales_and_no_bias(hip):
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(12))
    a = gen.integers(-127, 128, (200, 320), dtype=np.int8)
    bt = gen.integers(-127, 128, (96, 320), dtype=np.int8)
    out, acc = run_gemm(H, D, a, bt, [0.01], [0.02], None)
    eacc = O.ko_gemm_i8(a, bt)
    np.testing.assert_array_equal(acc, eacc)
    np.testing.assert_array_equal(bits32(out), bits32(O.ko_epilogue(eacc, [0.01], [0.02], None)))


@pytest.mark.parametrize("M,N", [(64, 128), (256, 256)])  # general and full-tile kernels
def test_gemm_i8_extreme_values(hip, M, N):
    """All -127: the largest accumulator magnitude, 127*127*K."""
    H, D = hip
    K = 8192
    a = np.full((M, K), -127, np.int8)
    bt = np.full((N, K), -127, np.int8)
    a[1] = 127
    _, acc = run_gemm(H, D, a, bt, [1.0], [1.0], None)
    assert (acc[0] == 127 * 127 * K).all() and (acc[1] == -127 * 127 * K).all()


def test_gemm_i8_c3a_full_size(hip):
    """Config C3a: M=N=K=8192, A,B uniform in [-127,127], per-tensor scales
    0.01/0.02, fused dequantize to fp32.  128 sampled rows are checked
    bit-exactly against the oracle (accumulators and outputs)."""
    H, D = hip
    M = N = K = 8192
    gen = np.random.Generator(np.random.PCG64(3))
    a = gen.integers(-127, 128, (M, K), dtype=np.int8)
    bt = gen.integers(-127, 128, (N, K), dtype=np.int8)
    out, acc = run_gemm(H, D, a, bt, [0.01], [0.02], None)
    rows = gen.choice(M, size=128, replace=False)
    eacc = O.ko_gemm_i8(a[rows], bt)
    np.testing.assert_array_equal(acc[rows], eacc)
    np.testing.assert_array_equal(bits32(out[rows]), bits32(O.ko_epilogue(eacc, [0.01], [0.02], None)))
    # column sample too (the tile grid's other axis)
    cols = gen.choice(N, size=64, replace=False)
    eacc_c = (a.astype(np.int64)[::97] @ bt[cols].astype(np.int64).T).astype(np.int32)
    np.testing.assert_array_equal(acc[::97][:, cols], eacc_c)
    # The bench's launch asks for the output alone, which takes the full-tile
    # kernel build (with the accumulators the general build runs); its
    # 256 MiB output goes out through non-temporal stores.  Every value must
    # equal the checked run's.
    fast, none = H.gemm_i8(D.from_host(a), D.from_host(bt), D.from_host(np.array([0.01])),
                           D.from_host(np.array([0.02])))
    assert none is None
    np.testing.assert_array_equal(bits32(fast.numpy()), bits32(out))


@pytest.mark.parametrize("row_scales", [False, True])
def test_gemm_i8_full_tile_256(hip, row_scales):
    """The 256x256 full-tile kernel builds (output only, K > 512, at least
    1.5 tiles per CU: C3a's launch, here with a bias and per-tensor or
    per-row activation scales; a 100 MB output, stored with ordinary stores)
    give the bits of the general build everywhere, and the oracle's on
    sampled rows."""
    H, D = hip
    M, N, K = 4096, 6144, 1024
    gen = np.random.Generator(np.random.PCG64(11 + int(row_scales)))
    a = gen.integers(-127, 128, (M, K), dtype=np.int8)
    bt = gen.integers(-127, 128, (N, K), dtype=np.int8)
    sa = gen.uniform(1e-4, 1e-3, M) if row_scales else np.array([0.01])
    sb = gen.uniform(1e-4, 1e-3, N)
    bias = gen.standard_normal(N).astype(np.float32)
    ad, bd, sad, sbd, biasd = D.from_host(a), D.from_host(bt), D.from_host(sa), D.from_host(sb), D.from_host(bias)
    fast, _ = H.gemm_i8(ad, bd, sad, sbd, biasd)
    general, acc = H.gemm_i8(ad, bd, sad, sbd, biasd, want_acc=True)
    fast_h = fast.numpy()
    np.testing.assert_array_equal(bits32(fast_h), bits32(general.numpy()))
    rows = gen.choice(M, size=64, replace=False)
    eacc = O.ko_gemm_i8(a[rows], bt)
    np.testing.assert_array_equal(acc.numpy()[rows], eacc)
    expect = O.ko_epilogue(eacc, sa[rows] if row_scales else sa, sb, bias)
    np.testing.assert_array_equal(bits32(fast_h[rows]), bits32(expect))


@pytest.mark.parametrize("K,N", [(4096, 11008), (4096, 4096)])
@pytest.mark.parametrize("M", [1, 3, 8, 16, 17, 32, 33, 48, 64])
def test_skinny_per_token_and_per_channel(hip, M, K, N):
    """Config C5 shapes through kh_linear_i8: per-token activations, per-output-
    channel weights with 0.5% outlier columns x20, K=4096, N=11008 and 4096."""
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(100 + M + N))
    x = gen.standard_normal((M, K), dtype=np.float32)
    w = gen.standard_normal((K, N), dtype=np.float32) * np.float32(0.02)
    cols = gen.choice(N, size=N // 200, replace=False)
    w[:, cols] *= np.float32(20.0)
    bias = gen.standard_normal(N).astype(np.float32)
    wd = D.from_host(w)
    qw, sw = H.quantize_cols_packed(wd)
    out = H.linear_i8(D.from_host(x), qw, sw, D.from_host(bias)).numpy()
    eqw, esw = O.ko_quantize_cols_packed(w)
    np.testing.assert_array_equal(qw.numpy(), eqw)
    qx, sx = O.ko_quantize_rows(x)
    expect = O.ko_epilogue(O.ko_gemm_i8(qx, eqw), sx, esw, bias)
    np.testing.assert_array_equal(bits32(out), bits32(expect))


_C5_WEIGHTS = {}


def _c5_weights(H, D, K, N):
    """C5's weights (N(0, 0.02), 0.5 % of the columns x20) as per-output-
    channel codes packed [N, K] and their binary64 scales, on the device and
    from the oracle (built once per shape)."""
    if (K, N) not in _C5_WEIGHTS:
        gen = np.random.Generator(np.random.PCG64(K + 7 * N))
        w = gen.standard_normal((K, N), dtype=np.float32) * np.float32(0.02)
        w[:, gen.choice(N, size=N // 200, replace=False)] *= np.float32(20.0)
        eqw, esw = O.ko_quantize_cols_packed(w)
        _C5_WEIGHTS[(K, N)] = (D.from_host(eqw), D.from_host(esw), eqw, esw)
    return _C5_WEIGHTS[(K, N)]


def _c5_activations(gen, M, K):
    """fp32 activations ~N(0, 1) with the rows a per-token quantizer must get
    right: row 0 all zeros (scale 1.0, codes 0), row 1 exact ties (max 127
    gives scale 1.0 and the other values k + 1/2, rounded to even), row 2
    near-ties (the binary32 neighbours of k + 1/2 at scale 1.0) and the
    last row a single outlier."""
    x = gen.standard_normal((M, K), dtype=np.float32)
    if M >= 2:
        x[0] = 0.0
    if M >= 3:
        k = gen.integers(-126, 126, K).astype(np.float32)
        x[1] = k + np.float32(0.5)
        x[1, 0] = 127.0
    if M >= 4:
        k = gen.integers(-126, 126, K).astype(np.float32) + np.float32(0.5)
        x[2] = np.where(gen.integers(0, 2, K) == 1, np.nextafter(k, np.float32(200)),
                        np.nextafter(k, np.float32(-200)))
        x[2, 5] = -127.0
    if M >= 5:
        x[M - 1, K // 2] = np.float32(-50.0)
    return x


@pytest.mark.parametrize("K,N", [(4096, 4096), (4096, 11008)])
@pytest.mark.parametrize("M", [2, 3, 4, 5, 8, 16, 17, 31, 32])
def test_c5_linear_i8_special_rows(hip, M, K, N):
    """Config C5 through kh_linear_i8 at every decode-path M: codes, scales
    and outputs bit-exact against the oracle's per-row quantize, int32 GEMM
    and binary64 epilogue, with a zero row, an exact-tie row, a near-tie row
    and an outlier row among the tokens."""
    H, D = hip
    qwd, swd, eqw, esw = _c5_weights(H, D, K, N)
    gen = np.random.Generator(np.random.PCG64(1000 + M + N))
    x = _c5_activations(gen, M, K)
    bias = gen.standard_normal(N).astype(np.float32)
    out, q, sx = H.linear_i8(D.from_host(x), qwd, swd, D.from_host(bias), return_codes=True)
    out = out.numpy()
    eq, es = O.ko_quantize_rows(x)
    np.testing.assert_array_equal(q.numpy(), eq)
    np.testing.assert_array_equal(sx.numpy().view(np.uint64), es.view(np.uint64))
    expect = O.ko_epilogue(O.ko_gemm_i8(eq, eqw), es, esw, bias)
    np.testing.assert_array_equal(bits32(out), bits32(expect))


def _linear_i8_raw(Nn, D, xd, qwd, swd, biasd, M, K, N):
    """kh_linear_i8 through the C ABI into fresh outputs: (out, codes, scales)."""
    q = D.empty([M, K], "int8")
    sx = D.empty([M], "float64")
    out = D.empty([M, N], "float32")
    Nn.call("kh_linear_i8", xd.ptr, M, K, qwd.ptr, N, swd.ptr, 1, biasd.ptr, q.ptr, sx.ptr, out.ptr)
    return out, q, sx


def test_c5_decode_calls_back_to_back(hip):
    """Consecutive kh_linear_i8 calls with new activations, different M and
    both (K, N), queued before any is checked: each call's codes, scales and
    outputs equal the oracle's (no call reads another's codes)."""
    from kansaiml_amd import _native as Nn
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(77))
    plan = [(8, 4096, 4096), (8, 4096, 4096), (32, 4096, 4096), (4, 2048, 2048), (17, 4096, 11008),
            (32, 4096, 11008), (8, 4096, 4096)]
    calls = []
    for M, K, N in plan:
        w = gen.integers(-127, 128, (N, K), dtype=np.int8)
        sw = gen.uniform(1e-4, 1e-3, N)
        bias = gen.standard_normal(N).astype(np.float32)
        x = _c5_activations(gen, M, K)
        wd, swd, bd, xd = D.from_host(w), D.from_host(sw), D.from_host(bias), D.from_host(x)
        calls.append((x, w, sw, bias, M, K, N) + _linear_i8_raw(Nn, D, xd, wd, swd, bd, M, K, N))
    for x, w, sw, bias, M, K, N, out, q, sx in calls:
        print(f"back-to-back M={M} K={K} N={N}", flush=True)
        eq, es = O.ko_quantize_rows(x)
        np.testing.assert_array_equal(q.numpy(), eq)
        np.testing.assert_array_equal(sx.numpy().view(np.uint64), es.view(np.uint64))
        np.testing.assert_array_equal(bits32(out.numpy()), bits32(O.ko_epilogue(O.ko_gemm_i8(eq, w), es, sw, bias)))


def test_c5_decode_graph_replays(hip):
    """kh_linear_i8 (per-row quantize + skinny GEMM at M = 8) recorded as a
    HIP graph and replayed with new activations copied in between, and eager
    calls between replays: every replay's codes and outputs equal the
    oracle's for the activations it found."""
    import ctypes
    from kansaiml_amd import _native as Nn
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(78))
    M, K, N = 8, 4096, 4096
    w = gen.integers(-127, 128, (N, K), dtype=np.int8)
    sw = gen.uniform(1e-4, 1e-3, N)
    bias = gen.standard_normal(N).astype(np.float32)
    wd, swd, bd = D.from_host(w), D.from_host(sw), D.from_host(bias)
    xd = D.empty([M, K], "float32")
    q, sx, out = D.empty([M, K], "int8"), D.empty([M], "float64"), D.empty([M, N], "float32")
    args = (xd.ptr, M, K, wd.ptr, N, swd.ptr, 1, bd.ptr, q.ptr, sx.ptr, out.ptr)
    xd.copy_from(gen.standard_normal((M, K), dtype=np.float32))
    Nn.call("kh_linear_i8", *args)
    Nn.synchronize()
    Nn.call("kh_graph_capture_begin")
    try:
        Nn.call("kh_linear_i8", *args)
    except BaseException:
        Nn.lib().kh_graph_capture_end(None)
        raise
    g = ctypes.c_void_p()
    Nn.call("kh_graph_capture_end", ctypes.byref(g))
    try:
        for r in range(4):
            x = _c5_activations(gen, M, K) * np.float32(r + 1)
            xd.copy_from(x)
            Nn.call("kh_graph_launch", g)
            if r == 2:  # an eager call between replays
                _linear_i8_raw(Nn, D, xd, wd, swd, bd, M, K, N)
            eq, es = O.ko_quantize_rows(x)
            np.testing.assert_array_equal(bits32(out.numpy()), bits32(O.ko_epilogue(O.ko_gemm_i8(eq, w), es, sw, bias)))
            np.testing.assert_array_equal(q.numpy(), eq)
    finally:
        Nn.call("kh_graph_destroy", g)


def test_linear_i8_per_token(hip):
    """kh_linear_i8: per-token quantize fused ahead of the GEMM (config C5)."""
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(8))
    for M in (1, 8, 32):
        K, N = 4096, 1024
        x = gen.standard_normal((M, K), dtype=np.float32)
        w = (gen.standard_normal((K, N), dtype=np.float32) * np.float32(0.02))
        bias = gen.standard_normal(N).astype(np.float32)
        qw, sw = O.ko_quantize_cols_packed(w)
        out = H.linear_i8(D.from_host(x), D.from_host(qw), D.from_host(sw), D.from_host(bias)).numpy()
        qx, sx = O.ko_quantize_rows(x)
        expect = O.ko_epilogue(O.ko_gemm_i8(qx, qw), sx, sw, bias)
        np.testing.assert_array_equal(bits32(out), bits32(expect))


@pytest.mark.parametrize("M,K,N", [(1, 4096, 4096), (2, 4096, 11008), (1, 2048, 1000), (2, 8192, 33),
                                   (1, 8192, 4096), (2, 2048, 17), (1, 8192, 1), (2, 4096, 2)])
def test_linear_i8_decode_fused(hip, M, K, N):
    """The fused one-launch decode path of kh_linear_i8 (M <= 2): outputs,
    activation codes and per-token scales bit-exact against the oracle, with
    an all-zero row, a row of exact ties (binary64 fallback), a per-tensor
    weight scale and no bias."""
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(M * 7919 + K + N))
    x = gen.standard_normal((M, K), dtype=np.float32)
    if M == 2:
        x[1] = 0.0                                        # zero row: scale 1.0, codes 0
    tie = x[0].copy()
    tie[: K // 2] = np.float32(0.5)                       # 0.5 / (1 / 127) = 63.5: an exact tie
    tie[K // 2:] = np.float32(1.0)                       # row max 1.0, so the scale is 1/127
    qw = gen.integers(-127, 128, (N, K), dtype=np.int8)
    sw = gen.uniform(1e-3, 1e-2, N)
    bias = gen.standard_normal(N).astype(np.float32)
    for xin, sb, bb in ((x, sw, bias), (x, sw[:1], None), (np.stack([tie] * M), sw, bias)):
        out, q, sx = H.linear_i8(D.from_host(xin), D.from_host(qw), D.from_host(np.asarray(sb, np.float64)),
                                 D.from_host(bb) if bb is not None else None, return_codes=True)
        eq, esx = O.ko_quantize_rows(xin)
        np.testing.assert_array_equal(q.numpy(), eq)
        np.testing.assert_array_equal(sx.numpy().view(np.uint64), np.asarray(esx, np.float64).view(np.uint64))
        expect = O.ko_epilogue(O.ko_gemm_i8(eq, qw), esx, sb, bb)
        np.testing.assert_array_equal(bits32(out.numpy()), bits32(expect))


@pytest.mark.parametrize("M,K,N", [(3, 4096, 4096), (3, 4096, 11008), (3, 2048, 1000), (3, 2048, 17),
                                   (3, 4096, 33), (8, 4096, 11008), (5, 2048, 1000), (8, 2048, 17), (7, 4096, 33),
                                   (4, 4096, 4096), (6, 2048, 4096), (3, 2048, 1), (3, 4096, 5), (2, 8192, 3)])
def test_linear_i8_decode_fused_tokens(hip, M, K, N):
    """kh_linear_i8 for 3 <= M <= 8 tokens (K = 2048 or 4096): the one-launch
    decode kernel for M = 3 (its lanes' partial products summed by the
    transposed butterfly), per-row quantize plus the skinny GEMM above.
    Outputs, codes and per-token scales bit-exact against the oracle, with an
    all-zero row, a row of exact ties (the binary64 fallback), a per-tensor
    weight scale and no bias, and N not a multiple of the 16-row weight
    tile."""
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(M * 7919 + K + N + 3))
    x = gen.standard_normal((M, K), dtype=np.float32)
    x[1] = 0.0                                            # zero row: scale 1.0, codes 0
    x[M - 1, : K // 2] = np.float32(0.5)                  # 0.5 / (1 / 127) = 63.5: exact ties
    x[M - 1, K // 2:] = np.float32(-1.0)                  # row max 1.0, so the scale is 1/127
    qw = gen.integers(-127, 128, (N, K), dtype=np.int8)
    sw = gen.uniform(1e-3, 1e-2, N)
    bias = gen.standard_normal(N).astype(np.float32)
    eq, esx = O.ko_quantize_rows(x)
    for sb, bb in ((sw, bias), (sw[:1], None)):
        print(f"decode M={M} K={K} N={N} per_col={len(sb) > 1} bias={bb is not None}", flush=True)
        out, q, sx = H.linear_i8(D.from_host(x), D.from_host(qw), D.from_host(np.asarray(sb, np.float64)),
                                 D.from_host(bb) if bb is not None else None, return_codes=True)
        np.testing.assert_array_equal(q.numpy(), eq)
        np.testing.assert_array_equal(sx.numpy().view(np.uint64), np.asarray(esx, np.float64).view(np.uint64))
        expect = O.ko_epilogue(O.ko_gemm_i8(eq, qw), esx, sb, bb)
        np.testing.assert_array_equal(bits32(out.numpy()), bits32(expect))


@pytest.mark.parametrize("M,K,N", [(64, 512, 512), (1, 512, 17), (16, 4096, 100), (17, 1024, 512),
                                   (33, 512, 1000), (64, 512, 33), (8, 2048, 4096), (40, 1536, 64),
                                   (8, 4096, 300), (3, 4096, 16)])
def test_linear_i8_tensor(hip, M, K, N):
    """kh_linear_i8_tensor (QLinear int8 with a per-tensor activation scale):
    the one-launch kernel (M <= 64, K = 512, 1024, 2048 or 4096, M*K <=
    32768) and the two-launch path beyond it ((16, 4096): M*K too large;
    (40, 1536): K not a power of two) give the oracle's codes, scale and
    outputs bit for bit, with a
    per-tensor and a per-column weight scale, no bias, an all-zero input
    (scale 1.0) and exact ties (binary64 fallback)."""
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(M * 131 + K + N))
    x = gen.standard_normal((M, K), dtype=np.float32)
    x[0, :4] = np.float32(0.5)                            # with absmax 1.0 below: 63.5, an exact tie
    x[M - 1, -1] = np.float32(-1.0)
    x = np.clip(x, -1.0, 1.0).astype(np.float32)          # absmax exactly 1.0: scale 1/127
    qw = gen.integers(-127, 128, (N, K), dtype=np.int8)
    sw = gen.uniform(1e-3, 1e-2, N)
    bias = gen.standard_normal(N).astype(np.float32)
    for xin, sb, bb in ((x, sw, bias), (x, sw[:1], None), (np.zeros_like(x), sw, bias)):
        print(f"linear_i8_tensor M={M} K={K} N={N} per_col={len(sb) > 1} bias={bb is not None}", flush=True)
        out, q, s = H.linear_i8_tensor(D.from_host(xin), D.from_host(qw), D.from_host(np.asarray(sb, np.float64)),
                                       D.from_host(bb) if bb is not None else None, return_codes=True)
        eq, es = O.ko_quantize_tensor(xin)
        np.testing.assert_array_equal(q.numpy().reshape(M, K), eq.reshape(M, K))
        np.testing.assert_array_equal(s.numpy().view(np.uint64), np.asarray([es], np.float64).view(np.uint64))
        expect = O.ko_epilogue(O.ko_gemm_i8(eq.reshape(M, K), qw), np.full(M, es), sb, bb)
        np.testing.assert_array_equal(bits32(out.numpy()), bits32(expect))


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_linear_i8_paths_report_nonfinite(hip, bad):
    """A NaN or infinite activation reaches a quantizer on every kh_linear_i8 /
    kh_linear_i8_tensor path (one-launch decode for M = 1 and 3, per-row
    quantize + skinny GEMM for M = 8, the one-launch and two-launch per-tensor
    Linear): the next synchronize raises ValueError, as the reference's
    round(nan) does, and clears the report, so a clean call afterwards is
    exact."""
    from kansaiml_amd import _native as Nn
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(99))
    cases = [("row", 1, 4096, 64), ("row", 3, 2048, 48), ("row", 8, 4096, 32), ("row", 17, 4096, 4096),
             ("row", 32, 4096, 11008),
             ("tensor", 64, 512, 40), ("tensor", 16, 4096, 24)]
    for gran, M, K, N_ in cases:
        print(f"nonfinite {gran} M={M} K={K} N={N_} value={bad}", flush=True)
        x = gen.standard_normal((M, K), dtype=np.float32)
        qw = D.from_host(gen.integers(-127, 128, (N_, K), dtype=np.int8))
        sw = D.from_host(gen.uniform(1e-3, 1e-2, N_))
        fn = H.linear_i8 if gran == "row" else H.linear_i8_tensor
        xbad = x.copy()
        xbad[M - 1, K // 3] = np.float32(bad)
        fn(D.from_host(xbad), qw, sw)
        with pytest.raises(ValueError):
            Nn.synchronize()
        out = fn(D.from_host(x), qw, sw).numpy()
        if gran == "row":
            eq, esx = O.ko_quantize_rows(x)
        else:
            eq, es = O.ko_quantize_tensor(x)
            eq, esx = eq.reshape(M, K), np.full(M, es)
        np.testing.assert_array_equal(bits32(out), bits32(O.ko_epilogue(O.ko_gemm_i8(eq, qw.numpy()), esx,
                                                                         sw.numpy(), None)))


def test_dequantize_acc_matches_fused(hip):
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(9))
    a = gen.integers(-127, 128, (70, 96), dtype=np.int8)
    bt = gen.integers(-127, 128, (50, 96), dtype=np.int8)
    sa, sb = gen.uniform(1e-3, 1e-1, 70), gen.uniform(1e-3, 1e-1, 50)
    bias = gen.standard_normal(50).astype(np.float32)
    out, acc = run_gemm(H, D, a, bt, sa, sb, bias)
    sep = H.dequantize_acc(D.from_host(acc), D.from_host(sa), D.from_host(sb), D.from_host(bias)).numpy()
    np.testing.assert_array_equal(bits32(sep), bits32(out))


# ---------------------------------------------------------------------------
# fp32 matmul
# ---------------------------------------------------------------------------

def _f32_bound(a, b):
    K = a.shape[1]
    return 2 * K * np.finfo(np.float32).eps * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)) + 1e-30


@pytest.mark.parametrize("M,K,N", [(17, 19, 15), (100, 77, 50), (1, 1, 1), (64, 512, 512), (16, 32, 24),
                                   (257, 129, 131), (512, 1024, 768), (1024, 1024, 1024),
                                   (4100, 68, 4000), (4097, 33, 4001),  # 256x256 tiles, partial; K % 4 != 0
                                   (4100, 64, 4004), (3000, 2048, 5000)])  # ping-pong kernel, partial tiles
def test_matmul_f32_vs_reference(hip, M, K, N):
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(M + 7 * K + 13 * N))
    a = gen.standard_normal((M, K), dtype=np.float32)
    b = gen.standard_normal((K, N), dtype=np.float32)
    bias = gen.standard_normal(N).astype(np.float32)
    got = H.matmul(D.from_host(a), D.from_host(b), D.from_host(bias)).numpy()
    ref64 = a.astype(np.float64) @ b.astype(np.float64) + bias.astype(np.float64)
    bound = _f32_bound(a, b) + np.abs(bias) * np.finfo(np.float32).eps
    assert (np.abs(got - ref64) <= bound).all()
    ref = O.ref_add_bias(O.ref_matmul(a, b), bias) if O.ref_available() else O.ko_add_bias(O.ko_matmul_f32(a, b), bias)
    assert (np.abs(got - ref) <= 2 * bound).all()
    # the reference's own GPU-vs-CPU bar (tests/test_metal_backend.py:22)
    if K <= 32:
        assert np.abs(got - ref).max() < 1e-3


def test_matmul_f32_c3b_full_size(hip):
    """Config C3b: M=N=K=4096 ~N(0,1); sampled rows against float64."""
    H, D = hip
    n = 4096
    gen = np.random.Generator(np.random.PCG64(4))
    a = gen.standard_normal((n, n), dtype=np.float32)
    b = gen.standard_normal((n, n), dtype=np.float32)
    got = H.matmul(D.from_host(a), D.from_host(b)).numpy()
    rows = gen.choice(n, size=64, replace=False)
    ref64 = a[rows].astype(np.float64) @ b.astype(np.float64)
    assert (np.abs(got[rows] - ref64) <= _f32_bound(a[rows], b)).all()


# ---------------------------------------------------------------------------
# Fused epilogues (kh_gemm_i8_ex) and absmax partials for per-tensor quantize
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("M,N,K", [(512, 512, 256),      # ping-pong, full tiles
                                   (300, 1152, 384),     # ping-pong, partial tiles
                                   (130, 70, 80),        # general kernel (K % 64 != 0)
                                   (16384, 65, 384),     # a vocabulary head: narrow-N kernel; with partials ping-pong
                                   (8, 512, 512),        # skinny kernel
                                   (24, 1000, 8192)])    # skinny kernel, K split over 4 workgroups
@pytest.mark.parametrize("row_scales", [False, True])
def test_gemm_i8_fused_epilogues(hip, M, N, K, row_scales):
    """GELU and residual epilogues give the same bits as the unfused graph
    (gemm -> gelu kernel, gemm -> fp32 add), and the absmax partials a fused
    GEMM writes quantize its output exactly like kh_quantize_tensor; with a
    per-tensor or a per-row (per-token) activation scale."""
    from kansaiml_amd import _native as Nn
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(M + 3 * N + 7 * K))
    a = gen.integers(-127, 128, (M, K), dtype=np.int8)
    bt = gen.integers(-127, 128, (N, K), dtype=np.int8)
    sa, sb = np.array([3e-4]), gen.uniform(1e-4, 1e-3, N)
    if row_scales:
        sa = gen.uniform(1e-4, 1e-3, M)
    bias = gen.standard_normal(N).astype(np.float32)
    res = gen.standard_normal((M, N)).astype(np.float32)
    ad, bd, sad, sbd, biasd = D.from_host(a), D.from_host(bt), D.from_host(sa), D.from_host(sb), D.from_host(bias)
    plain, _ = H.gemm_i8(ad, bd, sad, sbd, biasd)
    expect = O.ko_epilogue(O.ko_gemm_i8(a, bt), sa, sb, bias)
    np.testing.assert_array_equal(bits32(plain.numpy()), bits32(expect))

    g_out, g_parts = H.gemm_i8_fused(ad, bd, sad, sbd, biasd, act="gelu", absmax=True)
    g_ref = D([M, N])
    Nn.call("kh_gelu", plain.ptr, g_ref.ptr, M * N)
    np.testing.assert_array_equal(bits32(g_out.numpy()), bits32(g_ref.numpy()))
    q1, s1 = H.quantize_tensor_parts(g_out, g_parts)
    q2, s2 = H.quantize_tensor(g_out)
    np.testing.assert_array_equal(q1.numpy(), q2.numpy())
    assert s1.numpy()[0] == s2.numpy()[0]

    r_out, r_parts = H.gemm_i8_fused(ad, bd, sad, sbd, biasd, residual=D.from_host(res), absmax=True)
    np.testing.assert_array_equal(bits32(r_out.numpy()), bits32((res + expect).astype(np.float32)))
    q1, s1 = H.quantize_tensor_parts(r_out, r_parts)
    q2, s2 = H.quantize_tensor(r_out)
    np.testing.assert_array_equal(q1.numpy(), q2.numpy())
    assert s1.numpy()[0] == s2.numpy()[0]


@pytest.mark.parametrize("M,N,K", [(2055, 65, 384), (4096, 128, 448), (3000, 7, 64)])
@pytest.mark.parametrize("row_scales", [False, True])
def test_gemm_i8_narrow_fused_epilogues(hip, M, N, K, row_scales):
    """The narrow-N kernel (N <= 128, M >= 2048) with the GELU and residual
    epilogues and no partials: the same bits as the unfused graph, and its
    int32 accumulators equal the oracle's."""
    from kansaiml_amd import _native as Nn
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(M + 5 * N + 3 * K))
    a = gen.integers(-127, 128, (M, K), dtype=np.int8)
    bt = gen.integers(-127, 128, (N, K), dtype=np.int8)
    sa = gen.uniform(1e-4, 1e-3, M) if row_scales else np.array([3e-4])
    sb = gen.uniform(1e-4, 1e-3, N)
    bias = gen.standard_normal(N).astype(np.float32)
    res = gen.standard_normal((M, N)).astype(np.float32)
    ad, bd, sad, sbd, biasd = D.from_host(a), D.from_host(bt), D.from_host(sa), D.from_host(sb), D.from_host(bias)
    plain, acc = H.gemm_i8(ad, bd, sad, sbd, biasd, want_acc=True)
    eacc = O.ko_gemm_i8(a, bt)
    np.testing.assert_array_equal(acc.numpy(), eacc)
    expect = O.ko_epilogue(eacc, sa, sb, bias)
    np.testing.assert_array_equal(bits32(plain.numpy()), bits32(expect))
    g_out, _ = H.gemm_i8_fused(ad, bd, sad, sbd, biasd, act="gelu")
    g_ref = D([M, N])
    Nn.call("kh_gelu", plain.ptr, g_ref.ptr, M * N)
    np.testing.assert_array_equal(bits32(g_out.numpy()), bits32(g_ref.numpy()))
    r_out, _ = H.gemm_i8_fused(ad, bd, sad, sbd, None, residual=D.from_host(res))
    np.testing.assert_array_equal(bits32(r_out.numpy()),
                                  bits32((res + O.ko_epilogue(eacc, sa, sb, None)).astype(np.float32)))


@pytest.mark.parametrize("M,N,K", [(16384, 1536, 384),   # C4 fc1: ping-pong, two passes
                                   (300, 1152, 384),     # partial tiles
                                   (1000, 1000, 1536),   # K > 512: the passes still take 128x128 tiles
                                   (256, 258, 128),      # N % 4 == 2: full interior tiles store codes bytewise
                                   (130, 70, 80),        # general kernel (K % 64 != 0): fp32 temporary
                                   (8, 512, 512)])       # skinny kernel: fp32 temporary
def test_gemm_i8_quant_matches_unfused(hip, M, N, K):
    """kh_gemm_i8_quant's codes and scale equal the per-tensor quantize
    (the oracle's, and kh_quantize_tensor's) of the unfused GEMM's fp32
    output, for the plain, GELU and residual epilogues and per-row
    activation scales."""
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(M + 5 * N + 11 * K))
    a = gen.integers(-127, 128, (M, K), dtype=np.int8)
    bt = gen.integers(-127, 128, (N, K), dtype=np.int8)
    sb = gen.uniform(1e-4, 1e-3, N)
    bias = gen.standard_normal(N).astype(np.float32)
    res = (gen.standard_normal((M, N)) * 4).astype(np.float32)
    ad, bd, sbd, biasd, resd = D.from_host(a), D.from_host(bt), D.from_host(sb), D.from_host(bias), D.from_host(res)
    for sa in (np.array([3e-4]), gen.uniform(1e-4, 5e-4, M)):
        sad = D.from_host(sa)
        for act, residual in ((None, None), ("gelu", None), (None, resd)):
            y, _ = H.gemm_i8_fused(ad, bd, sad, sbd, biasd, act=act, residual=residual)
            yh = y.numpy()
            oq, os_ = O.ko_quantize_tensor(yh)
            q2, s2 = H.quantize_tensor(y)
            q, s = H.gemm_i8_quant(ad, bd, sad, sbd, biasd, act=act, residual=residual)
            np.testing.assert_array_equal(q.numpy().reshape(-1), oq.reshape(-1))
            np.testing.assert_array_equal(q.numpy(), q2.numpy())
            assert s.numpy()[0] == os_ == s2.numpy()[0]


def test_gemm_i8_quant_edge_cases(hip):
    """A zero result quantizes with scale 1.0 (quantize.py:68); an empty one
    too; a NaN in the residual is reported as ValueError, as the unfused
    quantize reports it."""
    from kansaiml_amd import _native as Nn
    H, D = hip
    a = np.zeros((256, 384), np.int8)
    bt = np.ones((512, 384), np.int8)
    sad, sbd = D.from_host(np.array([0.5])), D.from_host(np.full(512, 0.25))
    q, s = H.gemm_i8_quant(D.from_host(a), D.from_host(bt), sad, sbd)
    assert s.numpy()[0] == 1.0 and not q.numpy().any()
    q, s = H.gemm_i8_quant(D([0, 384], "int8"), D.from_host(bt), sad, sbd)
    assert s.numpy()[0] == 1.0
    res = np.zeros((256, 512), np.float32)
    res[7, 9] = np.nan
    H.gemm_i8_quant(D.from_host(a), D.from_host(bt), sad, sbd, residual=D.from_host(res))
    with pytest.raises(ValueError):
        Nn.synchronize()
    Nn.synchronize()


@pytest.mark.parametrize("M,N,K", [(16384, 1536, 384),  # C4 fc1, per token: the fused kernel
                                   (300, 1536, 384),    # a partial last workgroup (12 rows)
                                   (64, 512, 256),      # two blocks per wave, 8 k-substeps
                                   (1, 1024, 384),      # one row (a per-tensor scale), four blocks per wave
                                   (130, 1024, 256),
                                   (200, 1000, 384),    # other N: fp32 temporary + quantize_rows
                                   (100, 512, 448)])    # other K: the same
def test_gemm_i8_quant_rows_matches_unfused(hip, M, N, K):
    """kh_gemm_i8_quant_rows' codes and row scales equal the per-row
    quantize (kh_quantize_rows, and the oracle's) of the unfused GEMM's fp32
    output, plain and with GELU, bit for bit.  Rows of zero codes under an
    all-negative bias hold only negative values (their largest |GELU| is not
    GELU(max): the fused kernel's extra sweep), a row with a huge activation
    scale saturates, and a zero row scale gives a zero row."""
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(3 * M + 7 * N + K))
    a = gen.integers(-127, 128, (M, K), dtype=np.int8)
    bt = gen.integers(-127, 128, (N, K), dtype=np.int8)
    sa = gen.uniform(1e-4, 5e-4, M)
    a[M // 2] = 0
    sa[M - 1] = 0.0
    if M > 2:
        sa[1] = 1e30
    sb = gen.uniform(1e-4, 1e-3, N)
    ad, bd, sad, sbd = D.from_host(a), D.from_host(bt), D.from_host(sa), D.from_host(sb)
    for bias in (gen.standard_normal(N).astype(np.float32), -np.abs(gen.standard_normal(N)).astype(np.float32) - 0.01,
                 None):
        biasd = D.from_host(bias) if bias is not None else None
        for act in (None, "gelu"):
            y, _ = H.gemm_i8_fused(ad, bd, sad, sbd, biasd, act=act)
            q2, s2 = H.quantize_rows(y)
            q, s = H.gemm_i8_quant_rows(ad, bd, sad, sbd, biasd, act=act)
            np.testing.assert_array_equal(q.numpy(), q2.numpy())
            np.testing.assert_array_equal(s.numpy().view(np.uint64), s2.numpy().view(np.uint64))
            rows = np.unique(np.r_[0, 1, M // 2, M - 1, gen.integers(0, M, 64)]) % M
            oq, os_ = O.ko_quantize_rows(y.numpy()[rows])
            np.testing.assert_array_equal(q.numpy()[rows], oq)
            np.testing.assert_array_equal(s.numpy()[rows], os_)


def test_gemm_i8_quant_rows_edge_cases(hip):
    """An empty result: nothing for M = 0, every row scale 1.0 for N = 0
    (quantize.py:68 per row); a NaN row scale makes that row's values NaN:
    its codes are zero, its scale NaN, the others untouched, and the next
    synchronize raises ValueError as the unfused per-row quantize does."""
    from kansaiml_amd import _native as Nn
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(5))
    a = gen.integers(-127, 128, (192, 256), dtype=np.int8)
    bt = gen.integers(-127, 128, (384, 256), dtype=np.int8)
    sb = D.from_host(np.full(384, 1e-3))
    q, s = H.gemm_i8_quant_rows(D([0, 256], "int8"), D.from_host(bt), D([0], "float64"), sb)
    assert q.shape == [0, 384] and s.shape == [0]
    q, s = H.gemm_i8_quant_rows(D.from_host(a), D([0, 256], "int8"), D.from_host(np.full(192, 1e-3)),
                                D([0], "float64"))
    assert (s.numpy() == 1.0).all()
    sa = np.full(192, 1e-3)
    sa[70] = np.nan
    ad, bd, sad = D.from_host(a), D.from_host(bt), D.from_host(sa)
    for act in (None, "gelu"):
        q, s = H.gemm_i8_quant_rows(ad, bd, sad, sb, act=act)
        with pytest.raises(ValueError):
            Nn.synchronize()
        Nn.synchronize()
        y, _ = H.gemm_i8_fused(ad, bd, sad, sb, act=act)
        qh, sh = q.numpy(), s.numpy()
        assert not qh[70].any() and np.isnan(sh[70])
        keep = np.r_[0:70, 71:192]
        oq, os_ = O.ko_quantize_rows(y.numpy()[keep])
        np.testing.assert_array_equal(qh[keep], oq)
        np.testing.assert_array_equal(sh[keep], os_)


def _producer_parts(x):
    """Absmax partials of x as a producer would write them (kh_absmax_parts)."""
    import ctypes
    from kansaiml_amd import _native as Nn
    from kansaiml_amd import hip as H
    parts = H.AbsmaxParts()
    Nn.call("kh_absmax_parts", x.ptr, x.numel(), parts.buf.ptr, H.ABSMAX_PARTS, ctypes.byref(parts._n))
    return parts


@pytest.mark.parametrize("M,N,K", [(16384, 384, 1536),  # C4 fc2 (fused kernel, one 384-column tile)
                                   (16384, 384, 384),   # C4 O
                                   (512, 128, 64), (256, 256, 640), (1024, 768, 256),  # NB = 1, 2; two tiles
                                   (100, 384, 384), (256, 200, 128), (128, 384, 96)])  # other shapes: two steps
def test_gemm_i8_qload_matches_two_steps(hip, M, N, K):
    """kh_gemm_i8_qload equals kh_quantize_tensor_parts followed by
    kh_gemm_i8_ex with that scale, bit for bit (plain, bias, GELU and
    residual epilogues, its own absmax partials), and the oracle's quantize
    and GEMM on sampled rows."""
    from kansaiml_amd import _native as Nn
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(M * 3 + N * 7 + K))
    x = (gen.standard_normal((M, K)) * 2).astype(np.float32)
    x[gen.integers(0, M), gen.integers(0, K)] = 17.0  # the tensor's max, away from the rest
    bt = gen.integers(-127, 128, (N, K), dtype=np.int8)
    sb = gen.uniform(1e-4, 1e-3, N)
    bias = gen.standard_normal(N).astype(np.float32)
    res = gen.standard_normal((M, N)).astype(np.float32)
    xd, bd, sbd, biasd, resd = D.from_host(x), D.from_host(bt), D.from_host(sb), D.from_host(bias), D.from_host(res)
    parts = _producer_parts(xd)
    q2, s2 = H.quantize_tensor_parts(xd, parts)
    oq, os_ = O.ko_quantize_tensor(x)
    np.testing.assert_array_equal(q2.numpy().reshape(-1), oq.reshape(-1))
    for b_, act, r_ in ((None, None, None), (biasd, None, None), (biasd, "gelu", None), (biasd, None, resd)):
        out, oparts, sc = H.gemm_i8_qload(xd, parts, bd, sbd, b_, act=act, residual=r_, absmax=True,
                                          want_scale=True)
        ref, rparts = H.gemm_i8_fused(q2, bd, s2, sbd, b_, act=act, residual=r_, absmax=True)
        np.testing.assert_array_equal(bits32(out.numpy()), bits32(ref.numpy()))
        assert sc.numpy()[0] == s2.numpy()[0] == os_
        qa, sa_ = H.quantize_tensor_parts(out, oparts)
        qb, sb_ = H.quantize_tensor(out)
        np.testing.assert_array_equal(qa.numpy(), qb.numpy())
        assert sa_.numpy()[0] == sb_.numpy()[0]
    rows = gen.choice(M, size=min(M, 48), replace=False)
    eacc = O.ko_gemm_i8(oq.reshape(M, K)[rows], bt)
    out, _ = H.gemm_i8_qload(xd, parts, bd, sbd, biasd)
    np.testing.assert_array_equal(bits32(out.numpy()[rows]), bits32(O.ko_epilogue(eacc, [os_], sb, bias)))
    Nn.synchronize()


def test_gemm_i8_qload_ties_and_nonfinite(hip):
    """Values exactly between two codes (the exact binary64 path, ties to
    even) give the two-step codes; a NaN in x is reported as ValueError at
    the next synchronize, as the unfused quantize reports it."""
    from kansaiml_amd import _native as Nn
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(41))
    M, N, K = 256, 384, 384
    x = (gen.integers(-126, 126, (M, K)) + 0.5).astype(np.float32)
    x[3, 7] = 127.0  # scale exactly 1.0: every other value is a tie
    bt = gen.integers(-127, 128, (N, K), dtype=np.int8)
    sb = np.full(N, 0.01)
    xd, bd, sbd = D.from_host(x), D.from_host(bt), D.from_host(sb)
    parts = _producer_parts(xd)
    out, _, sc = H.gemm_i8_qload(xd, parts, bd, sbd, want_scale=True)
    oq, os_ = O.ko_quantize_tensor(x)
    assert os_ == 1.0 and sc.numpy()[0] == 1.0
    expect = O.ko_epilogue(O.ko_gemm_i8(oq.reshape(M, K), bt), [1.0], sb, None)
    np.testing.assert_array_equal(bits32(out.numpy()), bits32(expect))
    x[100, 5] = np.nan
    xd = D.from_host(x)
    parts = _producer_parts(xd)
    H.gemm_i8_qload(xd, parts, bd, sbd)
    with pytest.raises(ValueError):
        Nn.synchronize()
    Nn.synchronize()


@pytest.mark.parametrize("case", ["negative", "threshold", "nan_bias", "inf_bias", "neg_inf_bias"])
def test_gemm_i8_quant_gelu_absmax_paths(hip, case):
    """The absmax pass of a GELU epilogue takes each lane's largest value's
    GELU when that value is >= 0.3 and every value's GELU otherwise; both
    give the unfused scale and codes.  Pre-activations near -0.75 (the
    largest |GELU| of a negative argument; the second path everywhere),
    straddling 0.3 by a few ulps (both paths, lane by lane), and a NaN or
    infinite bias (a non-finite result: reported as ValueError, as the
    unfused quantize reports it, with the same codes)."""
    from kansaiml_amd import _native as Nn
    H, D = hip
    M, N, K = 512, 384, 128  # full 128x128 tiles
    gen = np.random.Generator(np.random.PCG64(77))
    a = gen.integers(-127, 128, (M, K), dtype=np.int8)
    bt = gen.integers(-127, 128, (N, K), dtype=np.int8)
    sa, sb = np.array([3e-4]), np.full(N, 1e-4)  # GEMM terms of about 2e-3
    if case == "negative":
        bias = np.float32(-0.75) + gen.uniform(-0.01, 0.01, N).astype(np.float32)
    elif case == "threshold":
        sb = np.full(N, 1e-9)  # terms of about 2e-8: a few ulps of 0.3
        bias = np.full(N, 0.3, np.float32)
    else:
        bias = gen.standard_normal(N).astype(np.float32)
        bias[N // 3] = {"nan_bias": np.nan, "inf_bias": np.inf, "neg_inf_bias": -np.inf}[case]
    ad, bd, sad, sbd, biasd = D.from_host(a), D.from_host(bt), D.from_host(sa), D.from_host(sb), D.from_host(bias)
    bad = case.endswith("_bias")
    q, s = H.gemm_i8_quant(ad, bd, sad, sbd, biasd, act="gelu")
    if bad:
        with pytest.raises(ValueError):
            Nn.synchronize()
    y, _ = H.gemm_i8_fused(ad, bd, sad, sbd, biasd, act="gelu")
    q2, s2 = H.quantize_tensor(y)
    if bad:
        with pytest.raises(ValueError):
            Nn.synchronize()
        assert np.isnan(s.numpy()[0]) and np.isnan(s2.numpy()[0])
    else:
        yh = y.numpy()
        if case == "threshold":  # pre-activations on both sides of 0.3
            pre = H.gemm_i8_fused(ad, bd, sad, sbd, biasd)[0].numpy()
            assert (pre >= np.float32(0.3)).any() and (pre < np.float32(0.3)).any()
        oq, os_ = O.ko_quantize_tensor(yh)
        np.testing.assert_array_equal(q.numpy().reshape(-1), oq.reshape(-1))
        assert s.numpy()[0] == os_
        assert s.numpy()[0] == s2.numpy()[0]
    np.testing.assert_array_equal(q.numpy(), q2.numpy())


@pytest.mark.parametrize("rows,d", [(1000, 384), (16384, 384), (37, 100), (1, 1024), (5, 3), (3001, 128),
                                    (777, 256), (4097, 512), (16, 384),
                                    (40000, 384)])
def test_layernorm_quant_matches_unfused(hip, rows, d):
    """kh_layernorm_quant's codes and scale equal the per-tensor quantize of
    kh_layernorm's output (two rows per wave for D = 128..512, vector and
    scalar row paths, one workgroup to 2500)."""
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(rows * 7 + d))
    x = (gen.standard_normal((rows, d)) * 3 + 0.5).astype(np.float32)
    w, b = gen.standard_normal(d).astype(np.float32), gen.standard_normal(d).astype(np.float32)
    xd, wd, bd = D.from_host(x), D.from_host(w), D.from_host(b)
    y, _ = H.layer_norm(xd, wd, bd)
    oq, os_ = O.ko_quantize_tensor(y.numpy())
    q, s = H.layer_norm_quant(xd, wd, bd)
    np.testing.assert_array_equal(q.numpy().reshape(-1), oq.reshape(-1))
    assert s.numpy()[0] == os_


def test_layernorm_quant_back_to_back(hip):
    """Consecutive LayerNorm quantizes with no synchronization between them
    (the partials scratch reused), of different sizes and data, each equal
    to the two-step result."""
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(12))
    w, b = gen.standard_normal(384).astype(np.float32), gen.standard_normal(384).astype(np.float32)
    wd, bd = D.from_host(w), D.from_host(b)
    xs = [D.from_host((gen.standard_normal((r, 384)) * (i + 1)).astype(np.float32))
          for i, r in enumerate((16384, 16, 5000, 16384, 1, 9000))]
    got = [H.layer_norm_quant(xd, wd, bd) for xd in xs]
    for xd, (q, s) in zip(xs, got):
        y, _ = H.layer_norm(xd, wd, bd)
        oq, os_ = O.ko_quantize_tensor(y.numpy())
        np.testing.assert_array_equal(q.numpy().reshape(-1), oq.reshape(-1))
        assert s.numpy()[0] == os_


def test_layernorm_quant_edge_cases(hip):
    from kansaiml_amd import _native as Nn
    H, D = hip
    w, b = D.from_host(np.ones(384, np.float32)), D.from_host(np.zeros(384, np.float32))
    q, s = H.layer_norm_quant(D([0, 384]), w, b)
    assert s.numpy()[0] == 1.0
    x = np.ones((20, 384), np.float32)  # constant rows normalize to exactly 0
    q, s = H.layer_norm_quant(D.from_host(x), w, b)
    assert s.numpy()[0] == 1.0 and not q.numpy().any()
    x[3, 5] = np.inf
    H.layer_norm_quant(D.from_host(x), w, b)
    with pytest.raises(ValueError):
        Nn.synchronize()
    Nn.synchronize()


def test_layernorm_and_attention_absmax_parts(hip):
    """LayerNorm and attention outputs quantized from the partials their
    kernels wrote equal kh_quantize_tensor of the same outputs; a partials
    buffer too small for the grid falls back to a separate absmax pass."""
    from kansaiml_amd import _native as Nn
    import ctypes
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(41))
    x = (gen.standard_normal((1000, 384)) * 3).astype(np.float32)
    w, b = gen.standard_normal(384).astype(np.float32), gen.standard_normal(384).astype(np.float32)
    out, parts = H.layer_norm(D.from_host(x), D.from_host(w), D.from_host(b), absmax=True)
    assert parts.count == 63  # one partial per 16-row workgroup
    q1, s1 = H.quantize_tensor_parts(out, parts)
    q_ln, s_ln = H.quantize_tensor(out)
    np.testing.assert_array_equal(q1.numpy(), q_ln.numpy())
    assert s1.numpy()[0] == s_ln.numpy()[0]

    qkv = (gen.standard_normal((2 * 100, 3 * 128)) * 1.5).astype(np.float32)
    aout, aparts = H.causal_attention(D.from_host(qkv), 2, 100, 2, 128, absmax=True)
    q1, s1 = H.quantize_tensor_parts(aout, aparts)
    q2, s2 = H.quantize_tensor(aout)
    np.testing.assert_array_equal(q1.numpy(), q2.numpy())
    assert s1.numpy()[0] == s2.numpy()[0]

    small = D([4], "int32")  # 4 slots < 63 workgroups: separate pass
    n = ctypes.c_int(0)
    out2 = D([1000, 384])
    xd, wd, bd = D.from_host(x), D.from_host(w), D.from_host(b)  # keep the buffers alive across the call
    Nn.call("kh_layernorm_ex", xd.ptr, 1000, 384, wd.ptr, bd.ptr, 1e-5, out2.ptr, small.ptr, 4, ctypes.byref(n))
    assert 1 <= n.value <= 4
    q3 = D([1000, 384], "int8")
    s3 = D([1], "float64")
    Nn.call("kh_quantize_tensor_parts", out2.ptr, 1000 * 384, small.ptr, n.value, q3.ptr, s3.ptr)
    np.testing.assert_array_equal(q3.numpy(), q_ln.numpy())
    assert s3.numpy()[0] == s_ln.numpy()[0]


def _row_parts_host(x, per_row):
    """Max |x| bits of per_row equal pieces of every row (a producer's row
    partials, computed on the host)."""
    bits = np.ascontiguousarray(x, np.float32).view(np.uint32) & np.uint32(0x7FFFFFFF)
    rows, k = bits.shape
    return bits.reshape(rows, per_row, k // per_row).max(axis=2).astype(np.uint32).view(np.int32)


@pytest.mark.parametrize("batch,seq,heads,causal", [(2, 100, 2, True), (3, 256, 6, True), (2, 64, 3, False)])
def test_attention_row_partials(hip, batch, seq, heads, causal):
    """kh_attention_rows writes the max |out| bits of every (row, head) of the
    output it stores, and the output is kh_attention_ex's bit for bit."""
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(batch * 1000 + seq + heads))
    d = 64 * heads
    qkv = D.from_host((gen.standard_normal((batch * seq, 3 * d)) * 1.5).astype(np.float32))
    out, rp = H.attention_rows(qkv, batch, seq, heads, d, causal=causal)
    ref, _ = H.attention(qkv, batch, seq, heads, d, causal=causal)
    o = out.numpy()
    np.testing.assert_array_equal(bits32(o), bits32(ref.numpy()))
    np.testing.assert_array_equal(rp.buf.numpy(), _row_parts_host(o, heads))


@pytest.mark.parametrize("M,N,K,P", [(1024, 384, 384, 6),    # C4's O: the fused kernel, 6 parts per row
                                     (2048, 384, 1536, 12),  # fc2's shape, 12 parts per row
                                     (512, 256, 512, 1),     # N = 256 tile, one part per row
                                     (128, 128, 64, 16),     # N = 128 tile, 16 parts
                                     (100, 200, 384, 6),     # unfused: per-row quantize + GEMM
                                     (1024, 384, 384, 32)])  # more than 16 parts: unfused
def test_gemm_i8_qload_rows_matches_two_steps(hip, M, N, K, P):
    """kh_gemm_i8_qload_rows equals the oracle's per-row quantize, int32 GEMM
    and binary64 epilogue, bit for bit, for the plain, GELU and residual
    epilogues; its row scales are the oracle's; rows of zeros, exact ties
    and outliers included."""
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(M + 7 * N + 3 * K + P))
    x = (gen.standard_normal((M, K)) * 2).astype(np.float32)
    x[3] = 0.0
    x[5] = gen.integers(-126, 126, K).astype(np.float32) + np.float32(0.5)
    x[5, 0] = 127.0
    x[7, K // 2] = 300.0
    bt = gen.integers(-127, 128, (N, K), dtype=np.int8)
    sb = gen.uniform(1e-4, 1e-3, N)
    bias = gen.standard_normal(N).astype(np.float32)
    res = gen.standard_normal((M, N)).astype(np.float32)
    rp = H.RowParts(M, P)
    rp.buf.copy_from(_row_parts_host(x, P))
    xd, bd, sbd, biasd = D.from_host(x), D.from_host(bt), D.from_host(sb), D.from_host(bias)
    qx, sx = O.ko_quantize_rows(x)
    eacc = O.ko_gemm_i8(qx, bt)
    expect = O.ko_epilogue(eacc, sx, sb, bias)
    out, scales = H.gemm_i8_qload_rows(xd, rp, bd, sbd, biasd, want_scales=True)
    np.testing.assert_array_equal(scales.numpy().view(np.uint64), sx.view(np.uint64))
    np.testing.assert_array_equal(bits32(out.numpy()), bits32(expect))
    plain, _ = H.gemm_i8(D.from_host(qx), bd, D.from_host(sx), sbd, biasd)
    g_ref = D([M, N])
    from kansaiml_amd import _native as Nn
    Nn.call("kh_gelu", plain.ptr, g_ref.ptr, M * N)
    g = H.gemm_i8_qload_rows(xd, rp, bd, sbd, biasd, act="gelu")
    np.testing.assert_array_equal(bits32(g.numpy()), bits32(g_ref.numpy()))
    r = H.gemm_i8_qload_rows(xd, rp, bd, sbd, None, residual=D.from_host(res))
    np.testing.assert_array_equal(bits32(r.numpy()), bits32((res + O.ko_epilogue(eacc, sx, sb, None)).astype(np.float32)))


def test_gemm_i8_qload_rows_reports_nonfinite(hip):
    """A NaN in a row reaches the per-row scale: ValueError at the next
    synchronize, as kh_quantize_rows reports it; a clean call afterwards is
    exact."""
    from kansaiml_amd import _native as Nn
    H, D = hip
    gen = np.random.Generator(np.random.PCG64(5))
    M, N, K = 256, 384, 384
    x = gen.standard_normal((M, K)).astype(np.float32)
    bt = gen.integers(-127, 128, (N, K), dtype=np.int8)
    sb = gen.uniform(1e-4, 1e-3, N)
    xb = x.copy()
    xb[17, 100] = np.nan
    rp = H.RowParts(M, 6)
    rp.buf.copy_from(_row_parts_host(xb, 6))
    H.gemm_i8_qload_rows(D.from_host(xb), rp, D.from_host(bt), D.from_host(sb))
    with pytest.raises(ValueError):
        Nn.synchronize()
    rp.buf.copy_from(_row_parts_host(x, 6))
    out = H.gemm_i8_qload_rows(D.from_host(x), rp, D.from_host(bt), D.from_host(sb)).numpy()
    qx, sx = O.ko_quantize_rows(x)
    np.testing.assert_array_equal(bits32(out), bits32(O.ko_epilogue(O.ko_gemm_i8(qx, bt), sx, sb, None)))
