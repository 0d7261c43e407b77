"""Op-level parity of the gfx950 kernels with the CPU oracle, through the C ABI.

The bar is bit-exact equality with the reference's scalar path for every op (integer, byte
and float results alike). NaN payloads of fp16 decoding are the one documented exception:
the hardware conversion quiets signalling NaNs, so NaNs are compared by class."""
import numpy as np
import pytest

from _bind import F32, Q4_0, Q8_0, nblocks, row_bytes

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(7)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def dev(qmh, a):
    return qmh.DeviceBuffer.from_array(a)


def test_fp16_decode_all_halves(gpu, oracle):
    h = np.arange(65536, dtype=np.uint16)
    dh, df = dev(gpu, h), gpu.DeviceBuffer(65536 * 4)
    gpu._check(gpu.load_library().qmh_fp16_to_fp32(dh.ptr, df.ptr, 65536, None), "h2f")
    got, want = df.to_array(np.float32), oracle.h2f(h)
    isn = np.isnan(want)
    assert np.array_equal(np.isnan(got), isn)
    assert np.array_equal(bits(got[~isn]), bits(want[~isn]))


def test_fp16_encode_sweep(gpu, oracle):
    u = np.arange(0, 1 << 32, 4099, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([u.view(np.float32), ((rng.random(1 << 20) - 0.5) *
                                             np.exp2(rng.integers(-30, 18, 1 << 20))).astype(np.float32)])
    dx, dh = dev(gpu, x), gpu.DeviceBuffer(x.size * 2)
    gpu._check(gpu.load_library().qmh_fp32_to_fp16(dx.ptr, dh.ptr, x.size, None), "f2h")
    assert np.array_equal(dh.to_array(np.uint16), oracle.f2h(x))


@pytest.mark.parametrize("dtype", [Q8_0, Q4_0])
def test_quantize_rows_bytes(gpu, oracle, dtype):
    fn = gpu.load_library().qmh_quantize_rows_q8 if dtype == Q8_0 else gpu.load_library().qmh_quantize_rows_q4
    for it in range(60):
        rows, n = int(rng.integers(1, 9)), int(rng.integers(1, 701))
        x = (rng.standard_normal((rows, n)) * np.exp2(rng.integers(-12, 13))).astype(np.float32)
        x[0, rng.integers(0, n)] *= 50.0
        if it % 5 == 0:
            x[-1, : min(n, 64)] = 0.0
        dx, dy = dev(gpu, x), gpu.DeviceBuffer(rows * row_bytes(dtype, n))
        gpu._check(fn(dx.ptr, dy.ptr, rows, n, None), "quantize")
        assert np.array_equal(dy.to_array(np.uint8).reshape(rows, -1), oracle.quantize(dtype, x)), (rows, n)


def test_quantize_q8_rounding_boundaries(gpu, oracle):
    """The device Q8_0 quantizer rounds v*(1/d) and defers to the exact division near k+1/2:
    values whose quotient sits on, or a few ulps beside, a half-integer (ties included) and
    scales down to fp16 subnormals must still give the reference's codes."""
    rows = []
    for d_target in (0.3, 0.5, 1.0 / 3.0, 0.0123, 7.7e-6, 2.0 ** -20, 3e-8, 1e-7, 5.5e-8):
        dd = np.float32(oracle.h2f(oracle.f2h(np.array([d_target], np.float32)))[0])
        if dd == 0:
            continue
        amax = np.float32(127) * dd
        vals = []
        for k in range(-127, 127):
            c = np.float32(k + 0.5) * dd
            vals += [c, np.nextafter(c, np.float32(np.inf)), np.nextafter(c, np.float32(-np.inf)),
                     np.nextafter(np.nextafter(c, np.float32(np.inf)), np.float32(np.inf))]
        vals = np.array(vals, np.float32)
        vals = vals[np.abs(vals) <= amax]
        for i in range(0, len(vals), 31):
            row = np.zeros(32, np.float32)
            row[0] = amax
            chunk = vals[i: i + 31]
            row[1: 1 + len(chunk)] = chunk
            rows.append(row)
    x = np.stack(rows)
    dx, dy = dev(gpu, x), gpu.DeviceBuffer(x.shape[0] * 34)
    gpu._check(gpu.load_library().qmh_quantize_rows_q8(dx.ptr, dy.ptr, x.shape[0], 32, None), "quantize")
    assert np.array_equal(dy.to_array(np.uint8).reshape(x.shape[0], -1), oracle.quantize(Q8_0, x))


@pytest.mark.parametrize("dtype", [F32, Q8_0, Q4_0])
def test_row_to_f32(gpu, oracle, dtype):
    n = 1000
    x = rng.standard_normal(n).astype(np.float32)
    row = x if dtype == F32 else oracle.quantize(dtype, x)[0]
    dr, dy = dev(gpu, row), gpu.DeviceBuffer(n * 4)
    gpu._check(gpu.load_library().qmh_row_to_f32(dtype, dr.ptr, dy.ptr, n, None), "row_to_f32")
    assert np.array_equal(bits(dy.to_array(np.float32)), bits(oracle.row_to_f32(dtype, row, n)))


def _matvec_case(gpu, oracle, dtype, rows, cols, scale=1.0):
    W = (rng.standard_normal((rows, cols)) * scale).astype(np.float32)
    Wq = W if dtype == F32 else oracle.quantize(dtype, W)
    x = rng.standard_normal(cols).astype(np.float32)
    want, want_xq = oracle.matvec(dtype, Wq, rows, cols, x)
    L = gpu.load_library()
    h = L.qmh_weight_upload(dtype, rows, cols, np.ascontiguousarray(Wq).ctypes.data)
    assert h, gpu.last_error()
    try:
        dx, dy, dq = dev(gpu, x), gpu.DeviceBuffer(rows * 4), gpu.DeviceBuffer(nblocks(cols) * 34)
        gpu._check(L.qmh_matvec(h, dx.ptr, dy.ptr, dq.ptr, None), "matvec")
        got = dy.to_array(np.float32)
        assert np.array_equal(bits(got), bits(want)), (dtype, rows, cols)
        if dtype != F32:
            assert np.array_equal(dq.to_array(np.uint8), want_xq)
    finally:
        L.qmh_weight_free(h)


@pytest.mark.parametrize("dtype", [F32, Q8_0, Q4_0])
def test_matvec_random_shapes(gpu, oracle, dtype):
    for it in range(25):
        _matvec_case(gpu, oracle, dtype, int(rng.integers(1, 300)), int(rng.integers(1, 400)))


@pytest.mark.parametrize("dtype", [Q8_0, Q4_0])
@pytest.mark.parametrize("rows,cols", [(4096, 4096), (11008, 4096), (4096, 11008), (32000, 288), (288, 768)])
def test_matvec_model_shapes(gpu, oracle, dtype, rows, cols):
    _matvec_case(gpu, oracle, dtype, rows, cols, scale=0.02)


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (288, 768), (700, 5000), (33, 4099), (17, 257)])
def test_matvec_f32_shapes(gpu, oracle, rows, cols):
    """f32 weights over several 256-column chunks: whole chunks, a ragged last chunk, n % 4 != 0."""
    _matvec_case(gpu, oracle, F32, rows, cols, scale=0.02)


def test_gemm_nt(gpu, oracle):
    L = gpu.load_library()
    shapes = [(4, 4, 8), (512, 512, 512), (17, 130, 600), (1, 1, 1), (40, 150, 257)]
    shapes += [(int(rng.integers(1, 41)), int(rng.integers(1, 151)), int(rng.integers(1, 601))) for _ in range(10)]
    for M, N, K in shapes:
        A = rng.standard_normal((M, K)).astype(np.float32)
        B = rng.standard_normal((N, K)).astype(np.float32)
        dA, dB, dC = dev(gpu, A), dev(gpu, B), gpu.DeviceBuffer(M * N * 4)
        gpu._check(L.qmh_matmul_nt(dA.ptr, dB.ptr, dC.ptr, M, N, K, None), "gemm")
        got = dC.to_array(np.float32).reshape(M, N)
        assert np.array_equal(bits(got), bits(oracle.gemm_nt(A, B))), (M, N, K)


def test_gemm_nt_empty_k(gpu):
    """K = 0: the reference zeroes C and has no panel to add (src/gemm_driver.h:9-10)."""
    L = gpu.load_library()
    M, N = 37, 70
    dA, dB = gpu.DeviceBuffer(4), gpu.DeviceBuffer(4)
    dC = dev(gpu, np.full(M * N, 7.0, np.float32))
    gpu._check(L.qmh_matmul_nt(dA.ptr, dB.ptr, dC.ptr, M, N, 0, None), "gemm")
    gpu.sync()
    assert np.array_equal(bits(dC.to_array(np.float32)), np.zeros(M * N, np.uint32))


@pytest.mark.parametrize("n", [1, 7, 77, 288, 4096, 11008])
def test_elementwise(gpu, oracle, n):
    L = gpu.load_library()
    x = rng.standard_normal(n).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    dx, dw, do = dev(gpu, x), dev(gpu, w), gpu.DeviceBuffer(n * 4)
    gpu._check(L.qmh_rmsnorm(do.ptr, dx.ptr, dw.ptr, n, 1e-5, None), "rmsnorm")
    assert np.array_equal(bits(do.to_array(np.float32)), bits(oracle.rmsnorm(x, w, 1e-5)))
    s = (x * 6).astype(np.float32)
    ds = dev(gpu, s)
    gpu._check(L.qmh_softmax(ds.ptr, n, None), "softmax")
    assert np.array_equal(bits(ds.to_array(np.float32)), bits(oracle.softmax(s)))
    dg, du = dev(gpu, x * 8), dev(gpu, w)
    gpu._check(L.qmh_swiglu(dg.ptr, du.ptr, n, None), "swiglu")
    assert np.array_equal(bits(dg.to_array(np.float32)), bits(oracle.swiglu((x * 8).astype(np.float32), w)))
    di = gpu.DeviceBuffer(4)
    gpu._check(L.qmh_argmax(dx.ptr, n, di.ptr, None), "argmax")
    assert di.to_array(np.int32)[0] == oracle.argmax(x)


def test_softmax_and_argmax_known_answers(gpu):
    L = gpu.load_library()
    s = np.array([1000.0, 1001.0, 999.0, -1e30, 1001.0], np.float32)
    ds = dev(gpu, s)
    gpu._check(L.qmh_softmax(ds.ptr, 5, None), "softmax")
    p = ds.to_array(np.float32)
    assert abs(p.sum() - 1.0) < 1e-6 and p[1] == p[4] and p[1] > p[0] and p[3] == 0.0
    lg = np.array([1.0, 3.0, 0.5, 2.5, -1.0, 3.0], np.float32)
    di = gpu.DeviceBuffer(4)
    gpu._check(L.qmh_argmax(dev(gpu, lg).ptr, 6, di.ptr, None), "argmax")
    assert di.to_array(np.int32)[0] == 1
    # ties across a long vector: the first index wins
    big = np.zeros(100000, np.float32)
    big[[777, 5000, 99999]] = 2.0
    gpu._check(L.qmh_argmax(dev(gpu, big).ptr, big.size, di.ptr, None), "argmax")
    assert di.to_array(np.int32)[0] == 777


@pytest.mark.parametrize("nh,hd,pos", [(2, 12, 37), (6, 48, 255), (32, 128, 4095), (4, 64, 0)])
def test_rope(gpu, oracle, nh, hd, pos):
    v = rng.standard_normal(nh * hd).astype(np.float32)
    dv = dev(gpu, v)
    gpu._check(gpu.load_library().qmh_rope(dv.ptr, nh, hd, pos, 10000.0, None), "rope")
    assert np.array_equal(bits(dv.to_array(np.float32)), bits(oracle.rope(v, nh, hd, pos, 10000.0)))


# ---- inputs at a float rounding boundary of the double sums (serial fallback paths)

@pytest.mark.parametrize("n", [64, 288, 4096, 11008])
def test_rmsnorm_boundary(gpu, oracle, n):
    from _boundary import rmsnorm_boundary_input

    L = gpu.load_library()
    for seed in range(6):
        x = rmsnorm_boundary_input(n, 1e-5, seed)
        w = np.random.default_rng(seed).standard_normal(n).astype(np.float32)
        dx, dw, do = dev(gpu, x), dev(gpu, w), gpu.DeviceBuffer(n * 4)
        gpu._check(L.qmh_rmsnorm(do.ptr, dx.ptr, dw.ptr, n, 1e-5, None), "rmsnorm")
        assert np.array_equal(bits(do.to_array(np.float32)), bits(oracle.rmsnorm(x, w, 1e-5))), (n, seed)


@pytest.mark.parametrize("dtype", [F32, Q8_0, Q4_0])
@pytest.mark.parametrize("n", [64, 288, 4096])
def test_rmsnorm_matvec_boundary_and_random(gpu, oracle, dtype, n):
    """The fused RMSNorm prologue of the matvec: boundary inputs (serial fallback) and plain
    random ones, against rmsnorm then matvec in the oracle."""
    from _boundary import rmsnorm_boundary_input

    L = gpu.load_library()
    rows = 200
    W = (rng.standard_normal((rows, n)) * 0.05).astype(np.float32)
    Wq = W if dtype == F32 else oracle.quantize(dtype, W)
    h = L.qmh_weight_upload(dtype, rows, n, np.ascontiguousarray(Wq).ctypes.data)
    assert h, gpu.last_error()
    try:
        for seed in range(4):
            x = rmsnorm_boundary_input(n, 1e-5, seed) if seed < 3 else rng.standard_normal(n).astype(np.float32)
            g = (1.0 + 0.1 * np.random.default_rng(seed).standard_normal(n)).astype(np.float32)
            xn = oracle.rmsnorm(x, g, 1e-5)
            want, want_xq = oracle.matvec(dtype, Wq, rows, n, xn)
            dx, dg, dy = dev(gpu, x), dev(gpu, g), gpu.DeviceBuffer(rows * 4)
            dq = gpu.DeviceBuffer(nblocks(n) * 34)
            gpu._check(L.qmh_rmsnorm_matvec(h, dx.ptr, dg.ptr, 1e-5, dy.ptr, dq.ptr, None), "rmsnorm_matvec")
            assert np.array_equal(bits(dy.to_array(np.float32)), bits(want)), (dtype, n, seed)
            if dtype != F32:
                assert np.array_equal(dq.to_array(np.uint8), want_xq)
    finally:
        L.qmh_weight_free(h)


@pytest.mark.parametrize("n", [64, 4096])
def test_rmsnorm_matvec_near_margin(gpu, oracle, n):
    """The prologue's inverse RMS without the exact double chain (v_rsq_f64, Newton steps, margin
    test): inputs whose 1/sqrt(ss/n + eps) sits 2^-44 .. 2^-36 (relative) from a float midpoint,
    either side, i.e. just outside and inside the margin (2^-40.7 at n = 4096, 2^-45.3 at 64)."""
    from _boundary import rmsnorm_offset_input

    L = gpu.load_library()
    rows = 64
    W = (rng.standard_normal((rows, n)) * 0.05).astype(np.float32)
    Wq = oracle.quantize(Q8_0, W)
    h = L.qmh_weight_upload(Q8_0, rows, n, np.ascontiguousarray(Wq).ctypes.data)
    assert h, gpu.last_error()
    try:
        for e in (44, 42, 40, 38, 36):
            for sign in (1.0, -1.0):
                for seed in range(2):
                    x = rmsnorm_offset_input(n, 1e-5, seed, sign * 2.0 ** -e)
                    g = np.ones(n, np.float32)
                    want, _ = oracle.matvec(Q8_0, Wq, rows, n, oracle.rmsnorm(x, g, 1e-5))
                    dx, dg, dy = dev(gpu, x), dev(gpu, g), gpu.DeviceBuffer(rows * 4)
                    dq = gpu.DeviceBuffer(nblocks(n) * 34)
                    gpu._check(L.qmh_rmsnorm_matvec(h, dx.ptr, dg.ptr, 1e-5, dy.ptr, dq.ptr, None), "rmsnorm_matvec")
                    assert np.array_equal(bits(dy.to_array(np.float32)), bits(want)), (n, e, sign, seed)
    finally:
        L.qmh_weight_free(h)


@pytest.mark.parametrize("n", [7, 64, 512, 4096])
def test_softmax_boundary(gpu, oracle, n):
    from _boundary import softmax_boundary_input

    L = gpu.load_library()
    for seed in range(6):
        s = softmax_boundary_input(n, seed)
        ds = dev(gpu, s)
        gpu._check(L.qmh_softmax(ds.ptr, n, None), "softmax")
        assert np.array_equal(bits(ds.to_array(np.float32)), bits(oracle.softmax(s))), (n, seed)


def test_argmax_nan_and_inf_semantics(gpu, oracle):
    """`if (x[i] > x[best]) best = i` from best = 0: NaN at 0 wins, other NaNs never do."""
    L = gpu.load_library()
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    cases = [
        [nan, 1.0, 2.0],
        [1.0, nan, 2.0, nan],
        [nan] * 5,
        [-inf, -inf, -inf],
        [-inf, nan, -inf, -1.0],
        [3.0, inf, nan, inf],
        [0.0, -0.0, 0.0],
    ]
    big = np.full(40000, -1.0, np.float32)
    big[::7] = nan
    big[12345], big[30001] = 5.0, 5.0
    cases.append(big)
    big2 = big.copy()
    big2[0] = nan
    cases.append(big2)
    di = gpu.DeviceBuffer(4)
    for c in cases:
        x = np.asarray(c, np.float32)
        gpu._check(L.qmh_argmax(dev(gpu, x).ptr, x.size, di.ptr, None), "argmax")
        assert di.to_array(np.int32)[0] == oracle.argmax(x), c[:6]


@pytest.mark.parametrize("n", [1, 3, 4, 5, 31999, 32000, 32001, 32768, 32771, 100003])
def test_argmax_vector_and_scalar_loads(gpu, oracle, n):
    """16-byte loads from an aligned vector (with the n % 4 tail), 4-byte loads from one that starts
    4 bytes past a 16-byte boundary: the same first index of the maximum, NaNs and ties included."""
    L = gpu.load_library()
    r = np.random.default_rng(n)
    x = r.standard_normal(n).astype(np.float32)
    x[r.integers(0, n, size=max(1, n // 50))] = np.float32(np.nan)
    top = r.integers(0, n, size=3)
    x[top] = np.float32(9.0)  # ties: the lowest of these indices wins unless it is NaN'd below
    if n > 8:
        x[top[0]] = np.float32(np.nan)
    di = gpu.DeviceBuffer(4)
    gpu._check(L.qmh_argmax(dev(gpu, x).ptr, n, di.ptr, None), "argmax")
    assert di.to_array(np.int32)[0] == oracle.argmax(x)
    padded = dev(gpu, np.concatenate([np.zeros(1, np.float32), x]))
    gpu._check(L.qmh_argmax(padded.ptr + 4, n, di.ptr, None), "argmax")
    assert di.to_array(np.int32)[0] == oracle.argmax(x)
