"""Pin the CPU oracle (our C restatement) against the compiled reference, the reference's own
known-answer tests, and closed forms. CPU only."""
import numpy as np
import pytest

from _bind import F32, Q4_0, Q8_0, accum_tol, nblocks

rng = np.random.default_rng(20261201)


# ---------------------------------------------------------------------------- fp16

def test_fp16_known_answers(oracle, ref):
    # reference tests/test_fp16.c:29-38
    kats = [(1.0, 0x3C00), (-2.0, 0xC000), (65504.0, 0x7BFF), (65519.0, 0x7BFF), (65520.0, 0x7C00),
            (5.9604644775390625e-08, 0x0001), (2.98023223876953125e-08, 0x0000), (-0.0, 0x8000)]
    for f, h in kats:
        assert oracle.L.or_f2h(f) == h, f
        assert ref.L.qm_fp32_to_fp16(f) == h, f
    assert oracle.L.or_h2f(0x3555) == np.float32(0.333251953125)
    nan_h = oracle.L.or_f2h(float("nan"))
    assert (nan_h & 0x7C00) == 0x7C00 and (nan_h & 0x3FF)


def test_fp16_exhaustive_halves(oracle, ref):
    h = np.arange(65536, dtype=np.uint16)
    f = oracle.h2f(h)
    # (ctypes returns the reference's float through a double, which quiets signalling NaNs,
    # so NaNs are compared by class here and by bit layout below)
    ref_f = np.array([ref.L.qm_fp16_to_fp32(int(x)) for x in h], np.float32)
    isn = np.isnan(ref_f)
    assert np.array_equal(np.isnan(f), isn)
    assert np.array_equal(f[~isn].view(np.uint32), ref_f[~isn].view(np.uint32))
    # NaN/inf halves keep sign and payload: bits = sign | 0x7f800000 | mant << 13 (src/fp16.c:27)
    hi = h[(h & 0x7C00) == 0x7C00].astype(np.uint32)
    want = ((hi & 0x8000) << 16) | 0x7F800000 | ((hi & 0x3FF) << 13)
    assert np.array_equal(f[(h & 0x7C00) == 0x7C00].view(np.uint32), want)
    # numpy's float16 is IEEE binary16: an independent decoder
    npf = h.view(np.float16).astype(np.float32)
    notnan = ~np.isnan(npf)
    assert np.array_equal(f[notnan].view(np.uint32), npf[notnan].view(np.uint32))
    # round trip for every non-NaN half
    assert np.array_equal(oracle.f2h(f[notnan]), h[notnan])


def test_fp16_encode_sweep(oracle, ref):
    # strided sweep of all 2^32 bit patterns (like tests/test_fp16.c:53-66) + values near the half range
    u = np.arange(0, 1 << 32, 65537 * 3, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([u.view(np.float32), ((rng.random(200000) - 0.5) *
                                             np.exp2(rng.integers(-30, 18, 200000))).astype(np.float32)])
    got = oracle.f2h(x)
    want = np.array([ref.L.qm_fp32_to_fp16(float(v)) for v in x[:60000]], np.uint16)
    assert np.array_equal(got[:60000], want)
    # numpy (IEEE RNE) agrees on every non-NaN input
    fin = ~np.isnan(x)
    with np.errstate(over="ignore"):
        assert np.array_equal(got[fin], x[fin].astype(np.float16).view(np.uint16))


# ---------------------------------------------------------------------------- quantization

def _rows(n, scale, outlier=True):
    x = (rng.standard_normal((3, n)) * scale).astype(np.float32)
    if outlier:
        x[1, rng.integers(0, n)] *= 50.0
    return x


@pytest.mark.parametrize("dtype", [Q8_0, Q4_0])
def test_quantize_bytes_match_reference(oracle, ref, dtype):
    for it in range(200):
        n = int(rng.integers(1, 701))
        x = _rows(n, float(np.exp2(rng.integers(-12, 13))))
        if it % 7 == 0:
            x[0, : min(n, 40)] = 0.0  # all-zero block
        assert np.array_equal(oracle.quantize(dtype, x), ref.quantize(dtype, x)), n


@pytest.mark.parametrize("dtype", [F32, Q8_0, Q4_0])
def test_row_to_f32_bitexact_vs_reference(oracle, ref, dtype):
    """or_row_to_f32 against the compiled qm_row_to_f32 (src/quant.c:65-101) on rows of every length
    1..300 and 4096: quantized rows from the reference's quantizer (zero blocks, subnormal and large
    scales), raw random bytes as codes and scales (every code value, NaN/inf/subnormal fp16 scales),
    and f32 rows."""
    for n in list(range(1, 301)) + [4096]:
        if dtype == F32:
            rows = [rng.standard_normal(n).astype(np.float32).view(np.uint8),
                    rng.integers(0, 256, 4 * n, dtype=np.uint8)]
        else:
            x = _rows(n, float(np.exp2(rng.integers(-20, 20))))
            if n % 5 == 0:
                x[0, : min(n, 40)] = 0.0
            q = ref.quantize(dtype, x)
            rows = [q[0], q[1], rng.integers(0, 256, q.shape[1], dtype=np.uint8)]
        for row in rows:
            a, b = oracle.row_to_f32(dtype, row, n), ref.row_to_f32(dtype, row, n)
            # NaN scales give NaN values whose payload bits are the x86 conversion's in both
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (dtype, n)


def test_quantize_known_answers(oracle):
    # zero input -> zero scale, zero codes; Q4 byte 0x88 (reference tests/test_quant.c:61-68)
    z = np.zeros(64, np.float32)
    q8, q4 = oracle.quantize(Q8_0, z)[0], oracle.quantize(Q4_0, z)[0]
    assert q8[0] == 0 and q8[1] == 0 and q8[34 + 2 + 5] == 0
    assert q4[18] == 0 and q4[19] == 0 and q4[18 + 2 + 3] == 0x88
    # large magnitudes stay finite and close (tests/test_quant.c:70-75)
    big = ((np.arange(32) - 16) * 3000.0).astype(np.float32)
    d = oracle.row_to_f32(Q8_0, oracle.quantize(Q8_0, big)[0], 32)
    assert np.all(np.isfinite(d)) and np.all(np.abs(d - big) < 300.0)
    # x[3] = -254 -> d = fp16(2.0) = 0x4000, code -127 (tests/test_python.py:32-36)
    x = np.zeros(32, np.float32)
    x[3] = -254.0
    b = oracle.quantize(Q8_0, x)[0]
    assert int(b[0]) | int(b[1]) << 8 == 0x4000 and np.int8(b[2 + 3]) == -127


@pytest.mark.parametrize("dtype", [Q8_0, Q4_0])
def test_quantize_error_bounds(oracle, dtype):
    # per-element bound d/2 + clamp term, padding quantizes to 0 (tests/test_quant.c:5-51)
    qmax = 127.0 if dtype == Q8_0 else 7.0
    for n in (1, 31, 32, 33, 100, 257, 700):
        x = _rows(n, 3.0)[0]
        blk = oracle.quantize(dtype, x)[0]
        y = oracle.row_to_f32(dtype, blk, n)
        bs = 34 if dtype == Q8_0 else 18
        for b in range(nblocks(n)):
            dd = oracle.L.or_h2f(int(blk[b * bs]) | int(blk[b * bs + 1]) << 8)
            seg = slice(b * 32, min(n, b * 32 + 32))
            amax = float(np.abs(x[seg]).max())
            bound = 0.5 * dd + max(0.0, amax - qmax * dd) + 1e-6 * amax
            assert np.all(np.abs(x[seg] - y[seg]) <= bound)
        if n % 32:
            full = oracle.row_to_f32(dtype, blk, nblocks(n) * 32)
            assert np.all(full[n:] == 0.0)


# ---------------------------------------------------------------------------- dots, gemm, matvec

def _quant_pair(n):
    w = rng.standard_normal(n).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    return w, x


def test_dots_bitexact_vs_reference_scalar(oracle, ref):
    dot_f32, dot_q8, dot_q4, _ = ref.kernels("scalar")
    for it in range(300):
        n = it if it < 70 else int(rng.integers(1, 3000))
        a, b = _quant_pair(n)
        assert np.float32(oracle.dot_f32(a, b)) == np.float32(dot_f32(a.ctypes.data, b.ctypes.data, n))
        nb = nblocks(max(n, 1))
        if n == 0:
            continue
        w8, w4, x8 = oracle.quantize(Q8_0, a)[0], oracle.quantize(Q4_0, a)[0], oracle.quantize(Q8_0, b)[0]
        g8, r8 = oracle.dot_q8(w8, x8, nb), dot_q8(w8.ctypes.data, x8.ctypes.data, nb)
        g4, r4 = oracle.dot_q4(w4, x8, nb), dot_q4(w4.ctypes.data, x8.ctypes.data, nb)
        assert np.float32(g8).view(np.uint32) == np.float32(r8).view(np.uint32)
        assert np.float32(g4).view(np.uint32) == np.float32(r4).view(np.uint32)


def test_quant_dots_within_float64_bound(oracle):
    # exact integer block oracle in double (tests/test_kernels.c:36-79)
    for it in range(100):
        n = int(rng.integers(1, 2000))
        nb = nblocks(n)
        a, b = _quant_pair(n)
        w8, w4, x8 = oracle.quantize(Q8_0, a)[0], oracle.quantize(Q4_0, a)[0], oracle.quantize(Q8_0, b)[0]
        r8 = a8 = r4 = a4 = 0.0
        for blk in range(nb):
            qx = w8[blk * 34 + 2: blk * 34 + 34].view(np.int8).astype(np.int64)
            xx = x8[blk * 34 + 2: blk * 34 + 34].view(np.int8).astype(np.int64)
            by = w4[blk * 18 + 2: blk * 18 + 18]
            q4 = np.empty(32, np.int64)
            q4[0::2], q4[1::2] = (by & 15).astype(np.int64) - 8, (by >> 4).astype(np.int64) - 8
            dx = oracle.L.or_h2f(int(x8[blk * 34]) | int(x8[blk * 34 + 1]) << 8)
            t8 = float((qx * xx).sum()) * oracle.L.or_h2f(int(w8[blk * 34]) | int(w8[blk * 34 + 1]) << 8) * dx
            t4 = float((q4 * xx).sum()) * oracle.L.or_h2f(int(w4[blk * 18]) | int(w4[blk * 18 + 1]) << 8) * dx
            r8, a8, r4, a4 = r8 + t8, a8 + abs(t8), r4 + t4, a4 + abs(t4)
        assert abs(oracle.dot_q8(w8, x8, nb) - r8) <= accum_tol(nb * 8, a8)
        assert abs(oracle.dot_q4(w4, x8, nb) - r4) <= accum_tol(nb * 8, a4)


def test_gemm_nt_bitexact_vs_reference_and_float64(oracle, ref):
    _, _, _, gemm = ref.kernels("scalar")
    for it in range(40):
        M, N, K = int(rng.integers(1, 41)), int(rng.integers(1, 151)), int(rng.integers(1, 601))
        if it == 0:
            M, N, K = 4, 4, 8
        A = rng.standard_normal((M, K)).astype(np.float32)
        B = rng.standard_normal((N, K)).astype(np.float32)
        C = oracle.gemm_nt(A, B)
        Cr = np.empty((M, N), np.float32)
        gemm(A.ctypes.data, B.ctypes.data, Cr.ctypes.data, M, N, K, K, K, N)
        assert np.array_equal(C.view(np.uint32), Cr.view(np.uint32))
        ref64 = A.astype(np.float64) @ B.astype(np.float64).T
        abs64 = np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64)).T
        assert np.all(np.abs(C - ref64) <= accum_tol(K, 1.0) * abs64 + 1e-30)


@pytest.mark.parametrize("dtype", [F32, Q8_0, Q4_0])
def test_matvec_bitexact_vs_reference(oracle, ref, dtype):
    assert ref.select("scalar")
    for it in range(15):
        rows, cols = int(rng.integers(1, 300)), int(rng.integers(1, 400))
        W = rng.standard_normal((rows, cols)).astype(np.float32)
        Wq = W if dtype == F32 else oracle.quantize(dtype, W)
        x = rng.standard_normal(cols).astype(np.float32)
        y, xq = oracle.matvec(dtype, Wq, rows, cols, x)
        yr, xqr = ref.matvec(dtype, np.ascontiguousarray(Wq), rows, cols, x)
        assert np.array_equal(y.view(np.uint32), yr.view(np.uint32))
        if dtype != F32:
            assert np.array_equal(xq, xqr)


# ---------------------------------------------------------------------------- elementwise

def test_elementwise_bitexact_vs_reference(oracle, ref):
    for n in (1, 7, 77, 288, 4096, 11008):
        x = rng.standard_normal(n).astype(np.float32)
        w = rng.standard_normal(n).astype(np.float32)
        out_r = np.empty(n, np.float32)
        ref.L.qm_rmsnorm(out_r.ctypes.data, x.ctypes.data, w.ctypes.data, n, 1e-5)
        assert np.array_equal(oracle.rmsnorm(x, w, 1e-5).view(np.uint32), out_r.view(np.uint32))
        s = (x * 4).astype(np.float32)
        sr = s.copy()
        ref.L.qm_softmax(sr.ctypes.data, n)
        assert np.array_equal(oracle.softmax(s).view(np.uint32), sr.view(np.uint32))
        g, u = x.copy(), w.copy()
        ref.L.qm_swiglu(g.ctypes.data, u.ctypes.data, n)
        assert np.array_equal(oracle.swiglu(x, w).view(np.uint32), g.view(np.uint32))
        assert oracle.argmax(x) == ref.L.qm_argmax(x.ctypes.data, n)
    for nh, hd, pos in ((2, 12, 37), (6, 48, 255), (32, 128, 4095), (4, 64, 0)):
        v = rng.standard_normal(nh * hd).astype(np.float32)
        vr = v.copy()
        ref.L.qm_rope(vr.ctypes.data, nh, hd, pos, 10000.0)
        assert np.array_equal(oracle.rope(v, nh, hd, pos, 10000.0).view(np.uint32), vr.view(np.uint32))


def test_elementwise_known_answers(oracle):
    # closed forms of reference tests/test_kernels.c:104-138
    n = 77
    x = rng.standard_normal(n).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    y = oracle.rmsnorm(x, w, 1e-5)
    inv = 1.0 / np.sqrt((x.astype(np.float64) ** 2).sum() / n + 1e-5)
    assert np.all(np.abs(y - x * inv * w) < 1e-5 * (1 + np.abs(x * inv * w)))
    s = oracle.softmax(np.array([1000.0, 1001.0, 999.0, -1e30, 1001.0], np.float32))
    assert abs(s.sum() - 1.0) < 1e-6 and s[1] == s[4] and s[1] > s[0] and s[3] == 0.0
    v0 = rng.standard_normal(24).astype(np.float32)
    assert np.array_equal(oracle.rope(v0, 2, 12, 0, 10000.0), v0)
    v = oracle.rope(v0, 2, 12, 37, 10000.0)
    for h in range(2):
        for i in range(6):
            ang = 37.0 * 10000.0 ** (-2.0 * i / 12.0)
            p, q = v[h * 12 + 2 * i: h * 12 + 2 * i + 2], v0[h * 12 + 2 * i: h * 12 + 2 * i + 2]
            assert abs(p[0] - (q[0] * np.cos(ang) - q[1] * np.sin(ang))) < 1e-5
            assert abs(p[1] - (q[0] * np.sin(ang) + q[1] * np.cos(ang))) < 1e-5
    g = oracle.swiglu(np.array([0.0, 2.0, -3.0], np.float32), np.array([5.0, 0.5, 2.0], np.float32))
    assert g[0] == 0.0 and abs(g[1] - 2.0 / (1.0 + np.exp(-2.0)) * 0.5) < 1e-6
    assert abs(g[2] - (-3.0 / (1.0 + np.exp(3.0)) * 2.0)) < 1e-6
    # argmax picks the first maximum (tests/test_sampler.c:8-12)
    assert oracle.argmax(np.array([1.0, 3.0, 0.5, 2.5, -1.0, 3.0], np.float32)) == 1
