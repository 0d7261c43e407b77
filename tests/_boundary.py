"""Inputs whose double-precision sums sit on a float rounding boundary -- TEST INFRASTRUCTURE.

The reference sums RMSNorm's squares and softmax's exponentials serially in double and rounds
a monotone function of the sum to float (src/ops.c:93-112). These builders place that function
within about 2^-46 (relative) of the midpoint between two adjacent floats, so the float result
depends on the last bits of the sum and a summation order other than the serial one can flip
it. The device kernels must detect such inputs and take their serial path.
"""
import ctypes
import math

import numpy as np

_libm = ctypes.CDLL("libm.so.6")
_libm.expf.restype = ctypes.c_float
_libm.expf.argtypes = [ctypes.c_float]


def glibc_expf(x: np.float32) -> np.float32:
    """glibc's expf, the function the reference links."""
    return np.float32(_libm.expf(float(x)))


def serial_sum(terms64: np.ndarray) -> float:
    """Left-to-right double sum (np.cumsum accumulates sequentially)."""
    return float(np.cumsum(terms64)[-1]) if terms64.size else 0.0


def rms_inv(ss: float, n: int, eps: float) -> np.float32:
    return np.float32(1.0 / math.sqrt(ss / n + float(np.float32(eps))))


def slack(s: float, n: int) -> float:
    """The device's bound on |serial sum - tree sum| (qmh_sum_slack)."""
    return s * (n * 2.5 + 8.0) * 2.0 ** -53


def _midpoint(f: np.float32) -> float:
    g = np.nextafter(f, np.float32(np.inf))
    return (float(f) + float(g)) / 2.0


def _largest_float_sq_at_most(r: float) -> np.float32:
    a = np.float32(math.sqrt(r))
    while float(a) * float(a) > r:
        a = np.nextafter(a, np.float32(0))
    return a


def rmsnorm_boundary_input(n: int, eps: float, seed: int, target: float = 0.73) -> np.ndarray:
    """x[n] (n >= 4) whose serial sum of squares lands within about an ulp of the sum that maps
    1/sqrt(sum/n + eps) onto a float midpoint."""
    rng = np.random.default_rng(seed)
    m = _midpoint(np.float32(target * (1.0 + 0.01 * rng.random())))
    ss_t = n * (1.0 / (m * m) - float(np.float32(eps)))
    bulk = rng.standard_normal(n - 3)
    bulk = (bulk * math.sqrt(0.5 * ss_t / float(np.sum(bulk * bulk)))).astype(np.float32)
    p = serial_sum(bulk.astype(np.float64) ** 2)
    tail = []
    for _ in range(3):  # each element closes the remaining gap to about 2^-24 of itself
        a = _largest_float_sq_at_most(max(ss_t - p, 0.0))
        tail.append(a)
        p = p + float(a) * float(a)
    return np.concatenate([bulk, np.array(tail, np.float32)])


def rmsnorm_offset_input(n: int, eps: float, seed: int, rel: float, target: float = 0.73) -> np.ndarray:
    """x[n] (n >= 4) whose 1/sqrt(sum/n + eps) sits at (1 + rel) times a float midpoint: just
    outside (or inside) the device's margin for taking the float without the exact double chain."""
    rng = np.random.default_rng(seed)
    m = _midpoint(np.float32(target * (1.0 + 0.01 * rng.random()))) * (1.0 + rel)
    ss_t = n * (1.0 / (m * m) - float(np.float32(eps)))
    bulk = rng.standard_normal(n - 3)
    bulk = (bulk * math.sqrt(0.5 * ss_t / float(np.sum(bulk * bulk)))).astype(np.float32)
    p = serial_sum(bulk.astype(np.float64) ** 2)
    tail = []
    for _ in range(3):
        a = _largest_float_sq_at_most(max(ss_t - p, 0.0))
        tail.append(a)
        p = p + float(a) * float(a)
    return np.concatenate([bulk, np.array(tail, np.float32)])


def softmax_boundary_input(n: int, seed: int) -> np.ndarray:
    """s[n] (n >= 4), max 0, with (float)(1/sum expf(s_i)) within ~2^-45 of a float midpoint."""
    rng = np.random.default_rng(seed)
    bulk = (-5.0 - 4.0 * rng.random(n - 3)).astype(np.float32)
    bulk[rng.integers(0, n - 3)] = np.float32(0.0)  # the maximum, somewhere in the bulk
    p0 = serial_sum(np.array([float(glibc_expf(v)) for v in bulk]))
    m = _midpoint(np.float32(1.0 / (p0 + 0.05 + 0.1 * rng.random())))
    sum_t = 1.0 / m
    out = list(bulk)
    p = p0
    for _ in range(3):  # three elements close the gap to sum_t from below
        r = sum_t - p
        if r <= 0.0:
            out.append(np.float32(-200.0))  # expf underflows to 0
            continue
        a = np.float32(math.log(r))
        while float(glibc_expf(a)) > r:
            a = np.nextafter(a, np.float32(-np.inf))
        while float(glibc_expf(np.nextafter(a, np.float32(np.inf)))) <= r:
            a = np.nextafter(a, np.float32(np.inf))
        out.append(a)
        p = p + float(glibc_expf(a))
    return np.array(out, np.float32)


def softmax_serial_inv(s: np.ndarray) -> np.float32:
    mx = np.float32(np.max(s))
    e = np.array([float(glibc_expf(np.float32(v - mx))) for v in s])
    return np.float32(1.0 / serial_sum(e))
