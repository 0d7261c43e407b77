"""The oracle's RMSNorm and softmax on inputs at a float rounding boundary of their double sums
(tests/_boundary.py): the results are those of the serial left-to-right double sum the reference
performs (src/ops.c:93-112), restated here with numpy's sequential cumsum and glibc's expf, and
on these inputs the pairwise (tree) order gives a different float for a good share of cases --
the reason the device kernels carry a serial fallback."""
import numpy as np
import pytest

from _boundary import (glibc_expf, rms_inv, rmsnorm_boundary_input, serial_sum, slack, softmax_boundary_input,
                       softmax_serial_inv)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.mark.parametrize("n", [64, 288, 4096, 11008])
def test_rmsnorm_boundary_serial_order(oracle, n):
    flips = 0
    for seed in range(8):
        x = rmsnorm_boundary_input(n, 1e-5, seed)
        w = np.random.default_rng(seed).standard_normal(n).astype(np.float32)
        t = x.astype(np.float64) ** 2
        ss = serial_sum(t)
        d = slack(ss, n)
        assert rms_inv(ss - d, n, 1e-5) != rms_inv(ss + d, n, 1e-5)  # on the boundary
        inv = rms_inv(ss, n, 1e-5)
        want = (x * inv).astype(np.float32) * w
        assert np.array_equal(bits(oracle.rmsnorm(x, w, 1e-5)), bits(want.astype(np.float32)))
        flips += rms_inv(float(np.sum(t)), n, 1e-5) != inv
    assert flips >= 1, "the construction no longer separates tree and serial order"


@pytest.mark.parametrize("n", [7, 64, 512, 4096])
def test_softmax_boundary_serial_order(oracle, n):
    for seed in range(6):
        s = softmax_boundary_input(n, seed)
        e = np.array([glibc_expf(np.float32(v - s.max())) for v in s], np.float32)
        S = serial_sum(e.astype(np.float64))
        d = slack(S, n)
        assert np.float32(1.0 / (S - d)) != np.float32(1.0 / (S + d))
        want = e * softmax_serial_inv(s)
        assert np.array_equal(bits(oracle.softmax(s)), bits(want))
