"""The device quantizer computes amax/127 without a division (qmh_div127: one product and two
FMAs). Check it against the IEEE quotient the reference takes (src/quant.c:47) on every
non-negative float, by compiling tests/exhaustive/div127_check.c on the host. CPU only."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def test_div127_equals_ieee_quotient_for_every_nonnegative_float(tmp_path):
    src = os.path.join(HERE, "exhaustive", "div127_check.c")
    exe = str(tmp_path / "div127_check")
    flags = ["-O2", "-std=c11", "-ffp-contract=off"]
    if " fma " in open("/proc/cpuinfo").read():
        flags.append("-mfma")  # hardware fmaf; libm's is correctly rounded too, only slower
    subprocess.run(["gcc", *flags, src, "-o", exe, "-lm"], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches 0" in r.stdout
    assert "checked 2147483647" in r.stdout  # every non-negative bit pattern but +inf, NaNs included
