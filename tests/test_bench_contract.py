"""bench.py's contract on the CPU side (no GPU):

* one GPU only: `--gpus N` with N != 1 exits with status 2 and says why, before any device work;
* the roofline's `traffic` comes from the committed counter summary of the dominant kernel, and that
  summary's figure is FETCH_SIZE + WRITE_SIZE per launch, within a few percent of the algorithmic bytes
  (the W1|W3 Q4_0 codes and fp16 scales of the c5a shape: 2 x 11008 rows x 128 blocks x 18 bytes).
"""
import importlib.util
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def load_bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""


def test_roofline_traffic_from_committed_counters():
    bench = load_bench()
    traffic = bench.pmc_traffic("k_matvec_w13_q4_0_c5a_pmc.txt")
    algorithmic = 2 * 11008 * (4096 // 32) * 18
    assert algorithmic == 50724864
    assert traffic is not None and 1.0 <= traffic / algorithmic < 1.05
    assert bench.pmc_traffic("no_such_summary.txt") is None
