"""The reference's own CLI and bench on the device path (oracle/hip_integration.patch):
`quillm run --isa hip` (and QUILLM_ISA=hip) prints exactly the text `--isa scalar` prints, greedy and
sampled, and `QUILLM_ISA=hip quillm-bench` completes its decode loop with a hip column and prints
device GFLOP/s for its matvec and gemm kernel rows -- the reference's cross-ISA identity check
(tests/test_cli.sh:14-19) with hip added."""
import os
import re
import subprocess
import sys

import pytest

from _cli import BENCH_HIP, PROMPT, QUILLM, QUILLM_HIP, run_cli
from _qlm import add_byte_pair_merges

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def c2_model(gpu, tmp_path_factory):
    for exe in (QUILLM, QUILLM_HIP, BENCH_HIP):
        if not os.path.exists(exe):
            pytest.fail(f"{exe} missing: run __graft_entry__.build() first")
    d = tmp_path_factory.mktemp("cli")
    w = gpu.WORKLOADS["c2"]
    raw, path = str(d / "c2_raw.qlm"), str(d / "c2.qlm")
    gpu.gen_model(raw, w.config(), w.wtype, seed=w.seed, threads=4)
    add_byte_pair_merges(raw, path, w.vocab_size - 258)
    os.remove(raw)
    return path


@pytest.mark.parametrize("args", [["--temp", "0"], ["--temp", "0.8", "--top-p", "0.95", "--seed", "7"]])
def test_cli_hip_prints_the_scalar_text(c2_model, args):
    common = ["-p", PROMPT, "-n", "200", "-t", "2", *args]
    say("cli scalar", args)
    rc0, out0, err0 = run_cli(QUILLM, c2_model, *common, "--isa", "scalar")
    say("cli hip", args)
    rc1, out1, err1 = run_cli(QUILLM_HIP, c2_model, *common, "--isa", "hip")
    rc2, out2, err2 = run_cli(QUILLM_HIP, c2_model, *common, env={"QUILLM_ISA": "hip"})
    assert rc0 == 0 and rc1 == 0 and rc2 == 0, err0 + err1 + err2
    assert "isa=hip" in err1 and "isa=hip" in err2, err1 + err2
    assert len(out0) > len(PROMPT) + 100
    assert out1 == out0
    assert out2 == out0


def test_bench_hip_decode_loop(c2_model):
    env = dict(os.environ, QUILLM_ISA="hip", QM_BENCH_THREADS="2")
    say("bench hip")
    r = subprocess.run([BENCH_HIP, c2_model], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    rows = [line for line in r.stdout.splitlines() if line.startswith(os.path.basename(c2_model))]
    assert len(rows) == 2, r.stdout  # 1 thread and QM_BENCH_THREADS threads
    for row in rows:
        m = re.search(r" hip\s+([0-9.]+)", row)
        assert m and float(m.group(1)) > 0, row
    # the kernel rows' hip column: device time per qmh_matvec / qmh_matmul_nt call
    kern = [line for line in r.stdout.splitlines() if line.startswith(("matvec", "gemm"))]
    assert len(kern) == 8, r.stdout
    for line in kern:
        assert float(line.split()[-1]) > 0, line
    dot = [line for line in r.stdout.splitlines() if line.startswith("dot f32")]
    assert dot and dot[0].split()[-1] == "n/a", r.stdout
