"""The reference's own callers through the boundary, CPU side: oracle/hip_integration.patch only
inserts lines, and with it applied the reference CLI's CPU path is unchanged (the same text as the
unmodified CLI for greedy and sampled generation), while `--isa hip` without a gfx950 device is
refused the way the reference refuses an unavailable ISA (src/main.c:90-96)."""
import os
import re

import pytest

from _cli import PROMPT, QUILLM, QUILLM_HIP, run_cli
from _qlm import add_byte_pair_merges

HERE = os.path.dirname(os.path.abspath(__file__))
PATCH = os.path.join(os.path.dirname(HERE), "oracle", "hip_integration.patch")


def test_patch_only_inserts_lines():
    text = open(PATCH).read().split("\n")
    start = next(i for i, line in enumerate(text) if line.startswith("--- a/"))
    hunks = 0
    for line in text[start:]:
        if line.startswith(("--- a/", "+++ b/")) or line == "":
            continue
        if line.startswith("@@"):
            assert re.match(r"@@ -\d+,0 \+\d+,\d+ @@$", line), line  # no line of the original is consumed
            hunks += 1
            continue
        assert line.startswith("+"), line
    assert hunks >= 10


@pytest.fixture(scope="module")
def c2_model(qmh, tmp_path_factory):
    """The c2 shape (stories15M, Q4_0, GQA 6/2, vocabulary 32000) with a tokenizer whose every id decodes
    to text."""
    if not (os.path.exists(QUILLM) and os.path.exists(QUILLM_HIP)):
        pytest.fail("oracle/_ref/quillm(-hip) missing: run __graft_entry__.build() first")
    d = tmp_path_factory.mktemp("cli")
    w = qmh.WORKLOADS["c2"]
    raw, path = str(d / "c2_raw.qlm"), str(d / "c2.qlm")
    qmh.gen_model(raw, w.config(), w.wtype, seed=w.seed, threads=4)
    add_byte_pair_merges(raw, path, w.vocab_size - 258)
    os.remove(raw)
    return path


@pytest.mark.parametrize("args", [["--temp", "0"], ["--temp", "0.8", "--top-p", "0.95", "--seed", "7"]])
def test_patched_cli_cpu_path_unchanged(c2_model, args):
    common = ["-p", PROMPT, "-n", "40", "--no-stats", "-t", "2", "--isa", "scalar", *args]
    rc0, out0, err0 = run_cli(QUILLM, c2_model, *common)
    rc1, out1, err1 = run_cli(QUILLM_HIP, c2_model, *common)
    assert rc0 == 0 and rc1 == 0, err0 + err1
    assert len(out0) > len(PROMPT) + 20  # the prompt echo plus generated text
    assert out1 == out0


def test_hip_isa_refused_without_device(qmh, c2_model):
    if qmh.available():
        pytest.skip("a gfx950 device is visible: tests/test_gpu_integration.py runs the hip ISA")
    rc, out, err = run_cli(QUILLM_HIP, c2_model, "-p", PROMPT, "--isa", "hip")
    assert rc == 1 and "ISA 'hip' not available" in err
