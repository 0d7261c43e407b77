"""The device path's library code performs no heap allocation per token, as the reference's forward
does not (src/model.h:35; its tests/test_noalloc.c:7-40 counts malloc/calloc/realloc/aligned_alloc
over max_seq decode steps). tests/noalloc/noalloc_check (its own process) replaces the allocator and
counts every heap allocation in the process over max_seq qmh_model_forward calls, a qmh_model_greedy
and a qmh_model_sample run, attributing each to libqmhip.so or to the HIP runtime call it came from;
loading is checked to allocate (the count is live). The HIP runtime itself allocates small objects in
its launch and copy calls (hipGraphLaunch, hipMemcpyAsync, ...): those are bounded per step."""
import os
import re
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CHECK = os.path.join(HERE, "noalloc", "noalloc_check")

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape,wt", [("gqa", "q4_0"), ("small", "q8_0"), ("c2", "q4_0")])
def test_decode_makes_no_heap_allocation(gpu, small_models, tmp_path, shape, wt):
    if not os.path.exists(CHECK):
        pytest.fail(f"{CHECK} missing: run __graft_entry__.build() first")
    if shape == "c2":  # vocabulary 32000: the sampler's multi-workgroup path
        w = gpu.WORKLOADS["c2"]
        path, max_seq = str(tmp_path / "c2.qlm"), 64
        gpu.gen_model(path, w.config(), w.wtype, seed=w.seed, threads=4)
    else:
        path, max_seq = small_models[(shape, wt)], 48
    print(f"noalloc {shape}/{wt} max_seq {max_seq}", flush=True)
    sys.stdout.flush()
    r = subprocess.run([CHECK, path, str(max_seq)], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    rows = {m.group(1): (int(m.group(2)), int(m.group(3))) for m in
            re.finditer(r"^(\S[^:]*): \d+ steps, (\d+) heap allocations, (\d+) by the library", r.stdout, re.M)}
    assert rows["load (expected to allocate)"][0] > 0  # the count is live
    for phase in ("qmh_model_forward", "qmh_model_greedy", "qmh_model_sample"):
        total, own = rows[phase]
        # the library's own code allocates nothing per token (the reference's contract)
        assert own == 0, f"{phase}: {own} heap allocations by libqmhip.so\n{r.stdout}"
        # the HIP runtime's per-call bookkeeping: bounded per step, never growing with the context
        assert total <= 64 * max_seq, f"{phase}: {total} heap allocations\n{r.stdout}"
