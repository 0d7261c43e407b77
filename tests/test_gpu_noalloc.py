"""The device path's library code performs no heap allocation per token, as the reference's forward
does not (src/model.h:35; its tests/test_noalloc.c:7-40 counts malloc/calloc/realloc/aligned_alloc
over max_seq decode steps). tests/noalloc/noalloc_check (its own process) replaces the allocator and
counts every heap allocation in the process over max_seq qmh_model_forward calls, a qmh_model_greedy
and a qmh_model_sample run, attributing each to libqmhip.so or to the HIP runtime call it came from;
loading is checked to allocate (the count is live). The HIP runtime itself allocates small objects in
its launch and copy calls (hipGraphLaunch, hipMemcpyAsync, ...): measured at 22-29 per decode step
and 43 per sampled step, held to per-phase bounds 10-20% above that, so that a regression shows.
The same binary then checks
qmh_sample_noalloc: no heap allocation by the library over 64 calls at vocabularies above and below
8192, the device's free memory unchanged across them, and the draw captured in a HIP graph replaying
the eager draws of a sampler object token for token and rng state for rng state."""
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
    # the HIP runtime's per-call bookkeeping per step, measured at 28.5 (forward: a graph replay and two
    # copies), 21.8 (greedy: a graph replay) and 43.4 (sampled: a replay and the sampler's launches at
    # vocabulary 32000) on c2; the bounds leave ~10-20% so that a regression shows
    bound = {"qmh_model_forward": 32, "qmh_model_greedy": 26, "qmh_model_sample": 48}
    for phase in ("qmh_model_forward", "qmh_model_greedy", "qmh_model_sample"):
        total, own = rows[phase]
        print(f"{phase}: {total / max_seq:.1f} heap allocations per step (HIP runtime), {own} by the library")
        # the library's own code allocates nothing per token (the reference's contract)
        assert own == 0, f"{phase}: {own} heap allocations by libqmhip.so\n{r.stdout}"
        # bounded per step, never growing with the context
        assert total <= bound[phase] * max_seq, \
            f"{phase}: {total} heap allocations ({total / max_seq:.1f} per step)\n{r.stdout}"
    total, own = rows["qmh_sample_noalloc"]
    assert own == 0, f"qmh_sample_noalloc: {own} heap allocations by libqmhip.so\n{r.stdout}"
    assert total <= 32 * 64, r.stdout
    assert "device free bytes" in r.stdout and "(unchanged)" in r.stdout, r.stdout
    assert "graph replays matching the eager draws: 8 of 8" in r.stdout, r.stdout
