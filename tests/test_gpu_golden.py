"""Whole-model parity with the compiled reference at every BASELINE config, replayed from the
committed fixtures in tests/golden/ (written by tests/golden/make_golden.py from the reference's
scalar ISA): the generated .qlm is byte-identical (xxh64), the logits at every prompt and decode
position are bit-identical (xxh64 of the float32 bytes), and the device greedy loop emits the
reference's ids at every step -- 128 steps at the 7B Q4_0 shape c5a."""
import glob
import json
import os
import shutil
import sys

import numpy as np
import pytest
import xxhash

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*_scalar.json")))


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def file_xxh64(path):
    h = xxhash.xxh64()
    with open(path, "rb") as f:
        while True:
            b = f.read(1 << 24)
            if not b:
                break
            h.update(b)
    return h.hexdigest()


def row_hashes(lg):
    return [xxhash.xxh64(np.ascontiguousarray(r).tobytes()).hexdigest() for r in lg]


def first_mismatch(got, want):
    for i, (a, b) in enumerate(zip(got, want)):
        if a != b:
            return i
    return None if len(got) == len(want) else min(len(got), len(want))


@pytest.mark.parametrize("fixture", FIXTURES, ids=[os.path.basename(f).split("_")[0] for f in FIXTURES])
def test_golden_config(gpu, tmp_path, fixture):
    g = json.load(open(fixture))
    w = gpu.WORKLOADS[g["config"]]
    P, G = g["n_prompt"], g["n_gen"]
    size = os.path.getsize(fixture)
    need = 8e9 if w.wtype == "q8_0" and w.dim >= 4096 else 4.2e9
    d = "/dev/shm" if shutil.disk_usage("/dev/shm").free > need * 1.5 else str(tmp_path)
    path = os.path.join(d, f"qmh_golden_{g['config']}_{os.getpid()}.qlm")
    say(f"case {g['config']}: generate ({w.wtype}, fixture {size} B)")
    try:
        gpu.gen_model(path, w.config(), w.wtype, seed=g["seed"])
        assert file_xxh64(path) == g["qlm_xxh64"], "generator output differs from the fixture's model"
        prompt = gpu.prompt_ids(P, w.vocab_size)
        assert [int(t) for t in prompt] == g["prompt"]
        with gpu.Model.load(path, max_seq=g["max_seq"]) as m:
            say(f"case {g['config']}: prefill {P} with logits")
            lg = m.prefill(prompt, 0, want_logits=True)
            i = first_mismatch(row_hashes(lg), g["logits_xxh64"][:P])
            assert i is None, f"prompt logits differ first at position {i}"
            say(f"case {g['config']}: device greedy {G}")
            ids = [int(t) for t in m.greedy(g["tokens"][0], P, G)]
            i = first_mismatch(ids, g["tokens"][1:])
            assert i is None, f"greedy ids differ first at step {i}: {ids[i:i + 4]} vs {g['tokens'][1 + i:i + 5]}"
            say(f"case {g['config']}: decode logits at {G} positions")
            got = [row_hashes(m.forward(g["tokens"][k], P + k)[None])[0] for k in range(G)]
            i = first_mismatch(got, g["logits_xxh64"][P:])
            assert i is None, f"decode logits differ first at position {P + i}"
            last = m.forward(g["tokens"][G - 1], P + G - 1)
            for tid, val in g["last_top5"]:
                assert np.float32(last[tid]) == np.float32(val)
    finally:
        if os.path.exists(path):
            os.remove(path)
