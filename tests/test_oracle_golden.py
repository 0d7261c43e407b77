"""The CPU oracle (C restatement) and the model generator against the committed whole-model
fixtures of the compiled reference (tests/golden/*_scalar.json): same .qlm bytes, the same
logits at every position (xxh64 of the float32 bytes) and the same greedy ids. Runs the small
configs c1 and c2; the GPU tests replay every fixture."""
import json
import os

import numpy as np
import pytest
import xxhash

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.parametrize("name", ["c1", "c2"])
def test_oracle_replays_reference_fixture(oracle, qmh, tmp_path, name):
    g = json.load(open(os.path.join(HERE, "golden", f"{name}_scalar.json")))
    w = qmh.WORKLOADS[name]
    assert g["reference"]["isa"] == "scalar" and g["dims"][0] == w.dim and g["wtype"] == w.wtype
    path = str(tmp_path / f"{name}.qlm")
    qmh.gen_model(path, w.config(), w.wtype, seed=g["seed"], threads=4)
    assert xxhash.xxh64(open(path, "rb").read()).hexdigest() == g["qlm_xxh64"]
    prompt = qmh.prompt_ids(g["n_prompt"], w.vocab_size)
    assert [int(t) for t in prompt] == g["prompt"]
    lg, ids = oracle.run_model(path, prompt, g["n_gen"], max_seq=g["max_seq"])
    assert [int(t) for t in ids] == g["tokens"]
    got = [xxhash.xxh64(np.ascontiguousarray(r).tobytes()).hexdigest() for r in lg]
    assert got == g["logits_xxh64"]


def test_fixtures_are_well_formed():
    """Every fixture: G+1 ids, P+G logits hashes, top-5 ordered and agreeing with the last id."""
    names = sorted(f for f in os.listdir(os.path.join(HERE, "golden")) if f.endswith("_scalar.json"))
    assert {"c1_scalar.json", "c2_scalar.json"} <= set(names)
    for f in names:
        g = json.load(open(os.path.join(HERE, "golden", f)))
        P, G = g["n_prompt"], g["n_gen"]
        assert len(g["prompt"]) == P and len(g["tokens"]) == G + 1 and len(g["logits_xxh64"]) == P + G
        vals = [v for _, v in g["last_top5"]]
        assert vals == sorted(vals, reverse=True) and g["last_top5"][0][0] == g["tokens"][-1]
