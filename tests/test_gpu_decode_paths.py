"""Decode-step variants, bit for bit.

* The one-launch attention (k_attn_fused: scores, softmax and V sum, the scores exchanged between a
  head's workgroups as epoch-tagged words) against the CPU oracle, at decode positions on both sides
  of its instances' limits (640 positions; 1024 for head_dim 64 and 128, and for 48 at 8 columns per
  workgroup), for the head shapes it takes (head_dim 128, 64 and 48; one and four query heads per kv
  head), with 8 output columns per workgroup (the width the library picks for grids that fill at most
  the device) and 16 (QMH_AF_CW=16, the width of larger models).
* The same steps replayed from hipGraphs, enqueued kernel by kernel (QMH_NO_GRAPH), with the
  two-launch attention (QMH_NO_FUSED_ATTN), with the 640-position instance alone
  (QMH_FUSED_ATTN_640) and with 16 columns per workgroup: identical logits and greedy ids.
* A rerun of the same decode steps gives the same bits (reference: tests/test_model.c:84-94 reruns a
  model, tests/test_threads.c:56-94 compares thread counts bitwise).
* The bounded wait of the one-launch attention, run to its end from the host (QMH_AF_FORCE_STALL):
  the call fails with a message instead of returning logits.
* Every RMSNorm of the matvecs on its serial path (QMH_EXACT_NORM: the sum of squares a failed
  certificate recomputes in the reference's order) against the oracle.
"""
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# dim / n_heads = 128, 64 (4 query heads on one kv head) and 48; contexts past 640 for the first two,
# past 1024 for af64x
AF_SHAPES = {
    "af128": dict(dim=256, hidden_dim=384, n_layers=2, n_heads=2, n_kv_heads=2, vocab_size=300, max_seq=700),
    "af64g": dict(dim=256, hidden_dim=384, n_layers=2, n_heads=4, n_kv_heads=1, vocab_size=300, max_seq=664),
    "af48": dict(dim=96, hidden_dim=160, n_layers=2, n_heads=2, n_kv_heads=1, vocab_size=300, max_seq=100),
    "af64x": dict(dim=256, hidden_dim=384, n_layers=2, n_heads=4, n_kv_heads=1, vocab_size=300, max_seq=1040),
    "af48x": dict(dim=96, hidden_dim=160, n_layers=2, n_heads=2, n_kv_heads=1, vocab_size=300, max_seq=700),
}
# prompt length and decode steps: the steps cross position 640 (and 1024) where the context allows it
RUN = {"af128": (630, 20), "af64g": (632, 20), "af48": (60, 30), "af64x": (1014, 20), "af48x": (630, 20)}


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def af_models(qmh, tmp_path_factory):
    d = tmp_path_factory.mktemp("af_models")
    out = {}
    for shape, dims in AF_SHAPES.items():
        for wt in ("q8_0", "q4_0"):
            p = str(d / f"{shape}_{wt}.qlm")
            cfg = qmh.QmhConfig(**dims, rope_theta=10000.0, norm_eps=1e-5)
            qmh.gen_model(p, cfg, wt, seed=31, threads=4)
            out[(shape, wt)] = p
    return out


class env:
    """Environment variables set while a model is created (the library reads them at load)."""

    def __init__(self, **kv):
        self.kv = kv

    def __enter__(self):
        self.old = {k: os.environ.get(k) for k in self.kv}
        os.environ.update(self.kv)

    def __exit__(self, *exc):
        for k, v in self.old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def decode(gpu, path, prompt, n_gen, **kv):
    """Prefill the prompt, then n_gen forwards (logits of each) from the oracle's first token, then the
    device greedy loop over the same positions: (logits [n_gen, V], greedy ids)."""
    with env(**kv):
        m = gpu.Model.load(path)
    with m:
        m.prefill(prompt, 0)
        first = int(np.argmax(m.forward(int(prompt[-1]), len(prompt) - 1)))
        lg, tok = [], first
        for g in range(n_gen):
            row = m.forward(tok, len(prompt) + g).copy()
            lg.append(row)
            tok = int(np.argmax(row))
        ids = m.greedy(first, len(prompt), n_gen)
    return first, np.stack(lg), np.asarray(ids)


@pytest.mark.parametrize("cw", ["8", "16"])
@pytest.mark.parametrize("shape", list(AF_SHAPES))
@pytest.mark.parametrize("wt", ["q8_0", "q4_0"])
def test_fused_attention_matches_oracle(gpu, oracle, af_models, shape, wt, cw):
    path = af_models[(shape, wt)]
    P, G = RUN[shape]
    prompt = gpu.prompt_ids(P, 300, seed=7)
    say(f"case {shape}/{wt}/cw{cw}: oracle {P}+{G}")
    want, want_ids = oracle.run_model(path, prompt, n_gen=G)
    say(f"case {shape}/{wt}/cw{cw}: device decode positions {P}..{P + G - 1}")
    first, lg, ids = decode(gpu, path, prompt, G, QMH_AF_CW=cw)
    assert first == int(want_ids[0])
    assert np.array_equal(bits(lg), bits(want[P:])), np.abs(lg - want[P:]).max()
    assert list(ids) == list(want_ids[1:])


def test_fused_attention_from_position_zero(gpu, oracle, af_models):
    """Sequential forwards from position 0 (the first positions leave most of a head's workgroups
    without a slice of scores)."""
    path = af_models[("af128", "q4_0")]
    prompt = gpu.prompt_ids(24, 300, seed=8)
    want, want_ids = oracle.run_model(path, prompt, n_gen=8)
    with gpu.Model.load(path) as m:
        got = [m.forward(int(t), i).copy() for i, t in enumerate(prompt)]
        tok = int(want_ids[0])
        for g in range(8):
            got.append(m.forward(tok, len(prompt) + g).copy())
            tok = int(np.argmax(got[-1]))
    got = np.stack(got)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("shape", ["af128", "af64g", "af64x", "af48x"])
def test_decode_variants_agree(gpu, af_models, shape):
    path = af_models[(shape, "q4_0")]
    P, G = RUN[shape]
    prompt = gpu.prompt_ids(P, 300, seed=9)
    runs = {}
    for name, kv in [("graph+fused", {}), ("no graph", {"QMH_NO_GRAPH": "1"}),
                     ("two-launch attention", {"QMH_NO_FUSED_ATTN": "1"}),
                     ("640-position instance alone", {"QMH_FUSED_ATTN_640": "1"}),
                     ("16 columns per workgroup", {"QMH_AF_CW": "16"}),
                     ("no graph, two-launch", {"QMH_NO_GRAPH": "1", "QMH_NO_FUSED_ATTN": "1"})]:
        say(f"case {shape}: {name}")
        runs[name] = decode(gpu, path, prompt, G, **kv)
    base = runs["graph+fused"]
    for name, r in runs.items():
        assert r[0] == base[0], name
        assert np.array_equal(bits(r[1]), bits(base[1])), name
        assert list(r[2]) == list(base[2]), name


def test_decode_rerun_is_bitwise_deterministic(gpu, af_models):
    path = af_models[("af128", "q8_0")]
    P, G = RUN["af128"]
    prompt = gpu.prompt_ids(P, 300, seed=10)
    a = decode(gpu, path, prompt, G)
    b = decode(gpu, path, prompt, G)
    assert a[0] == b[0]
    assert np.array_equal(bits(a[1]), bits(b[1]))
    assert list(a[2]) == list(b[2])
    # the same model object, the same steps twice
    with gpu.Model.load(path) as m:
        m.prefill(prompt, 0)
        r1 = m.greedy(int(prompt[-1]), P, G)
        r2 = m.greedy(int(prompt[-1]), P, G)
    assert list(r1) == list(r2)


def test_fused_attention_wait_runs_out(gpu, af_models):
    """QMH_AF_FORCE_STALL makes every workgroup wait for an epoch nobody writes: the wait ends after
    its bound, the kernels finish, and the library reports the failure (forward returns None), for
    both instances. A position past the one-launch kernel's limit takes the two-launch attention,
    which does not wait."""
    path = af_models[("af64x", "q4_0")]
    with env(QMH_AF_FORCE_STALL="1"):
        m = gpu.Model.load(path)
    with m:
        assert m.forward(5, 1030) is not None
        assert m.forward(5, 3) is None
        assert "ran out" in gpu.last_error()
        assert m.forward(5, 700) is None
        assert "ran out" in gpu.last_error()
        # the status word was cleared with the report: the next long-context step succeeds
        assert m.forward(5, 1031) is not None


def test_fused_attention_stage_timer(gpu, oracle, af_models):
    """The stage timer runs the one-launch attention back to back over the layers (no step between
    the launches); the steps after it still match the oracle."""
    path = af_models[("af64g", "q8_0")]
    prompt = gpu.prompt_ids(40, 300, seed=12)
    want, want_ids = oracle.run_model(path, prompt, n_gen=4)
    with gpu.Model.load(path) as m:
        m.prefill(prompt, 0)
        for pos in (0, 39, 600, 639, 640, 663):
            ms, nbytes = m.time_stage("attn", 9, pos=pos)
            assert ms > 0 and nbytes == 0
        m.prefill(prompt, 0)  # the timer wrote the caches at its positions
        ids = m.greedy(int(want_ids[0]), len(prompt), 4)
    assert list(ids) == list(want_ids[1:])
    # past the one-launch kernel's instances the stage timer refuses the one-launch stage
    with gpu.Model.load(af_models[("af64x", "q8_0")]) as m:
        with pytest.raises(gpu.QmhError, match="no one-launch attention"):
            m.time_stage("attn", 3, pos=1030)
        ms, _ = m.time_stage("attn", 3, pos=1000)
        assert ms > 0


@pytest.mark.parametrize("wt", ["q8_0", "q4_0"])
def test_exact_norm_path_matches_oracle(gpu, oracle, af_models, wt):
    path = af_models[("af64g", wt)]
    P, G = 24, 6
    prompt = gpu.prompt_ids(P, 300, seed=14)
    want, want_ids = oracle.run_model(path, prompt, n_gen=G)
    say(f"case exact norm {wt}")
    first, lg, ids = decode(gpu, path, prompt, G, QMH_EXACT_NORM="1")
    assert first == int(want_ids[0])
    assert np.array_equal(bits(lg), bits(want[P:]))
    assert list(ids) == list(want_ids[1:])
