"""Batched decode (qmh_batch_*): B independent sequences per step, each with its own KV cache.

Per sequence, the logits of every step must be bitwise those of the oracle's single-sequence forward
at the same token and position, and of the device's own single-sequence forward; the device greedy
loop must give each sequence the oracle's greedy continuation. Sequences sit at different positions
in the same step: sequence i holds its first position for i steps before advancing (recomputing a
position it already holds writes the same K/V values) and, once done, repeats its last one.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def oracle_logits(oracle, path, toks):
    """logits [len(toks), V] of single-sequence forwards at positions 0.. (the reference's loop)."""
    lg, _ = oracle.run_model(path, toks, 0)
    return lg


@pytest.mark.parametrize("shape,wt,B", [("small", "q8_0", 3), ("small", "q4_0", 5), ("gqa", "q4_0", 4),
                                        ("gqa48", "q4_0", 2), ("mha", "q8_0", 1), ("odd", "q4_0", 3)])
def test_batch_forward_matches_single_sequences(gpu, oracle, small_models, shape, wt, B):
    say("batch", shape, wt, B)
    path = small_models[(shape, wt)]
    rs = np.random.default_rng(7 + B)
    with gpu.Model.load(path) as m:
        V, S = m.vocab, m.cfg.max_seq
        lens = [min(S, 12 + 5 * i) for i in range(B)]
        toks = [rs.integers(0, V, L).astype(np.int32) for L in lens]
        want = [oracle_logits(oracle, path, t) for t in toks]
        steps = max(L + i for i, L in enumerate(lens)) + 2
        with gpu.Batch(m, B) as bt:
            for k in range(steps):
                pos = [min(max(k - i, 0), lens[i] - 1) for i in range(B)]
                tk = [int(toks[i][pos[i]]) for i in range(B)]
                lg = bt.forward(tk, pos)
                for i in range(B):
                    assert np.array_equal(bits(lg[i]), bits(want[i][pos[i]])), \
                        f"step {k} sequence {i} position {pos[i]}"
        # the device's own single-sequence path agrees too (first sequence)
        for p_, t in enumerate(toks[0][:6]):
            assert np.array_equal(bits(m.forward(int(t), p_)), bits(want[0][p_]))


@pytest.mark.parametrize("shape,wt,B", [("small", "q4_0", 4), ("gqa", "q8_0", 3)])
def test_batch_greedy_matches_oracle(gpu, oracle, small_models, shape, wt, B):
    say("batch greedy", shape, wt, B)
    path = small_models[(shape, wt)]
    rs = np.random.default_rng(11)
    P0, n = 9, 20
    with gpu.Model.load(path) as m:
        V = m.vocab
        prompts = [rs.integers(0, V, P0).astype(np.int32) for _ in range(B)]
        want = [oracle.run_model(path, p, n, keep_logits=False)[1] for p in prompts]
        with gpu.Batch(m, B) as bt:
            lg = None
            for k in range(P0):
                lg = bt.forward([int(p[k]) for p in prompts], [k] * B)
            first = [int(np.argmax(lg[i])) for i in range(B)]
            assert first == [int(w[0]) for w in want]
            ids, ms = bt.greedy(first, [P0] * B, n)
            assert ms > 0
            for i in range(B):
                assert list(ids[:, i]) == list(want[i][1:n + 1]), f"sequence {i}"


def test_batch_errors(gpu, small_models):
    with gpu.Model.load(small_models[("small", "q4_0")]) as m:
        with pytest.raises(gpu.QmhError):
            gpu.Batch(m, 0)
        with pytest.raises(gpu.QmhError):
            gpu.Batch(m, m.cfg.max_seq + 1)
        with gpu.Batch(m, 2) as bt:
            with pytest.raises(gpu.QmhError):
                bt.forward([0, m.vocab], [0, 0])
            with pytest.raises(gpu.QmhError):
                bt.forward([0, 1], [0, m.cfg.max_seq])
            with pytest.raises(gpu.QmhError):
                bt.greedy([0, 1], [m.cfg.max_seq - 2, 0], 3)
    with gpu.Model.load(small_models[("small", "f32")]) as m:
        with pytest.raises(gpu.QmhError):
            gpu.Batch(m, 2)  # f32 weights have no batched matmul path
