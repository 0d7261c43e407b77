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
                                        ("gqa48", "q4_0", 2), ("mha", "q8_0", 1), ("odd", "q4_0", 3),
                                        ("small", "q4_0", 40), ("odd", "q8_0", 64),
                                        # past 64 sequences: W1|W3's tiled matmul writes W2's quantized
                                        # input image, and the fused attention runs above 64 sequences
                                        ("gqa", "q4_0", 70), ("gqa", "q8_0", 128)])
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


def attention_reference(oracle, q, kt, v, n, n_kv, hd, scale):
    """One sequence's attention (src/model.c:127-156) in float32 single operations: each score the
    serial chain over head_dim times the scale, the oracle's softmax, each output element the chain
    +0 + p_0 v_0[i] + p_1 v_1[i] + ... in position order."""
    H = q.size // hd
    out = np.zeros(H * hd, np.float32)
    for h in range(H):
        kvh = h // (H // n_kv)
        s = np.zeros(n, np.float32)
        for d in range(hd):
            s = s + q[h * hd + d] * kt[kvh * hd + d, :n]
        p = oracle.softmax(s * np.float32(scale))
        acc = np.zeros(hd, np.float32)
        for t in range(n):
            acc = acc + p[t] * v[t, kvh * hd:(kvh + 1) * hd]
        out[h * hd:(h + 1) * hd] = acc
    return out


@pytest.mark.parametrize("n_heads,n_kv,hd,positions", [
    (4, 4, 64, [0, 127, 128, 129]),
    (2, 2, 128, [639, 641, 1300]),
    (8, 2, 128, [1023, 1024, 1025, 5]),
    (6, 3, 96, [255, 700, 2047]),
    (2, 1, 4, [0, 1, 300]),
])
def test_batch_attention_fused_and_split(gpu, oracle, n_heads, n_kv, hd, positions):
    """The fused attention kernel, the three-launch path it replaces up to 16384 positions and the
    automatic choice (the decode kernels with a sequence dimension for up to 3 MHA sequences of
    head_dim 128/64/48) give the same bits, and all the float32 restatement's; positions straddle
    the V chunk (128), the thread count (1024) and the decode P.V's 640-position chunk."""
    import ctypes
    say("batch attention", n_heads, n_kv, hd, positions)
    L = gpu.load_library()
    B, S = len(positions), max(positions) + 3
    kvd = n_kv * hd
    rs = np.random.default_rng(n_heads * 1000 + hd)
    q = (rs.standard_normal((B, n_heads * hd)) * 0.7).astype(np.float32)
    kt = (rs.standard_normal((B, kvd, S)) * 0.7).astype(np.float32)
    v = rs.standard_normal((B, S, kvd)).astype(np.float32)
    pos = np.array(positions, np.int32)
    scale = 1.0 / np.sqrt(np.float32(hd))
    bufs = [gpu.DeviceBuffer.from_array(a) for a in (q, kt, v, pos)]
    att = gpu.DeviceBuffer(B * n_heads * S * 4)
    outs = []
    try:
        fn = L.qmh_launch_bt_attention
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_longlong, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                              ctypes.c_void_p] + [ctypes.c_int] * 5 + [ctypes.c_float,
                                                                                      ctypes.c_int, ctypes.c_void_p]
        for split in (2, 1, 0):
            o = gpu.DeviceBuffer(B * n_heads * hd * 4)
            rc = fn(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, kvd * S, bufs[3].ptr, int(pos.max()), att.ptr, o.ptr, B,
                    n_heads, n_kv, hd, S, float(scale), split, L.qmh_stream())
            assert rc == 0
            gpu.sync()
            outs.append(o.to_array(np.float32).reshape(B, n_heads * hd))
            o.free()
    finally:
        for b in bufs + [att]:
            b.free()
    assert np.array_equal(bits(outs[0]), bits(outs[1])), "fused and split paths differ"
    assert np.array_equal(bits(outs[0]), bits(outs[2])), "fused path and the automatic choice differ"
    for b in range(B):
        want = attention_reference(oracle, q[b], kt[b], v[b], int(pos[b]) + 1, n_kv, hd, scale)
        assert np.array_equal(bits(outs[0][b]), bits(want)), f"sequence {b} (pos {pos[b]})"


@pytest.mark.parametrize("wt", ["q4_0", "q8_0"])
def test_batch_forward_wide(gpu, oracle, tmp_path, wt):
    """The 7B layer shapes (4096 wide, hidden 11008, one layer, vocabulary 8192): the multi-token matvec
    gives each workgroup 2-3 tiles of QKV, Wo, W2 and the output, and runs W1|W3 (344 tiles) in LDS
    rounds at 3 tokens (the skinny matmul takes 4), for both weight types (their slot widths differ); attention through the
    decode kernels with a sequence dimension up to 3 sequences, the fused kernel at 4. Per-sequence
    logits at 1-4 sequences, mixed positions, bitwise the oracle's single-sequence forwards."""
    say("batch wide", wt)
    cfg = gpu.QmhConfig(dim=4096, hidden_dim=11008, n_layers=1, n_heads=32, n_kv_heads=32, vocab_size=8192,
                        max_seq=16, rope_theta=10000.0, norm_eps=1e-5)
    path = str(tmp_path / f"wide_{wt}.qlm")
    gpu.gen_model(path, cfg, wt, seed=5, threads=8)
    rs = np.random.default_rng(3)
    with gpu.Model.load(path) as m:
        V = m.vocab
        for B in (1, 2, 3, 4):
            lens = [2 + i for i in range(B)]
            toks = [rs.integers(0, V, L).astype(np.int32) for L in lens]
            want = [oracle_logits(oracle, path, t) for t in toks]
            with gpu.Batch(m, B) as bt:
                for k in range(max(lens)):
                    pos = [min(k, lens[i] - 1) for i in range(B)]
                    lg = bt.forward([int(toks[i][pos[i]]) for i in range(B)], pos)
                    for i in range(B):
                        assert np.array_equal(bits(lg[i]), bits(want[i][pos[i]])), \
                            f"B={B} step {k} sequence {i} position {pos[i]}"
