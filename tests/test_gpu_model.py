"""Whole-model parity of the device forward with the CPU oracle and with the compiled
reference (scalar ISA), through the C ABI: per-position logits bit-exact, greedy ids identical,
prefill == sequential forwards, bad inputs rejected, bitwise run-to-run determinism."""
import os
import sys

import numpy as np
import pytest

from _bind import ref_run

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("shape", ["small", "odd", "mha", "gqa", "gqa48"])
@pytest.mark.parametrize("wt", ["f32", "q8_0", "q4_0"])
def test_forward_matches_oracle(gpu, oracle, small_models, shape, wt):
    path = small_models[(shape, wt)]
    say(f"case {shape}/{wt}: load {path}")
    # gqa: 270 prompt tokens, so the attention context passes one 256-position chunk;
    # gqa48: 100, so the scores cover two 64-position K tiles
    n_prompt = {"gqa": 270, "gqa48": 100}.get(shape, 6)
    prompt = gpu.prompt_ids(n_prompt, 458 if shape in ("small", "odd") else 300, seed=5)
    want, want_ids = oracle.run_model(path, prompt, n_gen=20)
    with gpu.Model.load(path) as m:
        got = []
        for i, t in enumerate(prompt):
            got.append(m.forward(int(t), i).copy())
        tok = int(want_ids[0])
        ids = [int(np.argmax(got[-1]))]
        for g in range(20):
            lg = m.forward(ids[-1], len(prompt) + g).copy()
            got.append(lg)
            ids.append(int(np.argmax(lg)))
        got = np.stack(got)
        assert np.array_equal(bits(got), bits(want)), np.abs(got - want).max()
        assert ids == list(want_ids)
        assert tok == ids[0]


@pytest.mark.parametrize("wt", ["f32", "q8_0", "q4_0"])
def test_greedy_prefill_and_errors(gpu, oracle, small_models, wt):
    path = small_models[("small", wt)]
    prompt = gpu.prompt_ids(9, 458, seed=9)
    want, want_ids = oracle.run_model(path, prompt, n_gen=40)
    with gpu.Model.load(path) as m:
        say(f"case small/{wt}: prefill")
        lg = m.prefill(prompt, 0, want_logits=True)
        assert np.array_equal(bits(lg), bits(want[: len(prompt)]))
        say(f"case small/{wt}: device greedy")
        ids = m.greedy(int(want_ids[0]), len(prompt), 40)
        assert list(ids) == list(want_ids[1:])
        # reference semantics: NULL on bad token / pos (src/model.c:160, tests/test_model.c:121-122)
        assert m.forward(0, m.cfg.max_seq) is None
        assert m.forward(m.cfg.vocab_size, 0) is None
        assert m.forward(-1, 0) is None
        with pytest.raises(gpu.QmhError):
            m.greedy(0, m.cfg.max_seq - 3, 10)


def test_rerun_is_bitwise_deterministic(gpu, small_models):
    path = small_models[("odd", "q4_0")]
    prompt = gpu.prompt_ids(30, 458, seed=2)
    outs = []
    for r in range(2):
        with gpu.Model.load(path) as m:
            outs.append(m.prefill(prompt, 0, want_logits=True))
    assert np.array_equal(bits(outs[0]), bits(outs[1]))


def test_stage_timing_after_greedy_to_end_of_context(gpu, oracle, small_models):
    """A greedy run that fills the context leaves the device position one past the end; the
    stage timer must set its own position (regression: it used the stale one)."""
    path = small_models[("small", "q8_0")]
    with gpu.Model.load(path, max_seq=24) as m:
        m.prefill(gpu.prompt_ids(8, 458, seed=4), 0)
        m.greedy(3, 8, 16)  # positions 8..23: the device position ends at 24 == max_seq
        for st in m.STAGES:
            if st == "attn":  # the one-launch attention takes head_dim 48/64/128 only (this model: 16)
                with pytest.raises(gpu.QmhError):
                    m.time_stage(st, 4, pos=23)
                continue
            ms, nbytes = m.time_stage(st, 4, pos=23)
            assert ms > 0
        with pytest.raises(gpu.QmhError):
            m.time_stage("qkv", 1, pos=24)
        lg = m.forward(5, 0)
        want, _ = oracle.run_model(path, [5], n_gen=0, max_seq=24)
        assert np.array_equal(bits(lg), bits(want[0]))


def test_max_seq_cap(gpu, small_models):
    with gpu.Model.load(small_models[("small", "q8_0")], max_seq=16) as m:
        assert m.cfg.max_seq == 16
        assert m.forward(1, 15) is not None and m.forward(1, 16) is None


@pytest.mark.parametrize("name", ["c1", "c2"])
def test_baseline_config_vs_reference(gpu, tmp_path, name):
    """BASELINE configs c1/c2 (stories15M shape): every position's logits bit-exact with the
    compiled reference (scalar ISA) and the greedy ids identical over the whole decode."""
    w = gpu.WORKLOADS[name]
    path = str(tmp_path / f"{name}.qlm")
    say(f"case {name}: generate")
    gpu.gen_model(path, w.config(), w.wtype, seed=w.seed)
    prompt = gpu.prompt_ids(w.n_prompt, w.vocab_size)
    say(f"case {name}: reference, {w.n_prompt} prompt + {w.n_gen} greedy")
    res, rl = ref_run(path, prompt, w.n_gen, isa="scalar", threads=4)
    rl = rl.reshape(w.n_prompt + w.n_gen, w.vocab_size)
    with gpu.Model.load(path) as m:
        say(f"case {name}: device prefill")
        lg = m.prefill(prompt, 0, want_logits=True)
        assert np.array_equal(bits(lg), bits(rl[: w.n_prompt]))
        say(f"case {name}: device greedy")
        ids = m.greedy(res["tokens"][0], w.n_prompt, w.n_gen)
        assert list(ids) == res["tokens"][1:]
        got = []
        toks = res["tokens"]
        for g in range(w.n_gen):
            got.append(m.forward(toks[g], w.n_prompt + g).copy())
        assert np.array_equal(bits(np.stack(got)), bits(rl[w.n_prompt:]))


@pytest.mark.parametrize("wt", ["q8_0", "q4_0"])
def test_batched_prefill_matches_sequential(gpu, tmp_path, wt):
    """The batched prefill (int8 MFMA matmuls, batched attention) against the one-token-at-a-time
    path on the same model: every position's logits, the KV cache (through the decode step that
    follows), across a second pass (600 tokens > 512 per pass), an odd-sized continuation at
    pos0 > 0, and GQA with head_dim 32."""
    import os

    path = str(tmp_path / f"pf_{wt}.qlm")
    cfg = gpu.QmhConfig(dim=128, hidden_dim=344, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=300, max_seq=700,
                        rope_theta=10000.0, norm_eps=1e-5)
    gpu.gen_model(path, cfg, wt, seed=31, threads=4)
    prompt, more = gpu.prompt_ids(600, 300, seed=8), gpu.prompt_ids(30, 300, seed=12)
    runs = []
    for seq in (False, True):
        if seq:
            os.environ["QMH_PREFILL_SEQ"] = "1"
        try:
            with gpu.Model.load(path) as m:
                say(f"case {wt}: prefill {'sequential' if seq else 'batched'}")
                a = m.prefill(prompt, 0, want_logits=True)
                b = m.prefill(more, 600, want_logits=True)
                c = m.forward(7, 630).copy()
                runs.append((a, b, c))
        finally:
            os.environ.pop("QMH_PREFILL_SEQ", None)
    for got, want in zip(runs[0], runs[1]):
        assert np.array_equal(bits(got), bits(want)), np.abs(got - want).max()


@pytest.mark.parametrize("hd,n_heads,n_kv,wt", [(128, 2, 1, "q4_0"), (64, 4, 4, "q8_0"), (64, 4, 2, "q4_0")])
def test_batched_prefill_head_dims(gpu, tmp_path, hd, n_heads, n_kv, wt):
    """head_dim 128 and 64 (the register-blocked prefill attention: scores of 64 tokens x 64
    positions per workgroup, P.V writing Wo's quantized input image), MHA and GQA, max_seq 301 (not
    a multiple of 4 or 64: the last tile's positions past max_seq), prompts of 150, 77, 20 and 3
    tokens (ragged tiles, pos0 > 0; Wo as the tiled matmul, the skinny matmul and the multi-token
    matvec, each reading that image), against sequential forwards."""
    import os

    path = str(tmp_path / f"pf_hd{hd}_{n_kv}_{wt}.qlm")
    cfg = gpu.QmhConfig(dim=hd * n_heads, hidden_dim=192, n_layers=2, n_heads=n_heads, n_kv_heads=n_kv,
                        vocab_size=300, max_seq=301, rope_theta=10000.0, norm_eps=1e-5)
    gpu.gen_model(path, cfg, wt, seed=35, threads=4)
    chunks = [gpu.prompt_ids(n, 300, seed=61 + n) for n in (150, 77, 20, 3)]
    runs = []
    for seq in (False, True):
        if seq:
            os.environ["QMH_PREFILL_SEQ"] = "1"
        try:
            with gpu.Model.load(path) as m:
                say(f"case hd{hd} kv{n_kv} {wt}: prefill {'sequential' if seq else 'batched'}")
                pos, outs = 0, []
                for ch in chunks:
                    outs.append(m.prefill(ch, pos, want_logits=True))
                    pos += len(ch)
                outs.append(m.forward(9, pos).copy())
                runs.append(outs)
        finally:
            os.environ.pop("QMH_PREFILL_SEQ", None)
    for got, want in zip(runs[0], runs[1]):
        assert np.array_equal(bits(got), bits(want)), np.abs(got - want).max()


@pytest.mark.parametrize("wt", ["q8_0", "q4_0"])
def test_batched_prefill_rows_not_multiple_of_4(gpu, tmp_path, wt):
    """W2's input rows of 202 values (n % 4 == 2): the activation quantizer's per-value path
    instead of its 16-byte loads (the skinny matmul at 20 and 33 tokens: two and four token tiles),
    beside the multi-token matvec's own quantization (3 tokens) and W1|W3's image epilogue (70: the
    tiled matmul), against sequential forwards.
    (The batched prefill needs head_dim % 4 == 0, so dim % 4 == 0.)"""
    import os

    path = str(tmp_path / f"pf_odd_{wt}.qlm")
    cfg = gpu.QmhConfig(dim=96, hidden_dim=202, n_layers=2, n_heads=8, n_kv_heads=4, vocab_size=300, max_seq=128,
                        rope_theta=10000.0, norm_eps=1e-5)
    gpu.gen_model(path, cfg, wt, seed=33, threads=4)
    chunks = [gpu.prompt_ids(n, 300, seed=20 + n) for n in (70, 33, 20, 3)]
    runs = []
    for seq in (False, True):
        if seq:
            os.environ["QMH_PREFILL_SEQ"] = "1"
        try:
            with gpu.Model.load(path) as m:
                say(f"case odd {wt}: prefill {'sequential' if seq else 'batched'}")
                pos, outs = 0, []
                for ch in chunks:
                    outs.append(m.prefill(ch, pos, want_logits=True))
                    pos += len(ch)
                outs.append(m.forward(5, pos).copy())
                runs.append(outs)
        finally:
            os.environ.pop("QMH_PREFILL_SEQ", None)
    for got, want in zip(runs[0], runs[1]):
        assert np.array_equal(bits(got), bits(want)), np.abs(got - want).max()
    # batched decode of 6 sequences (the skinny matmul after the quantizer at 1024 threads per row)
    seqs = [gpu.prompt_ids(4, 300, seed=50 + i) for i in range(6)]
    with gpu.Model.load(path) as m:
        say(f"case odd {wt}: batched decode")
        single = []
        for s in seqs:
            single.append(np.stack([m.forward(int(t), k).copy() for k, t in enumerate(s)]))
        with gpu.Batch(m, 6) as bt:
            for k in range(4):
                lg = bt.forward([int(s[k]) for s in seqs], [k] * 6)
                for i in range(6):
                    assert np.array_equal(bits(lg[i]), bits(single[i][k])), f"step {k} sequence {i}"


@pytest.mark.parametrize("name,dims,wt,spans", [
    # one query head per kv head, head_dim 128: decode attention past one 640-position chunk
    # (positions 638-642 cross into the second chunk, 1279-1281 into the third), and across the
    # one-launch attention's instances (640 and 1024 positions)
    ("mha128", dict(dim=256, hidden_dim=320, n_layers=1, n_heads=2, n_kv_heads=2, vocab_size=300, max_seq=1300),
     "q4_0", [(636, 646), (1019, 1029), (1277, 1286)]),
    # 4 query heads on one kv head of 64 dims (c4's grouping): both one-launch instances and the
    # two-launch path past 1024 positions
    ("gqa64", dict(dim=256, hidden_dim=320, n_layers=1, n_heads=4, n_kv_heads=1, vocab_size=300, max_seq=1100),
     "q8_0", [(636, 646), (1019, 1029)]),
    # 32 query heads on one kv head of 64 dims: the 8-column one-launch kernel on a full grid (32 heads
    # x 8 column groups = 256 workgroups), every head reading the one kv head's K and V
    ("gqa32x64", dict(dim=2048, hidden_dim=256, n_layers=1, n_heads=32, n_kv_heads=1, vocab_size=300,
                      max_seq=1040), "q4_0", [(636, 646), (1019, 1029)]),
    # grouped heads (2 and 8 query heads per kv head), head_dim 32 and 16: the per-query-head P.V
    # kernel reading its kv head's V, whole-context and streamed past 640 positions
    ("gqa32", dict(dim=128, hidden_dim=256, n_layers=1, n_heads=4, n_kv_heads=2, vocab_size=300, max_seq=1300),
     "q8_0", [(636, 646), (1277, 1286)]),
    ("gqa8x16", dict(dim=128, hidden_dim=256, n_layers=1, n_heads=8, n_kv_heads=1, vocab_size=300, max_seq=900),
     "q4_0", [(636, 646), (890, 900)]),
    # head_dim 10 (not a multiple of 4): the scalar-column decode attention, and prompts that run as
    # sequential forwards (the batched prompt path takes head_dim % 4 == 0 only)
    ("mha10", dict(dim=60, hidden_dim=128, n_layers=1, n_heads=6, n_kv_heads=6, vocab_size=300, max_seq=700),
     "q8_0", [(636, 646), (690, 700)]),
    # grouped heads with head_dim 6 and 10 (not a multiple of 4): the scalar-column kernel with the
    # group's scores in LDS (k_attn_pv<640, false>), across 256 and its 640-position chunk boundary
    ("gqa6", dict(dim=24, hidden_dim=64, n_layers=1, n_heads=4, n_kv_heads=2, vocab_size=300, max_seq=700),
     "q8_0", [(250, 262), (636, 646)]),
    ("gqa10", dict(dim=40, hidden_dim=96, n_layers=1, n_heads=4, n_kv_heads=2, vocab_size=300, max_seq=700),
     "q4_0", [(250, 262), (636, 646)]),
    # 20 query heads on one kv head of 10 dims: k_attn_pv<256, false> in two sub-groups (16 + 4 heads
    # per workgroup) around its 256-position chunk boundary
    ("gqa20x10", dict(dim=200, hidden_dim=128, n_layers=1, n_heads=20, n_kv_heads=1, vocab_size=300, max_seq=300),
     "q8_0", [(250, 262)]),
    # 12 query heads on one kv head of 10 dims: the 256-position chunks (k_attn_pv<256, false>)
    ("gqa10x12", dict(dim=120, hidden_dim=128, n_layers=1, n_heads=12, n_kv_heads=1, vocab_size=300, max_seq=530),
     "q8_0", [(250, 262), (508, 516)]),
    # one query head per kv head past 8192 positions: the chunked V sum (attn_pv_chunks<640, true>)
    ("mha16long", dict(dim=32, hidden_dim=64, n_layers=1, n_heads=2, n_kv_heads=2, vocab_size=300, max_seq=8200),
     "q4_0", [(8188, 8197)]),
])
def test_long_context_decode_matches_oracle(gpu, oracle, tmp_path, name, dims, wt, spans):
    """Decode forwards at positions on either side of the attention kernels' chunk boundaries
    (src/model.c:132-156 attends over every pos < max_seq), the positions between them filled by
    prefill: logits bitwise the oracle's at every position."""
    path = str(tmp_path / f"{name}.qlm")
    gpu.gen_model(path, gpu.QmhConfig(**dims, rope_theta=10000.0, norm_eps=1e-5), wt, seed=41, threads=4)
    n = spans[-1][1]
    toks = gpu.prompt_ids(n, dims["vocab_size"], seed=17)
    say(f"case {name}: oracle over {n} positions")
    want, _ = oracle.run_model(path, toks, n_gen=0)
    with gpu.Model.load(path) as m:
        p = 0
        for lo, hi in spans:
            say(f"case {name}: prefill {p}..{lo - 1}, forwards {lo}..{hi - 1}")
            lg = m.prefill(toks[p:lo], p, want_logits=True)
            assert np.array_equal(bits(lg), bits(want[p:lo])), f"prefill positions {p}..{lo - 1}"
            for i in range(lo, hi):
                got = m.forward(int(toks[i]), i)
                assert np.array_equal(bits(got), bits(want[i])), f"position {i}: max |d| {np.abs(got - want[i]).max()}"
            p = hi


@pytest.mark.parametrize("dim,hidden,heads,kv,layers,wt,P", [
    (512, 14336, 8, 2, 2, "q4_0", 40), (512, 13824, 8, 2, 2, "q8_0", 40), (512, 28672, 8, 2, 1, "q4_0", 100),
    (8192, 512, 64, 8, 1, "q8_0", 40)])
def test_wide_hidden_matches_oracle(gpu, oracle, tmp_path, dim, hidden, heads, kv, layers, wt, P):
    """Feed-forward widths past 12288 (Llama-2-13B's 13824, Mistral-7B's and Llama-3-8B's 14336, the 70B
    shapes' 28672): W2's input arrives as W1|W3's quantized image of 432-896 blocks (a second matvec
    instance past 16 KiB of image); and the 70B width 8192 with 64 query heads on 8 kv heads, whose
    64-row W1|W3 tiles need more than 64 KiB of LDS per workgroup. Prefill logits, decode forwards and
    the device greedy loop bitwise the oracle's; batched forwards (multi-token matvec at 2 sequences,
    skinny matmul at 5) bitwise the oracle's single-sequence logits. A 100-token prompt runs the tiled
    prefill matmul, whose W1|W3 epilogue writes W2's image."""
    cfg = gpu.QmhConfig(dim=dim, hidden_dim=hidden, n_layers=layers, n_heads=heads, n_kv_heads=kv,
                        vocab_size=300, max_seq=P + 40, rope_theta=10000.0, norm_eps=1e-5)
    path = str(tmp_path / f"wide_d{dim}_h{hidden}_{wt}.qlm")
    gpu.gen_model(path, cfg, wt, seed=23, threads=4)
    G = 8
    prompt = gpu.prompt_ids(P, 300, seed=19)
    say(f"case dim {dim} hidden {hidden}/{wt}: oracle {P}+{G}")
    want, want_ids = oracle.run_model(path, prompt, n_gen=G)
    with gpu.Model.load(path) as m:
        lg = m.prefill(prompt, 0, want_logits=True)
        assert np.array_equal(bits(lg), bits(want[:P])), "prefill logits"
        tok = int(want_ids[0])
        for g in range(G):
            got = m.forward(tok, P + g)
            assert np.array_equal(bits(got), bits(want[P + g])), f"position {P + g}"
            tok = int(np.argmax(got))
        m.prefill(prompt, 0)
        ids = m.greedy(int(want_ids[0]), P, G)
        assert list(ids) == list(want_ids[1:])
        rs = np.random.default_rng(hidden)
        for B in (2, 5):
            toks = [rs.integers(0, 300, 6 + i).astype(np.int32) for i in range(B)]
            wl = [oracle.run_model(path, t, 0)[0] for t in toks]
            with gpu.Batch(m, B) as bt:
                for k in range(6 + B - 1):
                    pos = [min(k, 6 + i - 1) for i in range(B)]
                    out = bt.forward([int(toks[i][pos[i]]) for i in range(B)], pos)
                    for i in range(B):
                        assert np.array_equal(bits(out[i]), bits(wl[i][pos[i]])), f"B={B} step {k} sequence {i}"


@pytest.mark.parametrize("name,dim,hidden,layers,heads,kv,vocab,theta", [
    ("llama3_8b", 4096, 14336, 32, 32, 8, 128256, 500000.0), ("llama2_13b", 5120, 13824, 40, 40, 40, 32000, 10000.0)])
def test_full_size_shapes_vs_reference(gpu, tmp_path, name, dim, hidden, layers, heads, kv, vocab, theta):
    """Full-size Llama-3-8B and Llama-2-13B shapes in Q4_0 (every layer and the real vocabulary; random
    weights): the batched prefill's 8 prompt logits and 8 greedy forwards bitwise the compiled reference's
    scalar ISA, and the device greedy loop's ids the reference's."""
    cfg = gpu.QmhConfig(dim, hidden, layers, heads, kv, vocab, 64, theta, 1e-5)
    path = str(tmp_path / f"{name}.qlm")
    say(f"case {name}: generate")
    gpu.gen_model(path, cfg, "q4_0", seed=1, threads=16)
    try:
        P, G = 8, 8
        prompt = gpu.prompt_ids(P, vocab, seed=1234)
        say(f"case {name}: reference, {P} prompt + {G} greedy")
        res, rl = ref_run(path, prompt, G, isa="scalar", threads=16)
        rl = rl.reshape(P + G, vocab)
        toks = res["tokens"]
        with gpu.Model.load(path) as m:
            say(f"case {name}: device prefill and forwards")
            lg = m.prefill(prompt, 0, want_logits=True)
            assert np.array_equal(bits(lg), bits(rl[:P])), "prefill logits"
            for g in range(G):
                got = m.forward(toks[g], P + g)
                assert np.array_equal(bits(got), bits(rl[P + g])), f"position {P + g}"
            say(f"case {name}: device greedy")
            m.prefill(prompt, 0)
            assert list(m.greedy(toks[0], P, G)) == toks[1:]
    finally:
        os.remove(path)
