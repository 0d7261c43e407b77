"""Device sampler parity: qmh_sample vs the compiled reference's qm_sample (src/sampler.c:50-106).

Every draw must return the reference's token and leave the reference's rng state; the
normalised probabilities and the serial double normaliser must be bitwise the oracle's; every
chunk replay inside the kernel must agree with the chunk start its parallel scan computed
(diag status 0). Logit families cover heavy ties, underflowing exponentials and denormal
probabilities, near-uniform and peaked distributions, NaN and infinite logits, vocabularies of
1 .. 128256, and every parameter path of the reference (greedy shortcut, prefilter, top-k,
nucleus, out-of-range values normalised by init).
"""
import ctypes
import sys
import zlib

import numpy as np
import pytest

from _bind import RefSampler
from test_oracle_sampler import CONFIGS, LOGITS6, logit_family

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def check_seq(gpu, oracle, ref, n, cfg, seed, seq, check_probs=True, forced=False):
    dev = gpu.Sampler(n, *cfg, seed)
    rs = RefSampler(ref, n, *cfg, seed)
    orc = oracle.sampler(n, *cfg, seed)
    greedy = rs.st.temperature == 0.0 or rs.st.top_k == 1
    try:
        for k, lg in enumerate(seq):
            want = rs.sample(lg)
            got = dev.sample(lg)
            assert got == want, f"n={n} cfg={cfg} draw {k}: device {got} reference {want}"
            assert dev.rng == rs.rng, f"n={n} cfg={cfg} draw {k}: rng state differs"
            if greedy:
                continue
            d, q = dev.diag(probs=check_probs)
            if forced:  # every exact sum took the serial pass
                assert d[1] != 0 or np.isnan(d[0]), "forced serial pass not reported"
            else:
                assert d[1] == 0, f"chunk replay mismatch (status {d[1]})"
            orc.sample(lg)
            if np.isnan(orc.total.value):
                continue
            assert d[0] == orc.total.value, f"normaliser {d[0]!r} vs {orc.total.value!r}"
            if check_probs:
                assert np.array_equal(bits(q), bits(orc.q)), "probabilities differ"
    finally:
        dev.close()


@pytest.mark.parametrize("cfg", CONFIGS)
def test_sampler_families_small_vocab(gpu, oracle, ref, cfg):
    say("sampler", cfg)
    for kind in ("normal2", "peaky", "flat", "ties", "wide", "zeros"):
        rs = np.random.default_rng(zlib.crc32(repr((kind, cfg)).encode()))
        for n in (1, 2, 6, 300, 5000):
            check_seq(gpu, oracle, ref, n, cfg, 1 + n, [logit_family(kind, n, rs) for _ in range(4)])


@pytest.mark.parametrize("cfg", [(0.8, 0, 0.95), (1.0, 0, 1.0), (0.9, 40, 0.9), (0.6, 0, 0.5), (1.3, 1000, 1.0)])
def test_sampler_32k(gpu, oracle, ref, cfg):
    say("sampler 32k", cfg)
    rs = np.random.default_rng(zlib.crc32(repr(cfg).encode()))
    seq = [logit_family(k, 32000, rs) for k in ("normal2", "peaky", "flat", "wide", "ties", "zeros", "normal2")]
    check_seq(gpu, oracle, ref, 32000, cfg, 17, seq)


@pytest.mark.parametrize("n", [8193, 20000])
def test_sampler_grid_path_sizes(gpu, oracle, ref, n):
    # vocabularies above 8192 take the multi-workgroup path: every family and parameter path
    say("sampler grid path", n)
    for cfg in [(0.8, 0, 0.95), (1.0, 0, 1.0), (0.7, 40, 0.9), (1.0, 3, 1.0), (1.0, 0, 1e-6), (0.5, 0, 0.5)]:
        rs = np.random.default_rng(zlib.crc32(repr((n, cfg)).encode()))
        seq = [logit_family(k, n, rs) for k in ("normal2", "peaky", "flat", "ties", "wide", "zeros")]
        check_seq(gpu, oracle, ref, n, cfg, 23, seq)


@pytest.mark.parametrize("n", [5000, 32000])
def test_sampler_serial_fallback(gpu, oracle, ref, monkeypatch, n):
    """The path a failed binade certificate takes (recomputing every chunk start and end by one
    serial pass), forced from the host for a sampler created with QMH_SAMPLER_SERIAL set: tokens and
    rng states stay the reference's, on both the one-workgroup (n <= 8192) and the grid path."""
    say("sampler serial fallback", n)
    monkeypatch.setenv("QMH_SAMPLER_SERIAL", "1")
    rs = np.random.default_rng(zlib.crc32(repr(("fallback", n)).encode()))
    seq = [logit_family(k, n, rs) for k in ("normal2", "peaky", "flat", "ties", "wide")]
    for cfg in [(0.8, 0, 0.95), (1.0, 0, 1.0), (0.7, 40, 0.9)]:
        check_seq(gpu, oracle, ref, n, cfg, 31, seq, forced=True)


def test_sampler_large_vocab(gpu, oracle, ref):
    # a Llama-3-sized vocabulary: 126 elements per chunk
    rs = np.random.default_rng(3)
    seq = [logit_family(k, 128256, rs) for k in ("normal2", "peaky", "flat")]
    check_seq(gpu, oracle, ref, 128256, (0.8, 0, 0.95), 5, seq)
    check_seq(gpu, oracle, ref, 128256, (1.0, 0, 1.0), 6, seq[:2])


def test_sampler_adversarial_sums(gpu, oracle, ref):
    """Exponentials that are small multiples of powers of two: the serial normaliser meets exact
    round-half-even ties and lands on binade edges; leading underflowed zeros; a lone 1.0."""
    rs = np.random.default_rng(21)
    n = 32000
    seq = []
    for _ in range(4):
        k = rs.integers(0, 40, n)
        m = rs.integers(4, 8, n).astype(np.float64) / 4.0  # 1, 1.25, 1.5, 1.75
        seq.append(np.log(m * 2.0 ** -k).astype(np.float32))
    x = np.full(n, -200.0, np.float32)  # every exponential underflows except one
    x[n - 1] = 0.0
    seq.append(x)
    x = (rs.standard_normal(n) * 3).astype(np.float32)
    x[: n // 2] = -150.0  # a long run of denormal / zero probabilities before the mass
    seq.append(x)
    for cfg in [(1.0, 0, 1.0), (0.8, 0, 0.95), (1.0, 0, 0.5)]:
        check_seq(gpu, oracle, ref, n, cfg, 99, seq)


def test_sampler_nonfinite(gpu, oracle, ref):
    rs = np.random.default_rng(11)
    for n in (1, 2, 7, 300, 4096, 20000):
        base = (rs.standard_normal(n) * 2).astype(np.float32)
        cases = []
        for v in (np.nan, np.inf, -np.inf):
            for at in sorted({0, n // 2, n - 1}):
                x = base.copy()
                x[at] = v
                cases.append(x)
        cases.append(np.full(n, -np.inf, np.float32))
        cases.append(np.full(n, np.nan, np.float32))
        for cfg in [(0.8, 0, 0.95), (1.0, 0, 1.0), (1.0, 2, 1.0), (np.inf, 0, 0.9), (np.nan, 0, 0.9), (1e-30, 0, 0.9)]:
            check_seq(gpu, oracle, ref, n, cfg, 3, cases)


def test_sampler_kats_and_long_sequence(gpu, ref):
    # tests/test_sampler.c:11-16, 77-85
    with gpu.Sampler(6, 0.0, 0, 1.0, 1) as s:
        assert s.sample(LOGITS6) == 1 and s.rng == 1  # greedy draws nothing
    with gpu.Sampler(6, 1.0, 1, 1.0, 1) as s:
        assert s.sample(LOGITS6) == 1
    with gpu.Sampler(6, 1.0, 0, 1e-6, 1) as s:
        assert all(s.sample(LOGITS6) == 1 for _ in range(50))
    with gpu.Sampler(1000, 1.0, 0, 1e-6, 4) as s:
        assert all(s.sample(np.zeros(1000, np.float32)) == 0 for _ in range(20))
    # 2000 draws of the reference's temperature test: the same sequence, hence the same counts
    with gpu.Sampler(6, 0.7, 0, 1.0, 123) as s:
        r = RefSampler(ref, 6, 0.7, 0, 1.0, 123)
        got = [s.sample(LOGITS6) for _ in range(2000)]
        want = [r.sample(LOGITS6) for _ in range(2000)]
        assert got == want and s.rng == r.rng
    with pytest.raises(gpu.QmhError):
        gpu.Sampler(0, 1.0, 0, 1.0, 1)


def test_sampler_device_pointer_and_stream(gpu, ref):
    n = 5000
    lg = (np.random.default_rng(8).standard_normal(n) * 2).astype(np.float32)
    buf = gpu.DeviceBuffer.from_array(lg)
    with gpu.Sampler(n, 0.9, 0, 0.9, 77) as s:
        r = RefSampler(ref, n, 0.9, 0, 0.9, 77)
        for _ in range(5):
            assert s.sample(buf) == r.sample(lg)
    buf.free()


def oracle_sampled_run(oracle, path, prompt, n_gen, cfg, seed):
    """The reference's generation loop (src/main.c:127-141) on the oracle, EOS not a stop:
    prompt forwards, then sample -> forward, n_gen times."""
    err = ctypes.create_string_buffer(256)
    m = oracle.L.or_model_load(path.encode(), 0, err, 256)
    assert m, err.value.decode()
    try:
        dims = np.zeros(7, np.int32)
        oracle.L.or_model_dims(m, dims.ctypes.data)
        V = int(dims[5])
        s = oracle.sampler(V, *cfg, seed)
        lg = None
        for i, t in enumerate(prompt):
            lg = np.ctypeslib.as_array(oracle.L.or_model_forward(m, int(t), i), shape=(V,)).copy()
        ids = []
        pos = len(prompt)
        for _ in range(n_gen):
            ids.append(s.sample(lg))
            lg = np.ctypeslib.as_array(oracle.L.or_model_forward(m, ids[-1], pos), shape=(V,)).copy()
            pos += 1
        return ids, s.rng
    finally:
        oracle.L.or_model_free(m)


@pytest.mark.parametrize("cfg", [(0.8, 0, 0.95), (1.0, 0, 1.0), (0.7, 20, 0.9), (0.0, 0, 0.9)])
def test_model_sample_matches_oracle(gpu, oracle, small_models, cfg):
    say("model sample", cfg)
    path = small_models[("small", "q4_0")]
    prompt = [3, 17, 101, 5, 42]
    n_gen = 40
    want, want_rng = oracle_sampled_run(oracle, path, prompt, n_gen, cfg, 42)
    with gpu.Model.load(path) as m, gpu.Sampler(m.vocab, *cfg, 42) as s:
        m.prefill(prompt[:-1], 0)
        got = m.sample(s, prompt[-1], len(prompt) - 1, n_gen)
        assert list(got) == want
        assert s.rng == want_rng


def test_model_sample_reference_protocol(gpu, oracle, small_models):
    """tests/test_model.c:104-126: BOS at position 0, qm_sampler_init(0.9, 20, 0.9, 1234), 40 sampled
    steps on a q8_0 model; the sequence is the oracle's, and a second run repeats it."""
    path = small_models[("small", "q8_0")]
    cfg = (0.9, 20, 0.9)
    # oracle: forward(BOS, 0), then 40 x (sample, forward); the device loop is the same 40 draws
    want, want_rng = oracle_sampled_run(oracle, path, [0], 40, cfg, 1234)
    runs = []
    for _ in range(2):
        with gpu.Model.load(path) as m, gpu.Sampler(m.vocab, *cfg, 1234) as s:
            runs.append((list(m.sample(s, 0, 0, 40)), s.rng))
    assert runs[0] == runs[1]
    assert runs[0][0] == want and runs[0][1] == want_rng
