"""Pin the oracle's whole-model forward against the compiled reference (scalar ISA) on
generated .qlm files, and check the generator against the reference's own loader and
quantizer. CPU only."""
import os
import subprocess

import numpy as np
import pytest

from _bind import F32, Q4_0, Q8_0, REF_CLI, ref_run, row_bytes

DT = {"f32": F32, "q8_0": Q8_0, "q4_0": Q4_0}


@pytest.mark.parametrize("shape", ["small", "odd", "mha", "gqa"])
@pytest.mark.parametrize("wt", ["f32", "q8_0", "q4_0"])
def test_oracle_forward_bitexact_vs_reference(oracle, small_models, qmh, shape, wt):
    path = small_models[(shape, wt)]
    prompt = qmh.prompt_ids(270 if shape == "gqa" else 6, 300 if shape in ("mha", "gqa") else 458, seed=5)
    lg, ids = oracle.run_model(path, prompt, n_gen=14)
    res, rl = ref_run(path, prompt, 14, isa="scalar")
    rl = rl.reshape(lg.shape)
    assert np.array_equal(lg.view(np.uint32), rl.view(np.uint32))
    assert list(ids) == res["tokens"]


def test_oracle_rejects_bad_token_and_pos(oracle, small_models):
    import ctypes
    m = oracle.model_forward_checks(small_models[("small", "q8_0")])
    try:
        assert not oracle.L.or_model_forward(m, 0, 64)      # pos beyond context
        assert not oracle.L.or_model_forward(m, 458, 0)     # token beyond vocab
        assert not oracle.L.or_model_forward(m, -1, 0)
        assert oracle.L.or_model_forward(m, 3, 0)
    finally:
        oracle.L.or_model_free(m)
    del ctypes


def test_oracle_c1_shape_bitexact(oracle, qmh, tmp_path):
    """BASELINE config c1 (stories15M shape, Q8_0): a few positions, bit-exact with the reference."""
    w = qmh.WORKLOADS["c1"]
    p = str(tmp_path / "c1.qlm")
    qmh.gen_model(p, w.config(), w.wtype, seed=w.seed)
    prompt = qmh.prompt_ids(w.n_prompt, w.vocab_size)
    lg, ids = oracle.run_model(p, prompt, n_gen=4)
    res, rl = ref_run(p, prompt, 4, isa="scalar")
    assert np.array_equal(lg.view(np.uint32), rl.reshape(lg.shape).view(np.uint32))
    assert list(ids) == res["tokens"]


# ---------------------------------------------------------------------------- generator

def test_generator_file_is_read_by_reference(small_models):
    path = small_models[("odd", "q4_0")]
    r = subprocess.run([REF_CLI, "info", path], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    # same check as the reference's CLI test (tests/test_cli.sh:20)
    assert any(line.split()[:3] == ["layers.0.wq", "q4_0", "[72,"] for line in r.stdout.splitlines()), r.stdout


@pytest.mark.parametrize("wt", ["q8_0", "q4_0"])
def test_generator_quantizes_like_reference(ref, qmh, small_models, wt):
    """Bytes in the file == the reference quantizer applied to the generator's f32 values."""
    path = small_models[("small", wt)]
    buf = np.fromfile(path, np.uint8)
    # tensor table: re-parse with numpy (format: reference src/qlm_file.h:1-9)
    import struct
    ver, n_kv, n_t, data_off = struct.unpack_from("<IIIQ", buf, 4)
    off = 24
    for _ in range(n_kv):
        (kl,) = struct.unpack_from("<I", buf, off)
        off += 4 + kl
        (ty,) = struct.unpack_from("<I", buf, off)
        off += 4
        if ty in (0, 1):
            off += 4
        elif ty == 2:
            (sl,) = struct.unpack_from("<I", buf, off)
            off += 4 + sl
        else:
            (cnt,) = struct.unpack_from("<I", buf, off)
            off += 4 + 4 * cnt
    tensors = []
    for ti in range(n_t):
        (nl,) = struct.unpack_from("<I", buf, off)
        name = bytes(buf[off + 4: off + 4 + nl]).decode()
        off += 4 + nl
        dt, nd = struct.unpack_from("<II", buf, off)
        off += 8
        ne = struct.unpack_from(f"<{nd}Q", buf, off)
        off += 8 * nd
        (toff,) = struct.unpack_from("<Q", buf, off)
        off += 8
        tensors.append((ti, name, dt, ne, toff))
    names = [t[1] for t in tensors]
    assert names[0] == "tok_embd" and names[-2:] == ["norm", "output"] and names[1:10] == [
        f"layers.0.{s}" for s in ("attn_norm", "wq", "wk", "wv", "wo", "ffn_norm", "w1", "w2", "w3")]
    seed = 11
    for ti, name, dt, ne, toff in tensors:
        if len(ne) == 1:
            vals = np.frombuffer(buf[data_off + toff: data_off + toff + 4 * ne[0]].tobytes(), np.float32)
            assert np.all(vals == 1.0), name
            continue
        assert dt == DT[wt]
        rows, cols = ne
        rb = row_bytes(dt, cols)
        for r in (0, rows // 2, rows - 1):
            x = qmh.gen_values(seed, ti, r * cols, cols)
            want = ref.quantize(dt, x)[0]
            got = buf[data_off + toff + r * rb: data_off + toff + (r + 1) * rb]
            assert np.array_equal(got, want), (name, r)
    # N(0, 0.02): sample moments of one big tensor
    v = qmh.gen_values(seed, 7, 0, 200000)
    assert abs(v.mean()) < 3e-4 and abs(v.std() - 0.02) < 3e-4


def test_generator_is_thread_count_invariant(qmh, tmp_path):
    cfg = qmh.QmhConfig(64, 172, 2, 4, 2, 458, 64, 10000.0, 1e-5)
    a, b = str(tmp_path / "a.qlm"), str(tmp_path / "b.qlm")
    qmh.gen_model(a, cfg, "q4_0", seed=3, threads=1)
    qmh.gen_model(b, cfg, "q4_0", seed=3, threads=7)
    assert open(a, "rb").read() == open(b, "rb").read()
    assert os.path.getsize(a) % 64 == 0
