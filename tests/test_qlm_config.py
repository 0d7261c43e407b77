"""The .qlm metadata reader against the compiled reference's own qm_model_load (CPU only).

The reference looks a key up by its first entry (qlm_find_kv, src/qlm_file.c:181-185) and
takes the configuration from it (src/model.c:8-21,35-53): a duplicated key's later entries are
ignored, a first entry of the wrong type makes a required key "missing/invalid" and an optional
one take its default. The files are generated models whose metadata table is rewritten here;
the tensor table and data are kept byte for byte."""
import numpy as np
import pytest

from _qlm import ARR, F32, STR, U32, f32, read_qlm, u32, write_qlm  # noqa: F401


@pytest.fixture(scope="module")
def base(qmh, tmp_path_factory):
    d = tmp_path_factory.mktemp("qlmcfg")
    p = str(d / "base.qlm")
    cfg = qmh.QmhConfig(64, 172, 2, 4, 2, 300, 64, 10000.0, 1e-5)
    qmh.gen_model(p, cfg, "q8_0", seed=3, threads=2)
    return d, read_qlm(p)


def edited(base, name, edit):
    d, (ver, kv, n_t, table, data) = base
    p = str(d / f"{name}.qlm")
    write_qlm(p, ver, edit(list(kv)), n_t, table, data)
    return p


def insert_after(kv, key, entry):
    i = next(j for j, e in enumerate(kv) if e[0] == key)
    return kv[:i + 1] + [entry] + kv[i + 1:]


def insert_before(kv, key, entry):
    i = next(j for j, e in enumerate(kv) if e[0] == key)
    return kv[:i] + [entry] + kv[i:]


CASES = {
    "unchanged": lambda kv: kv,
    # a later duplicate of a required key does not override the first
    "dup_dim_later": lambda kv: insert_after(kv, "llama.dim", ("llama.dim", U32, u32(72))),
    "dup_max_seq_later": lambda kv: kv + [("llama.max_seq", U32, u32(16))],
    # a first entry of the wrong type makes the key invalid although a valid one follows
    "first_n_layers_f32": lambda kv: insert_before(kv, "llama.n_layers", ("llama.n_layers", F32, f32(2.0))),
    "first_vocab_zero": lambda kv: insert_before(kv, "llama.vocab_size", ("llama.vocab_size", U32, u32(0))),
    # optional keys: the first entry's value, or the default when its type is wrong
    "rope_first_wins": lambda kv: [("llama.rope_theta", F32, f32(500000.0))] + kv + [("llama.rope_theta", F32, f32(7.0))],
    "eps_first_wrong_type": lambda kv: [("llama.norm_eps", U32, u32(1))] + kv + [("llama.norm_eps", F32, f32(1e-3))],
    "eps_later_only": lambda kv: kv + [("llama.norm_eps", F32, f32(2e-6))],
}


@pytest.mark.parametrize("case", sorted(CASES))
@pytest.mark.parametrize("max_seq", [0, 20])
def test_config_matches_reference_loader(qmh, ref, base, case, max_seq):
    path = edited(base, case, CASES[case])
    want, err = ref.model_config(path, max_seq)
    if want is None:
        with pytest.raises(qmh.QmhError) as e:
            qmh.qlm_config(path, max_seq)
        assert err in str(e.value)
        return
    got = qmh.qlm_config(path, max_seq).as_dict()
    for k, v in want.items():
        if isinstance(v, float):
            assert np.float32(got[k]).tobytes() == np.float32(v).tobytes(), (case, k, got[k], v)
        else:
            assert got[k] == v, (case, k, got[k], v)


def test_duplicate_cases_are_not_vacuous(ref, base):
    """The edits reach the paths they name: the reference rejects the wrong-type first entries
    and keeps the first values elsewhere."""
    assert ref.model_config(edited(base, "first_n_layers_f32", CASES["first_n_layers_f32"]))[0] is None
    assert ref.model_config(edited(base, "dup_dim_later", CASES["dup_dim_later"]))[0]["dim"] == 64
    assert ref.model_config(edited(base, "rope_first_wins", CASES["rope_first_wins"]))[0]["rope_theta"] == 500000.0
    eps = ref.model_config(edited(base, "eps_first_wrong_type", CASES["eps_first_wrong_type"]))[0]["norm_eps"]
    assert np.float32(eps) == np.float32(1e-5)
