import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import _bind  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 (MI355X) device; run with -m gpu")


def _need(path, what):
    if not os.path.exists(path):
        pytest.fail(f"{what} missing at {path}: run __graft_entry__.build() first")


@pytest.fixture(scope="session")
def oracle():
    _need(_bind.ORACLE_SO, "oracle library")
    return _bind.Oracle()


@pytest.fixture(scope="session")
def ref():
    _need(_bind.REF_SO, "compiled reference")
    return _bind.Ref()


@pytest.fixture(scope="session")
def qmh():
    import quillm_amd

    quillm_amd.load_library()
    return quillm_amd


@pytest.fixture(scope="session")
def gpu(qmh):
    """The HIP library initialised on device 0 (fails, not skips, without a gfx950 device)."""
    if not qmh.available():
        pytest.fail("no gfx950 device visible")
    qmh.init(0)
    return qmh


# small model shapes in the spirit of the reference's fixtures (tests/gen_fixtures.py:36-44):
# GQA, hidden not a multiple of 32, dim 72 (partial blocks everywhere), head_dim 12
SMALL_SHAPES = {
    "small": dict(dim=64, hidden_dim=172, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=458, max_seq=64),
    "odd": dict(dim=72, hidden_dim=200, n_layers=3, n_heads=6, n_kv_heads=3, vocab_size=458, max_seq=64),
    "mha": dict(dim=96, hidden_dim=256, n_layers=2, n_heads=3, n_kv_heads=3, vocab_size=300, max_seq=48),
    # 12 query heads on one kv head, and a context past one 256-position attention chunk
    "gqa": dict(dim=96, hidden_dim=256, n_layers=2, n_heads=12, n_kv_heads=1, vocab_size=300, max_seq=300),
    # 2 query heads per kv head of 48 dims: the K-tile scores kernel, over two 64-position tiles
    "gqa48": dict(dim=192, hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=300, max_seq=136),
}


@pytest.fixture(scope="session")
def small_models(qmh, tmp_path_factory):
    """{(shape, wtype): path} of generated small models (seeded, N(0,0.02) weights)."""
    d = tmp_path_factory.mktemp("models")
    out = {}
    for shape, dims in SMALL_SHAPES.items():
        for wt in ("f32", "q8_0", "q4_0"):
            p = str(d / f"{shape}_{wt}.qlm")
            cfg = qmh.QmhConfig(**dims, rope_theta=10000.0, norm_eps=1e-5)
            qmh.gen_model(p, cfg, wt, seed=11 if shape == "small" else 22, threads=4)
            out[(shape, wt)] = p
    return out
