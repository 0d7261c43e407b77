"""The C-ABI library loads and exports every symbol include/qmhip.h declares; without a GPU
its entry points fail loudly (an error code and message), never silently on the CPU."""
import ctypes

import numpy as np
import pytest


def test_library_exports_every_declared_symbol(qmh):
    lib = ctypes.CDLL(qmh.LIB_PATH)
    names = qmh.exported_symbols()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_header_is_plain_c(qmh):
    import re
    text = open(qmh.INCLUDE).read()
    assert 'extern "C"' in text
    code = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    for banned in ("torch", "hipStream_t", "std::", "template", "class "):
        assert banned not in code


def test_no_device_fails_loudly(qmh):
    if qmh.available():
        pytest.skip("a GPU is visible: covered by the gpu tests")
    L = qmh.load_library()
    assert L.qmh_init(0) == -1
    assert "device" in qmh.last_error().lower()
    assert not L.qmh_model_load(b"/nonexistent.qlm", 0)
    with pytest.raises(qmh.QmhError):
        qmh.Model.load("/nonexistent.qlm")


def test_prompt_ids_are_seeded_and_in_range(qmh):
    a = qmh.prompt_ids(512, 32000, seed=1234)
    b = qmh.prompt_ids(512, 32000, seed=1234)
    assert np.array_equal(a, b) and a.min() >= 2 and a.max() < 32000
    assert not np.array_equal(a, qmh.prompt_ids(512, 32000, seed=1235))
