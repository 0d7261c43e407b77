"""quillm_amd -- the quillm token loop on one MI355X (gfx950), behind a plain C ABI.

The product is ``libqmhip.so`` (HIP kernels + C11 host runtime, declared in
``include/qmhip.h``). This module is a thin ctypes binding over that ABI, shaped like the
reference's C interface (reference src/model.h:32-36, src/ops.h:25-34) so tests and the bench
read like the reference's own tests. It never falls back to any CPU path: if the library or a
gfx950 device is missing, calls raise.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqmhip.so")
INCLUDE = os.path.join(os.path.dirname(_HERE), "include", "qmhip.h")

F32, Q8_0, Q4_0 = 0, 2, 3
DTYPES = {"f32": F32, "q8_0": Q8_0, "q4_0": Q4_0}


class QmhConfig(ctypes.Structure):
    """qmh_config == the reference's qm_config (src/model.h:8-11)."""

    _fields_ = [("dim", ctypes.c_int32), ("hidden_dim", ctypes.c_int32), ("n_layers", ctypes.c_int32),
                ("n_heads", ctypes.c_int32), ("n_kv_heads", ctypes.c_int32), ("vocab_size", ctypes.c_int32),
                ("max_seq", ctypes.c_int32), ("rope_theta", ctypes.c_float), ("norm_eps", ctypes.c_float)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


class TensorView(ctypes.Structure):
    """qmh_tensor_view == the reference's qm_tensor minus the name (src/ops.h:9-15)."""

    _fields_ = [("dtype", ctypes.c_int32), ("ndim", ctypes.c_int32), ("ne", ctypes.c_int64 * 4),
                ("data", ctypes.c_void_p)]


_lib = None


class QmhError(RuntimeError):
    pass


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libqmhip.so (built by ``__graft_entry__.build()`` / ``make -C quillm_amd``)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise QmhError(f"{path} not built: run `python -c 'import __graft_entry__ as g; g.build()'`")
    L = ctypes.CDLL(path)
    vp, i32, i64, f32, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t
    sig = {
        "qmh_available": (ctypes.c_int, []),
        "qmh_init": (ctypes.c_int, [ctypes.c_int]),
        "qmh_last_error": (ctypes.c_char_p, []),
        "qmh_stream": (vp, []),
        "qmh_dev_alloc": (vp, [sz]),
        "qmh_dev_free": (ctypes.c_int, [vp]),
        "qmh_memcpy_h2d": (ctypes.c_int, [vp, vp, sz]),
        "qmh_memcpy_d2h": (ctypes.c_int, [vp, vp, sz]),
        "qmh_memset": (ctypes.c_int, [vp, ctypes.c_int, sz]),
        "qmh_sync": (ctypes.c_int, []),
        "qmh_fp16_to_fp32": (ctypes.c_int, [vp, vp, i64, vp]),
        "qmh_fp32_to_fp16": (ctypes.c_int, [vp, vp, i64, vp]),
        "qmh_quantize_rows_q8": (ctypes.c_int, [vp, vp, i64, i64, vp]),
        "qmh_quantize_rows_q4": (ctypes.c_int, [vp, vp, i64, i64, vp]),
        "qmh_row_to_f32": (ctypes.c_int, [ctypes.c_int, vp, vp, i64, vp]),
        "qmh_weight_upload": (vp, [ctypes.c_int, i64, i64, vp]),
        "qmh_weight_free": (None, [vp]),
        "qmh_matvec": (ctypes.c_int, [vp, vp, vp, vp, vp]),
        "qmh_time_matvec": (ctypes.c_int, [ctypes.POINTER(vp), ctypes.c_int, vp, vp, ctypes.c_int,
                                           ctypes.POINTER(ctypes.c_double)]),
        "qmh_time_matmul_nt": (ctypes.c_int, [vp, vp, vp, i64, i64, i64, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]),
        "qmh_rmsnorm_matvec": (ctypes.c_int, [vp, vp, vp, f32, vp, vp, vp]),
        "qmh_matmul_nt": (ctypes.c_int, [vp, vp, vp, i64, i64, i64, vp]),
        "qmh_rmsnorm": (ctypes.c_int, [vp, vp, vp, i64, f32, vp]),
        "qmh_softmax": (ctypes.c_int, [vp, i64, vp]),
        "qmh_rope": (ctypes.c_int, [vp, i64, i64, i64, f32, vp]),
        "qmh_swiglu": (ctypes.c_int, [vp, vp, i64, vp]),
        "qmh_argmax": (ctypes.c_int, [vp, i32, vp, vp]),
        "qmh_model_create": (vp, [ctypes.POINTER(QmhConfig), ctypes.POINTER(TensorView), ctypes.POINTER(TensorView),
                                  ctypes.POINTER(TensorView), ctypes.POINTER(TensorView)]),
        "qmh_model_load": (vp, [ctypes.c_char_p, i32]),
        "qmh_model_free": (None, [vp]),
        "qmh_model_config": (ctypes.POINTER(QmhConfig), [vp]),
        "qmh_qlm_config": (ctypes.c_int, [ctypes.c_char_p, i32, ctypes.POINTER(QmhConfig)]),
        "qmh_model_forward": (ctypes.POINTER(ctypes.c_float), [vp, i32, i32]),
        "qmh_model_prefill": (ctypes.c_int, [vp, vp, i32, i32, vp]),
        "qmh_model_greedy": (ctypes.c_int, [vp, i32, i32, i32, vp]),
        "qmh_batch_create": (vp, [vp, i32]),
        "qmh_batch_free": (None, [vp]),
        "qmh_batch_forward": (ctypes.c_int, [vp, vp, vp, vp]),
        "qmh_batch_greedy": (ctypes.c_int, [vp, vp, vp, i32, vp, ctypes.POINTER(ctypes.c_double)]),
        "qmh_sampler_create": (vp, [i32, f32, ctypes.c_int, f32, ctypes.c_uint64]),
        "qmh_sampler_free": (None, [vp]),
        "qmh_sample": (ctypes.c_int, [vp, vp, vp, vp]),
        "qmh_sample_sync": (i32, [vp, vp]),
        "qmh_sample_noalloc": (ctypes.c_int, [vp, i32, f32, ctypes.c_int, f32, vp, vp, vp]),
        "qmh_sampler_rng": (ctypes.c_int, [vp, ctypes.POINTER(ctypes.c_uint64)]),
        "qmh_sampler_diag": (ctypes.c_int, [vp, vp, vp]),
        "qmh_model_sample": (ctypes.c_int, [vp, vp, i32, i32, i32, vp]),
        "qmh_gen_qlm": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(QmhConfig), ctypes.c_int, ctypes.c_uint64,
                                       ctypes.c_int]),
        "qmh_gen_values": (None, [ctypes.c_uint64, ctypes.c_int, i64, i64, vp]),
        "qmh_model_time_stage": (ctypes.c_int, [vp, ctypes.c_int, i32, ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                                                ctypes.POINTER(ctypes.c_double)]),
        "qmh_model_time_greedy": (ctypes.c_int, [vp, i32, i32, i32, vp, ctypes.POINTER(ctypes.c_double)]),
        "qmh_model_time_prefill": (ctypes.c_int, [vp, vp, i32, i32, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]),
        "qmh_model_time_forward": (ctypes.c_int, [vp, i32, i32, i32, vp, ctypes.POINTER(ctypes.c_double)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def exported_symbols() -> list[str]:
    """Every function name declared in include/qmhip.h."""
    import re
    text = open(INCLUDE).read()
    return sorted(set(re.findall(r"\b(qmh_[a-z0-9_]+)\s*\(", text)))


def last_error() -> str:
    return load_library().qmh_last_error().decode(errors="replace")


def _check(rc: int, what: str):
    if rc != 0:
        raise QmhError(f"{what}: {last_error()}")


def qlm_config(path: str, max_seq: int = 0) -> "QmhConfig":
    """The configuration a .qlm file gives the model (qmh_qlm_config; no device needed)."""
    c = QmhConfig()
    _check(load_library().qmh_qlm_config(path.encode(), int(max_seq), ctypes.byref(c)), "qlm_config")
    return c


def available() -> bool:
    return bool(load_library().qmh_available())


def init(device: int = 0):
    _check(load_library().qmh_init(device), "qmh_init")


# ----------------------------------------------------------------------------- device buffers

class DeviceBuffer:
    """A device allocation made through the library (no torch needed)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = load_library().qmh_dev_alloc(max(self.nbytes, 1))
        if not self.ptr:
            raise QmhError(f"qmh_dev_alloc: {last_error()}")

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        if a.nbytes:
            _check(load_library().qmh_memcpy_h2d(b.ptr, a.ctypes.data, a.nbytes), "h2d")
        return b

    def to_array(self, dtype, count: int | None = None) -> np.ndarray:
        dtype = np.dtype(dtype)
        n = self.nbytes // dtype.itemsize if count is None else count
        out = np.empty(n, dtype=dtype)
        if out.nbytes:
            _check(load_library().qmh_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes), "d2h")
        return out

    def free(self):
        if self.ptr:
            load_library().qmh_dev_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def sync():
    _check(load_library().qmh_sync(), "qmh_sync")


# ----------------------------------------------------------------------------- model

class Model:
    """Device model: the HIP counterpart of the reference's qm_model (src/model.h:17-36)."""

    def __init__(self, handle):
        self._h = handle
        self.cfg = load_library().qmh_model_config(handle).contents
        self.vocab = self.cfg.vocab_size

    @classmethod
    def load(cls, path: str, max_seq: int = 0) -> "Model":
        h = load_library().qmh_model_load(path.encode(), int(max_seq))
        if not h:
            raise QmhError(f"qmh_model_load({path}): {last_error()}")
        return cls(h)

    def forward(self, token: int, pos: int) -> np.ndarray | None:
        """Logits (a view of model-owned pinned memory, valid until the next call) or None."""
        p = load_library().qmh_model_forward(self._h, int(token), int(pos))
        if not p:
            return None
        return np.ctypeslib.as_array(p, shape=(self.vocab,))

    def prefill(self, tokens, pos0: int = 0, want_logits: bool = False):
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty((len(toks), self.vocab), np.float32) if want_logits else None
        _check(load_library().qmh_model_prefill(self._h, toks.ctypes.data, len(toks), int(pos0),
                                                 out.ctypes.data if out is not None else None), "prefill")
        return out

    def greedy(self, token: int, pos: int, n_steps: int) -> np.ndarray:
        out = np.zeros(max(n_steps, 1), np.int32)
        _check(load_library().qmh_model_greedy(self._h, int(token), int(pos), int(n_steps), out.ctypes.data),
               "greedy")
        return out[:n_steps]

    def sample(self, sampler: "Sampler", token: int, pos: int, n_steps: int) -> np.ndarray:
        """Sampled decode on the device (qmh_model_sample): the n_steps sampled tokens."""
        out = np.zeros(max(n_steps, 1), np.int32)
        _check(load_library().qmh_model_sample(self._h, sampler._h, int(token), int(pos), int(n_steps),
                                                out.ctypes.data), "model_sample")
        return out[:n_steps]

    STAGES = {"qkv": 0, "wo": 1, "w13": 2, "w2": 3, "output": 4, "attn_scores": 5, "attn_pv": 6, "attn": 7}

    def time_stage(self, stage: str, iters: int, pos: int):
        """(ms per launch, weight bytes per launch) of one decode-step stage at position pos, from HIP events."""
        ms, nbytes = ctypes.c_double(), ctypes.c_double()
        _check(load_library().qmh_model_time_stage(self._h, self.STAGES[stage], int(pos), int(iters),
                                                    ctypes.byref(ms), ctypes.byref(nbytes)), "time_stage")
        return ms.value, nbytes.value

    def time_greedy(self, token: int, pos: int, n_steps: int):
        """(ids, device ms for the n_steps graph replays) of a device greedy run."""
        out = np.zeros(max(n_steps, 1), np.int32)
        ms = ctypes.c_double()
        _check(load_library().qmh_model_time_greedy(self._h, int(token), int(pos), int(n_steps), out.ctypes.data,
                                                     ctypes.byref(ms)), "time_greedy")
        return out[:n_steps], ms.value

    PREFILL_LOGITS = {"none": 0, "last": 1, "all": 2}

    def time_prefill(self, tokens, pos0: int = 0, logits: str = "all") -> float:
        """Device ms of a prefill of tokens at pos0 (logits computed on the device: none, last, all)."""
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        ms = ctypes.c_double()
        _check(load_library().qmh_model_time_prefill(self._h, toks.ctypes.data, len(toks), int(pos0),
                                                      self.PREFILL_LOGITS[logits], ctypes.byref(ms)), "time_prefill")
        return ms.value

    def time_forward(self, token: int, pos: int, n_steps: int):
        """(ids, host ms) of the reference bench's loop: token = argmax(forward(token, pos+k)) on the host."""
        out = np.zeros(max(n_steps, 1), np.int32)
        ms = ctypes.c_double()
        _check(load_library().qmh_model_time_forward(self._h, int(token), int(pos), int(n_steps), out.ctypes.data,
                                                      ctypes.byref(ms)), "time_forward")
        return out[:n_steps], ms.value

    def close(self):
        if self._h:
            load_library().qmh_model_free(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ----------------------------------------------------------------------------- batched decode

class Batch:
    """n_seq independent sequences decoded together over a Model's weights (qmh_batch_*)."""

    def __init__(self, model: "Model", n_seq: int):
        self.model, self.n, self.vocab = model, int(n_seq), model.vocab
        self._h = load_library().qmh_batch_create(model._h, self.n)
        if not self._h:
            raise QmhError(f"qmh_batch_create: {last_error()}")

    def forward(self, tokens, pos, want_logits: bool = True):
        """One step (sequence i takes tokens[i] at pos[i]); logits [n_seq, vocab] or None."""
        t = np.ascontiguousarray(tokens, np.int32)
        p = np.ascontiguousarray(pos, np.int32)
        assert t.size == self.n and p.size == self.n
        out = np.empty((self.n, self.vocab), np.float32) if want_logits else None
        _check(load_library().qmh_batch_forward(self._h, t.ctypes.data, p.ctypes.data,
                                                 out.ctypes.data if out is not None else None), "batch_forward")
        return out

    def greedy(self, tokens, pos, n_steps: int):
        """(ids [n_steps, n_seq], device ms) of n_steps device greedy steps of every sequence."""
        t = np.ascontiguousarray(tokens, np.int32)
        p = np.ascontiguousarray(pos, np.int32)
        out = np.zeros((max(n_steps, 1), self.n), np.int32)
        ms = ctypes.c_double()
        _check(load_library().qmh_batch_greedy(self._h, t.ctypes.data, p.ctypes.data, int(n_steps), out.ctypes.data,
                                                ctypes.byref(ms)), "batch_greedy")
        return out[:n_steps], ms.value

    def close(self):
        if getattr(self, "_h", None):
            load_library().qmh_batch_free(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ----------------------------------------------------------------------------- sampler

class Sampler:
    """Device sampler: the HIP counterpart of the reference's qm_sampler (src/sampler.h:8-24)."""

    def __init__(self, n_vocab: int, temperature: float, top_k: int, top_p: float, seed: int):
        self.n = int(n_vocab)
        self._h = load_library().qmh_sampler_create(self.n, float(temperature), int(top_k), float(top_p),
                                                     int(seed) & (2**64 - 1))
        if not self._h:
            raise QmhError(f"qmh_sampler_create: {last_error()}")
        self._logits = DeviceBuffer(4 * self.n)

    def sample(self, logits) -> int:
        """qm_sample of host logits (uploaded) or of a DeviceBuffer holding n floats."""
        if isinstance(logits, DeviceBuffer):
            ptr = logits.ptr
        else:
            lg = np.ascontiguousarray(logits, np.float32)
            if lg.size != self.n:
                raise ValueError(f"logits of {lg.size} values for a vocabulary of {self.n}")
            _check(load_library().qmh_memcpy_h2d(self._logits.ptr, lg.ctypes.data, 4 * self.n), "h2d")
            ptr = self._logits.ptr
        tok = load_library().qmh_sample_sync(self._h, ptr)
        if tok < 0:
            raise QmhError(f"qmh_sample: {last_error()}")
        return int(tok)

    @property
    def rng(self) -> int:
        st = ctypes.c_uint64()
        _check(load_library().qmh_sampler_rng(self._h, ctypes.byref(st)), "sampler_rng")
        return int(st.value)

    def diag(self, probs: bool = False):
        """(diag[8], probabilities or None) of the last non-greedy draw."""
        d = np.zeros(8, np.float64)
        q = np.zeros(self.n, np.float32) if probs else None
        _check(load_library().qmh_sampler_diag(self._h, d.ctypes.data, q.ctypes.data if probs else None),
               "sampler_diag")
        return d, q

    def close(self):
        if getattr(self, "_h", None):
            load_library().qmh_sampler_free(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ----------------------------------------------------------------------------- workloads

@dataclass(frozen=True)
class Workload:
    """One BASELINE.json config: model shape, weight dtype, seed, prompt and decode lengths."""

    name: str
    dim: int
    hidden_dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    vocab_size: int
    max_seq: int
    wtype: str
    seed: int
    n_prompt: int
    n_gen: int

    def config(self, max_seq: int | None = None) -> QmhConfig:
        return QmhConfig(self.dim, self.hidden_dim, self.n_layers, self.n_heads, self.n_kv_heads, self.vocab_size,
                         self.max_seq if max_seq is None else max_seq, 10000.0, 1e-5)

    @property
    def kvd(self):
        return self.dim // self.n_heads * self.n_kv_heads


# BASELINE.json configs c1..c5 (weights N(0,0.02); seed 1 where the config names none).
# c2 decodes at positions 16..255 (240 steps): 16 + 256 exceeds its seq_len of 256.
WORKLOADS = {
    "c1": Workload("c1", 288, 768, 6, 6, 6, 32000, 256, "q8_0", 1, 4, 64),
    "c2": Workload("c2", 288, 768, 6, 6, 2, 32000, 256, "q4_0", 1, 16, 240),
    "c3": Workload("c3", 768, 2048, 12, 12, 12, 32000, 1024, "q8_0", 1, 128, 512),
    "c4": Workload("c4", 2048, 5632, 22, 32, 4, 32000, 2048, "q4_0", 1, 512, 256),
    "c5a": Workload("c5a", 4096, 11008, 32, 32, 32, 32000, 4096, "q4_0", 1, 512, 128),
    "c5b": Workload("c5b", 4096, 11008, 32, 32, 32, 32000, 4096, "q8_0", 1, 512, 128),
}


def _mix64(z: int) -> int:
    m = (1 << 64) - 1
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
    return z ^ (z >> 31)


def prompt_ids(n: int, vocab: int, seed: int = 1234) -> np.ndarray:
    """n token ids uniform in [2, vocab) from a fixed seed (splitmix64 stream)."""
    out = np.empty(n, np.int32)
    for i in range(n):
        out[i] = 2 + _mix64((seed * 0x9E3779B97F4A7C15 + (i + 1) * 0xD1B54A32D192ED03) & ((1 << 64) - 1)) % (vocab - 2)
    return out


def gen_model(path: str, cfg: QmhConfig, wtype, seed: int = 1, threads: int | None = None):
    """Write a random-init .qlm (N(0,0.02) weights, gains 1.0) with the library's generator."""
    wt = DTYPES[wtype] if isinstance(wtype, str) else int(wtype)
    if threads is None:
        threads = min(os.cpu_count() or 1, 16)
    _check(load_library().qmh_gen_qlm(path.encode(), ctypes.byref(cfg), wt, seed, threads), "qmh_gen_qlm")


def gen_values(seed: int, tensor_index: int, k0: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    load_library().qmh_gen_values(seed, tensor_index, k0, n, out.ctypes.data)
    return out
