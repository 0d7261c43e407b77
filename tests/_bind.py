"""ctypes bindings for the CPU checkers -- TEST INFRASTRUCTURE.

* ``Oracle``: our C restatement of the reference's scalar path (oracle/_build/liboracle.so).
* ``Ref``: the reference itself, compiled from /root/reference/src into oracle/_ref/ by
  oracle/Makefile (shared library for per-function checks, ``ref_driver`` for whole-model
  runs). Built in this container and shipped prebuilt to the GPU box.
"""
from __future__ import annotations

import ctypes
import json
import os
import subprocess
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "_build", "liboracle.so")
REF_DIR = os.path.join(ROOT, "oracle", "_ref")
REF_SO = os.path.join(REF_DIR, "libquillm_ref.so")
REF_DRIVER = os.path.join(REF_DIR, "ref_driver")
REF_CLI = os.path.join(REF_DIR, "quillm")

F32, Q8_0, Q4_0 = 0, 2, 3
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18}

vp, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float


def nblocks(n: int) -> int:
    return (n + 31) // 32


def row_bytes(dtype: int, n: int) -> int:
    return n * 4 if dtype == F32 else nblocks(n) * BLOCK_BYTES[dtype]


def _ptr(a):
    return a.ctypes.data if a is not None else None


class Oracle:
    def __init__(self, path: str = ORACLE_SO):
        L = ctypes.CDLL(path)
        sig = {
            "or_h2f": (f32, [ctypes.c_uint16]),
            "or_f2h": (ctypes.c_uint16, [f32]),
            "or_f2h_array": (None, [vp, vp, i64]),
            "or_h2f_array": (None, [vp, vp, i64]),
            "or_quantize_q8": (None, [vp, vp, i64]),
            "or_quantize_q4": (None, [vp, vp, i64]),
            "or_quantize_rows": (None, [ctypes.c_int, vp, vp, i64, i64]),
            "or_row_to_f32": (None, [ctypes.c_int, vp, vp, i64]),
            "or_dot_f32": (f32, [vp, vp, i64]),
            "or_dot_q8": (f32, [vp, vp, i64]),
            "or_dot_q4": (f32, [vp, vp, i64]),
            "or_gemm_nt": (None, [vp, vp, vp, i64, i64, i64, i64, i64, i64]),
            "or_matvec": (None, [ctypes.c_int, vp, i64, i64, vp, vp, vp]),
            "or_rmsnorm": (None, [vp, vp, vp, i64, f32]),
            "or_softmax": (None, [vp, i64]),
            "or_rope": (None, [vp, i64, i64, i64, f32]),
            "or_swiglu": (None, [vp, vp, i64]),
            "or_argmax": (i32, [vp, i32]),
            "or_sampler_init": (None, [vp, i32, f32, ctypes.c_int, f32, ctypes.c_uint64]),
            "or_rng_uniform": (f32, [vp]),
            "or_sample": (i32, [vp, vp, vp, vp, vp]),
            "or_model_load": (vp, [ctypes.c_char_p, ctypes.c_int, ctypes.c_char_p, ctypes.c_size_t]),
            "or_model_free": (None, [vp]),
            "or_model_forward": (ctypes.POINTER(f32), [vp, i32, i32]),
            "or_model_dims": (None, [vp, vp]),
        }
        for n, (r, a) in sig.items():
            fn = getattr(L, n)
            fn.restype, fn.argtypes = r, a
        self.L = L

    # numerics
    def f2h(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.size, np.uint16)
        self.L.or_f2h_array(_ptr(x), _ptr(out), x.size)
        return out

    def h2f(self, h: np.ndarray) -> np.ndarray:
        h = np.ascontiguousarray(h, np.uint16)
        out = np.empty(h.size, np.float32)
        self.L.or_h2f_array(_ptr(h), _ptr(out), h.size)
        return out

    def quantize(self, dtype: int, x: np.ndarray) -> np.ndarray:
        """rows x n floats -> rows x row_bytes uint8 (reference layout)."""
        x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
        rows, n = x.shape
        out = np.zeros((rows, row_bytes(dtype, n)), np.uint8)
        self.L.or_quantize_rows(dtype, _ptr(x), _ptr(out), rows, n)
        return out

    def row_to_f32(self, dtype: int, row: np.ndarray, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        self.L.or_row_to_f32(dtype, _ptr(np.ascontiguousarray(row)), _ptr(out), n)
        return out

    def dot_f32(self, a, b):
        return self.L.or_dot_f32(_ptr(a), _ptr(b), a.size)

    def dot_q8(self, w, x, nb):
        return self.L.or_dot_q8(_ptr(w), _ptr(x), nb)

    def dot_q4(self, w, x, nb):
        return self.L.or_dot_q4(_ptr(w), _ptr(x), nb)

    def gemm_nt(self, A, B):
        M, K = A.shape
        N = B.shape[0]
        C = np.empty((M, N), np.float32)
        self.L.or_gemm_nt(_ptr(A), _ptr(B), _ptr(C), M, N, K, K, K, N)
        return C

    def matvec(self, dtype, W, rows, cols, x):
        y = np.empty(rows, np.float32)
        xq = np.zeros(nblocks(cols) * 34, np.uint8)
        self.L.or_matvec(dtype, _ptr(W), rows, cols, _ptr(x), _ptr(y), _ptr(xq))
        return y, xq

    def rmsnorm(self, x, w, eps):
        out = np.empty_like(x)
        self.L.or_rmsnorm(_ptr(out), _ptr(x), _ptr(w), x.size, eps)
        return out

    def softmax(self, x):
        x = x.copy()
        self.L.or_softmax(_ptr(x), x.size)
        return x

    def rope(self, v, n_heads, hd, pos, theta):
        v = v.copy()
        self.L.or_rope(_ptr(v), n_heads, hd, pos, theta)
        return v

    def swiglu(self, g, u):
        g = g.copy()
        self.L.or_swiglu(_ptr(g), _ptr(u), g.size)
        return g

    def argmax(self, x):
        return self.L.or_argmax(_ptr(x), x.size)

    # sampler
    def sampler(self, n_vocab, temperature, top_k, top_p, seed):
        return OracleSampler(self, n_vocab, temperature, top_k, top_p, seed)

    # model
    def run_model(self, path: str, prompt, n_gen: int, max_seq: int = 0, keep_logits=True):
        """P forwards over prompt then n_gen greedy steps; returns (logits [P+n_gen, V] or None, ids)."""
        err = ctypes.create_string_buffer(256)
        m = self.L.or_model_load(path.encode(), max_seq, err, 256)
        assert m, err.value.decode()
        try:
            dims = np.zeros(7, np.int32)
            self.L.or_model_dims(m, _ptr(dims))
            V = int(dims[5])
            rows = []
            lg = None
            for i, t in enumerate(prompt):
                p = self.L.or_model_forward(m, int(t), i)
                lg = np.ctypeslib.as_array(p, shape=(V,)).copy()
                if keep_logits:
                    rows.append(lg)
            ids = [self.argmax(lg)]
            for g in range(n_gen):
                p = self.L.or_model_forward(m, ids[-1], len(prompt) + g)
                lg = np.ctypeslib.as_array(p, shape=(V,)).copy()
                if keep_logits:
                    rows.append(lg)
                ids.append(self.argmax(lg))
            return (np.stack(rows) if keep_logits else None), np.array(ids, np.int32)
        finally:
            self.L.or_model_free(m)

    def model_forward_checks(self, path: str, max_seq: int = 0):
        err = ctypes.create_string_buffer(256)
        m = self.L.or_model_load(path.encode(), max_seq, err, 256)
        assert m, err.value.decode()
        return m


class OrSampler(ctypes.Structure):
    """oracle/oracle.h or_sampler."""

    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_int), ("top_p", ctypes.c_float),
                ("rng", ctypes.c_uint64), ("n_vocab", ctypes.c_int32)]


class OracleSampler:
    """A seeded oracle sampler: sample(logits) -> token; q / total of the last call kept."""

    def __init__(self, oracle, n_vocab, temperature, top_k, top_p, seed):
        self.o, self.n = oracle, n_vocab
        self.st = OrSampler()
        oracle.L.or_sampler_init(ctypes.byref(self.st), n_vocab, temperature, top_k, top_p, seed)
        self.q = np.zeros(n_vocab, np.float32)
        self.order = np.zeros(n_vocab, np.int32)
        self.total = ctypes.c_double(0.0)

    @property
    def rng(self):
        return int(self.st.rng)

    def sample(self, logits) -> int:
        lg = np.ascontiguousarray(logits, np.float32)
        assert lg.size == self.n
        return int(self.o.L.or_sample(ctypes.byref(self.st), _ptr(lg), _ptr(self.q), _ptr(self.order),
                                      ctypes.byref(self.total)))


class QmTensor(ctypes.Structure):
    """The reference's qm_tensor (src/ops.h:9-15)."""

    _fields_ = [("name", ctypes.c_char * 64), ("type", ctypes.c_int), ("ndim", ctypes.c_int),
                ("ne", ctypes.c_int64 * 4), ("data", ctypes.c_void_p)]


class Ref:
    """The compiled reference: per-function calls through its own exported C symbols."""

    ISA = {"scalar": 0, "avx2": 1, "avx512": 2}

    def __init__(self, path: str = REF_SO):
        L = ctypes.CDLL(path)
        sig = {
            "qm_fp16_to_fp32": (f32, [ctypes.c_uint16]),
            "qm_fp32_to_fp16": (ctypes.c_uint16, [f32]),
            "qm_quantize_row_q8": (None, [vp, vp, i64]),
            "qm_quantize_row_q4": (None, [vp, vp, i64]),
            "qm_row_to_f32": (None, [ctypes.c_int, vp, vp, i64]),
            "qm_kernels_for": (vp, [ctypes.c_int]),
            "qm_kernels_select": (ctypes.c_int, [ctypes.c_int]),
            "qm_matvec": (None, [vp, ctypes.POINTER(QmTensor), vp, vp, vp]),
            "qm_matmul_nt": (None, [vp, vp, vp, vp, i64, i64, i64]),
            "qm_rmsnorm": (None, [vp, vp, vp, i64, f32]),
            "qm_softmax": (None, [vp, i64]),
            "qm_rope": (None, [vp, i64, i64, i64, f32]),
            "qm_swiglu": (None, [vp, vp, i64]),
            "qm_argmax": (i32, [vp, i32]),
            "qm_arena_init": (ctypes.c_int, [vp, ctypes.c_size_t]),
            "qm_arena_reset": (None, [vp]),
            "qm_arena_free": (None, [vp]),
            "qm_sampler_init": (ctypes.c_int, [vp, vp, i32, f32, ctypes.c_int, f32, ctypes.c_uint64]),
            "qm_sample": (i32, [vp, vp]),
            "qm_rng_uniform": (f32, [vp]),
            "qm_model_load": (ctypes.c_int, [vp, ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_char_p,
                                             ctypes.c_size_t]),
            "qm_model_free": (None, [vp]),
        }
        for n, (r, a) in sig.items():
            fn = getattr(L, n)
            fn.restype, fn.argtypes = r, a
        self.L = L

    def kernels(self, isa: str):
        """(dot_f32, dot_q8, dot_q4, gemm_nt) of an ISA's vtable (src/kernels.h:7-18), or None."""
        p = self.L.qm_kernels_for(self.ISA[isa])
        if not p:
            return None
        ptrs = ctypes.cast(p, ctypes.POINTER(ctypes.c_void_p))
        # struct {qm_isa isa; 4 function pointers}: isa is padded to 8 bytes
        fdot = ctypes.CFUNCTYPE(f32, vp, vp, i64)
        fgemm = ctypes.CFUNCTYPE(None, vp, vp, vp, i64, i64, i64, i64, i64, i64)
        return fdot(ptrs[1]), fdot(ptrs[2]), fdot(ptrs[3]), fgemm(ptrs[4])

    def select(self, isa: str) -> bool:
        return self.L.qm_kernels_select(self.ISA[isa]) == 0

    def quantize(self, dtype: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
        rows, n = x.shape
        out = np.zeros((rows, row_bytes(dtype, n)), np.uint8)
        fn = self.L.qm_quantize_row_q8 if dtype == Q8_0 else self.L.qm_quantize_row_q4
        for r in range(rows):
            fn(_ptr(x[r]), out[r].ctypes.data, n)
        return out

    def row_to_f32(self, dtype: int, row: np.ndarray, n: int) -> np.ndarray:
        out = np.zeros(n, np.float32)
        self.L.qm_row_to_f32(dtype, _ptr(np.ascontiguousarray(row)), _ptr(out), n)
        return out

    def model_config(self, path: str, max_seq: int = 0):
        """(config dict, None) from the reference's own qm_model_load (src/model.c:35-117), or
        (None, its error message). qm_config is the first member of qm_model (src/model.h:17-18)."""
        m = ctypes.create_string_buffer(1 << 16)  # larger than sizeof(qm_model)
        err = ctypes.create_string_buffer(256)
        if self.L.qm_model_load(m, path.encode(), 1, max_seq, err, 256) != 0:
            return None, err.value.decode()
        v = np.frombuffer(m.raw[:36], dtype=np.int32)
        f = np.frombuffer(m.raw[28:36], dtype=np.float32)
        cfg = dict(zip(("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "vocab_size", "max_seq"),
                       (int(x) for x in v[:7])))
        cfg["rope_theta"], cfg["norm_eps"] = float(f[0]), float(f[1])
        self.L.qm_model_free(m)
        return cfg, None

    def matvec(self, dtype, W, rows, cols, x):
        t = QmTensor(b"w", dtype, 2, (ctypes.c_int64 * 4)(rows, cols, 0, 0), W.ctypes.data)
        y = np.empty(rows, np.float32)
        xq = np.zeros(nblocks(cols) * 34, np.uint8)
        self.L.qm_matvec(None, ctypes.byref(t), _ptr(x), _ptr(y), _ptr(xq))
        return y, xq


class QmArena(ctypes.Structure):
    """The reference's qm_arena (src/qm_base.h:49-52)."""

    _fields_ = [("base", ctypes.c_void_p), ("cap", ctypes.c_size_t), ("used", ctypes.c_size_t),
                ("peak", ctypes.c_size_t)]


class QmSampler(ctypes.Structure):
    """The reference's qm_sampler (src/sampler.h:8-16)."""

    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_int), ("top_p", ctypes.c_float),
                ("rng", ctypes.c_uint64), ("n_vocab", ctypes.c_int32), ("probs", ctypes.c_void_p),
                ("idx", ctypes.c_void_p)]


class RefSampler:
    """The compiled reference's own qm_sampler_init / qm_sample, with its arena."""

    def __init__(self, ref, n_vocab, temperature, top_k, top_p, seed):
        self.r, self.n = ref, n_vocab
        self.arena = QmArena()
        assert ref.L.qm_arena_init(ctypes.byref(self.arena), 8 * n_vocab + 4096) == 0
        self.st = QmSampler()
        assert ref.L.qm_sampler_init(ctypes.byref(self.st), ctypes.byref(self.arena), n_vocab, temperature, top_k,
                                     top_p, seed) == 0

    @property
    def rng(self):
        return int(self.st.rng)

    def sample(self, logits) -> int:
        lg = np.ascontiguousarray(logits, np.float32)
        assert lg.size == self.n
        return int(self.r.L.qm_sample(ctypes.byref(self.st), _ptr(lg)))

    def __del__(self):
        try:
            self.r.L.qm_arena_free(ctypes.byref(self.arena))
        except Exception:
            pass


def ref_run(model: str, prompt, n_gen: int, isa: str = "scalar", threads: int = 1, max_seq: int = 0,
            logits: bool = True, warm: bool = False, timeout: float = 900.0):
    """Run the compiled reference on a model: returns (json result, logits [P+G, V] or None)."""
    with tempfile.TemporaryDirectory() as d:
        pf = os.path.join(d, "prompt.txt")
        with open(pf, "w") as f:
            f.write(" ".join(str(int(t)) for t in prompt))
        cmd = [REF_DRIVER, model, "--prompt", pf, "--gen", str(n_gen), "--isa", isa, "--threads", str(threads),
               "--max-seq", str(max_seq)]
        lf = os.path.join(d, "logits.f32")
        if logits:
            cmd += ["--logits", lf]
        if warm:
            cmd += ["--warm"]
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
        if r.returncode != 0:
            raise RuntimeError(f"ref_driver failed ({r.returncode}): {r.stderr}")
        res = json.loads(r.stdout)
        lg = np.fromfile(lf, np.float32) if logits else None
        return res, lg


def accum_tol(n: int, abs_sum: float) -> float:
    """The reference's float accumulation bound (tests/test_kernels.c:13)."""
    return 4.0 * (n + 16) * 6e-8 * abs_sum + 1e-30
