"""qmh_sample_noalloc (the sampler entry point that allocates nothing; its scratch is one static
device array per GPU) against qmh_sample with a sampler object (the existing entry point), through
the C ABI: the same token and the same rng state after every draw, over calls in a row whose
vocabularies shrink (the static scratch keeps the previous call's contents), on the grid path
(vocabulary > 8192) and the one-workgroup path, and the greedy shortcut. Also: sizes beyond the
scratch are rejected with an error, and the entry point recorded into a HIP graph by stream capture
(what it is for) replays to the same draws as eager calls."""
import ctypes
import sys
import zlib

import numpy as np
import pytest

from test_oracle_sampler import logit_family

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def draw_noalloc(q, logits_dev, n, cfg, rng_dev, out_dev):
    L = q.load_library()
    rc = L.qmh_sample_noalloc(logits_dev.ptr, n, cfg[0], cfg[1], cfg[2], rng_dev.ptr, out_dev.ptr, None)
    assert rc == 0, q.last_error()
    q.sync()
    return int(out_dev.to_array(np.int32)[0]), int(rng_dev.to_array(np.uint64)[0])


# (vocabulary sequence: each call after the previous one, sizes shrinking), sampler parameters
CASES = [
    ((32000, 20000), (0.8, 0, 0.95)),
    ((131072, 9000), (1.0, 0, 1.0)),
    ((20000, 5000), (0.7, 40, 0.9)),
    ((8192, 300), (0.9, 0, 0.5)),
    ((32000, 2000), (0.0, 0, 1.0)),  # greedy shortcut: argmax, the rng untouched
]


@pytest.mark.parametrize("sizes,cfg", CASES)
def test_noalloc_matches_sampler_object(gpu, sizes, cfg):
    q = gpu
    seed = 0x1234567 + sizes[0]
    rs = np.random.default_rng(zlib.crc32(repr((sizes, cfg)).encode()))
    rng_dev = q.DeviceBuffer.from_array(np.array([seed], np.uint64))
    out_dev = q.DeviceBuffer(4)
    for n in sizes:
        say("noalloc", n, cfg)
        ref = q.Sampler(n, *cfg, seed)
        try:
            # the object sampler and the no-alloc one start from the same state
            rng_dev.free()
            rng_dev = q.DeviceBuffer.from_array(np.array([ref.rng], np.uint64))
            for kind in ("normal2", "peaky", "ties", "flat"):
                lg = logit_family(kind, n, rs)
                ldev = q.DeviceBuffer.from_array(lg)
                want = ref.sample(ldev)
                got, st = draw_noalloc(q, ldev, n, cfg, rng_dev, out_dev)
                assert got == want, f"n={n} {kind}: noalloc {got} vs sampler {want}"
                assert st == ref.rng, f"n={n} {kind}: rng state differs"
                ldev.free()
        finally:
            ref.close()
    rng_dev.free()
    out_dev.free()


def test_noalloc_rejects_oversize(gpu):
    q = gpu
    L = q.load_library()
    big = 131073
    lg = q.DeviceBuffer(4 * big)
    rng_dev = q.DeviceBuffer.from_array(np.array([7], np.uint64))
    out_dev = q.DeviceBuffer(4)
    assert L.qmh_sample_noalloc(lg.ptr, big, 1.0, 0, 1.0, rng_dev.ptr, out_dev.ptr, None) == -1
    assert "131072" in q.last_error()
    assert L.qmh_sample_noalloc(lg.ptr, 0, 1.0, 0, 1.0, rng_dev.ptr, out_dev.ptr, None) == -1
    assert L.qmh_sample_noalloc(None, 100, 1.0, 0, 1.0, rng_dev.ptr, out_dev.ptr, None) == -1
    for b in (lg, rng_dev, out_dev):
        b.free()


def _hip():
    for name in ("libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"):
        try:
            return ctypes.CDLL(name)
        except OSError:
            continue
    pytest.skip("HIP runtime library not found")


@pytest.mark.parametrize("n", [32000, 6000])
def test_noalloc_under_graph_capture(gpu, n):
    """qmh_sample_noalloc recorded into a graph on a stream of the caller's (thread-local capture),
    then replayed five times with new logits copied in between (eager copies and synchronizations
    around every replay): each replay draws the same token and leaves the same rng state as an eager
    call from the graph's state on the same logits. n = 6000 takes the one-workgroup path."""
    q = gpu
    L = q.load_library()
    hip = _hip()
    vp = ctypes.c_void_p
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(vp)]
    hip.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
    hip.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
    hip.hipGraphInstantiate.argtypes = [ctypes.POINTER(vp), vp, vp, vp, ctypes.c_size_t]
    hip.hipGraphLaunch.argtypes = [vp, vp]
    for f in (hip.hipStreamSynchronize, hip.hipGraphExecDestroy, hip.hipGraphDestroy, hip.hipStreamDestroy):
        f.argtypes = [vp]
    cfg = (0.8, 0, 0.95)
    rs = np.random.default_rng(n)
    ldev = q.DeviceBuffer(4 * n)
    rng_g = q.DeviceBuffer.from_array(np.array([0x2545F4914F6CDD1D + n], np.uint64))
    rng_e = q.DeviceBuffer(8)
    out_g, out_e = q.DeviceBuffer(4), q.DeviceBuffer(4)
    stream, graph, exe = vp(), vp(), vp()
    assert hip.hipStreamCreate(ctypes.byref(stream)) == 0
    try:
        say("capture", n)
        assert hip.hipStreamBeginCapture(stream, 1) == 0
        rc = L.qmh_sample_noalloc(ldev.ptr, n, cfg[0], cfg[1], cfg[2], rng_g.ptr, out_g.ptr, stream)
        assert hip.hipStreamEndCapture(stream, ctypes.byref(graph)) == 0
        assert rc == 0, q.last_error()
        assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        for kind in ("normal2", "peaky", "ties", "flat", "normal2"):
            say("replay", n, kind)
            lg = logit_family(kind, n, rs)
            assert L.qmh_memcpy_h2d(ldev.ptr, lg.ctypes.data, lg.nbytes) == 0
            st0 = rng_g.to_array(np.uint64)
            assert L.qmh_memcpy_h2d(rng_e.ptr, st0.ctypes.data, 8) == 0
            want, want_st = draw_noalloc(q, ldev, n, cfg, rng_e, out_e)
            assert hip.hipGraphLaunch(exe, stream) == 0
            assert hip.hipStreamSynchronize(stream) == 0
            got, got_st = int(out_g.to_array(np.int32)[0]), int(rng_g.to_array(np.uint64)[0])
            assert got == want, f"{kind}: replay {got} vs eager {want}"
            assert got_st == want_st != int(st0[0]), f"{kind}: rng state"
    finally:
        if exe:
            hip.hipGraphExecDestroy(exe)
        if graph:
            hip.hipGraphDestroy(graph)
        hip.hipStreamDestroy(stream)
        for b in (ldev, rng_g, rng_e, out_g, out_e):
            b.free()
