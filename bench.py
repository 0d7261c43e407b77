#!/usr/bin/env python3
"""Decode/prefill benchmark of the quillm token loop on one MI355X.

Workload (BASELINE.json metric): config c5a, a 7B-shaped Llama in Q4_0 (dim 4096, hidden 11008,
32 layers, 32/32 heads, vocab 32000), random-init N(0,0.02) weights from a fixed seed, batch 1:
a 512-token random-id prompt, then greedy decode. One "step" is one decode token (a full
forward + argmax, replayed as one hipGraph, inputs resident in HBM); W untimed warmup steps,
then exactly K timed steps at positions P..P+K-1.

Prints one JSON line: decode tok/s (value), prefill tok/s (every position's logits computed, as the
reference's prompt loop does; also with the last position's only), the fraction of the HBM roofline,
`roofline` for the dominant kernel (the fused RMSNorm + W1|W3 Q4_0 matvec + SwiGLU), the prefill
against the int8- and FP32-MFMA peaks, the reference bench's forward loop (logits copied to the host),
the other BASELINE configs (c1-c4, c5b) as extra keys, and `cpu_baseline` = the compiled reference
(best CPU ISA) on a bounded sample of the same workload.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c5a] [--no-cpu] [--no-configs]
  python bench.py --probe-stream        the read ceiling for the weight sizes (probe line, then exit)
  python bench.py --probe-stages POS    the decode stages' times at position POS (probe line, then exit)
"""
import argparse
import json
import os
import shutil
import statistics
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0      # MI355X published HBM3E bandwidth
INT8_PEAK_TOPS = 5000.0    # MI355X dense int8 MFMA
FP32_MFMA_PEAK_TFS = 157.3  # MI355X dense fp32 MFMA
VALU_LANE_OPS = 256 * 4 * 16 * 2.4e9  # fp32 VALU lane operations per second (256 CUs x 4 SIMD x 16 lanes x 2.4 GHz)
CPU_SHARE = 16  # host threads the GPU box allots one GPU's jobs


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def row_bytes(w, n):
    bb = 18 if w.wtype == "q4_0" else 34 if w.wtype == "q8_0" else None
    return (n + 31) // 32 * bb if bb else 4 * n


def decode_bytes_per_token(w, positions):
    """Algorithmic HBM bytes of one decode token, averaged over `positions`: every weight
    stream + K and V reads up to pos + KV writes + norm gains + logits + one embedding row."""
    D, H, L, V, kvd = w.dim, w.hidden_dim, w.n_layers, w.vocab_size, w.kvd
    rb = lambda n: row_bytes(w, n)
    weights = L * ((D + 2 * kvd) * rb(D) + D * rb(D) + 2 * H * rb(D) + D * rb(H)) + V * rb(D)
    kv_read = sum(2 * L * (p + 1) * kvd * 4 for p in positions) / len(positions)
    small = 2 * L * kvd * 4 + (2 * L + 1) * D * 4 + V * 4 + rb(D)
    return weights + kv_read + small, weights


def prefill_flops(w, P, logits_rows):
    """Prefill flops as the reference counts them: every matmul over P tokens, the output matmul over
    logits_rows positions, attention 4*L*D per (query, key) pair of the causal prompt."""
    D, H, L, V, kvd = w.dim, w.hidden_dim, w.n_layers, w.vocab_size, w.kvd
    layer = 2 * D * D + 2 * kvd * D + 3 * H * D
    return 2 * P * L * layer + 2 * logits_rows * V * D + 4 * L * D * P * (P + 1) // 2


def prefill_valu_floor_s(w, P, logits_rows):
    """The bitwise matmul epilogue's VALU floor: 3 operations (cvt, mul, add) per (row, token, block) in
    the reference's order (the scale product dw*dx, exact, comes from an f16 MFMA), at the device's fp32
    VALU rate."""
    D, H, L, V, kvd = w.dim, w.hidden_dim, w.n_layers, w.vocab_size, w.kvd
    nb = lambda n: (n + 31) // 32
    rows_nb = L * ((2 * D + 2 * kvd) * nb(D) + 2 * H * nb(D) + D * nb(H))
    return 3 * (P * rows_nb + logits_rows * V * nb(D)) / VALU_LANE_OPS


def pmc_traffic(name):
    """HBM bytes per launch of a kernel from its committed counter summary (profiles/NAME), the
    line `traffic_bytes_per_launch: N` (FETCH_SIZE + WRITE_SIZE, scaled by a copy kernel)."""
    try:
        for line in open(os.path.join(ROOT, "profiles", name)):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def host_cpus():
    """The host's CPU topology (from /proc/cpuinfo) and the cores this process may run on."""
    logical, cores, model = 0, set(), "?"
    phys = core = None
    for line in open("/proc/cpuinfo"):
        k, _, v = line.partition(":")
        k, v = k.strip(), v.strip()
        if k == "processor":
            logical += 1
        elif k == "physical id":
            phys = v
        elif k == "core id":
            core = v
        elif k == "model name":
            model = v
        elif not k and phys is not None and core is not None:
            cores.add((phys, core))
            phys = core = None
    if phys is not None and core is not None:
        cores.add((phys, core))
    n_phys = len(cores) or logical
    return {"model": model, "logical_cpus": logical, "physical_cores": n_phys,
            "threads_per_core": round(logical / n_phys, 2) if n_phys else None,
            "sockets": len({p for p, _ in cores}) or None, "affinity": len(os.sched_getaffinity(0))}


def cpu_baseline(path, w, q, P, G, runs=3, warm=True, one_thread=True):
    """The compiled reference (oracle/_ref/ref_driver, best CPU ISA) on the config's whole workload, as
    BASELINE.md's plan has it: P sequential qm_model_forward calls over the prompt (the reference's
    only prompt method, src/main.c:127-130), then G greedy steps (bench/bench.c:143-149), max_seq
    P + G, on the box's CPU share of threads; the median of `runs` runs after one untimed warm pass
    over the mmap'd file; optionally one single-thread run on a short sample."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from _bind import REF_DRIVER, ref_run

    if not os.path.exists(REF_DRIVER):
        return None
    flags = open("/proc/cpuinfo").read()
    isa = "avx512" if (" avx512f " in flags and " avx512bw " in flags and " avx512vl " in flags) else "avx2"
    host = host_cpus()
    threads = min(host["affinity"], CPU_SHARE)
    prompt = q.prompt_ids(P, w.vocab_size)
    res = []
    for r in range(runs):
        out, _ = ref_run(path, prompt, G, isa=isa, threads=threads, max_seq=P + G, logits=False,
                         warm=warm and r == 0, timeout=900)
        res.append(out)
        log(f"[bench] cpu baseline {w.name} run {r}: decode {out['decode_tok_s']:.2f} prefill "
            f"{out['prompt_tok_s']:.2f} tok/s")
    dec = [x["decode_tok_s"] for x in res]
    pre = [x["prompt_tok_s"] for x in res]
    cb = {
        "value": round(statistics.median(dec), 3), "unit": "tok/s", "cores": threads, "kind": "reference",
        "isa": res[0]["isa"], "prefill_tok_s": round(statistics.median(pre), 3),
        "runs_decode_tok_s": [round(x, 3) for x in dec], "runs_prefill_tok_s": [round(x, 3) for x in pre],
        "host": host,
        "sample": f"the whole {w.name} workload on the same .qlm file: {P} prompt tokens (sequential "
                  f"qm_model_forward, logits at every position) + {G} greedy decode steps, max_seq {P + G}, "
                  f"QUILLM isa {res[0]['isa']}, {threads} threads (the box's CPU share for one GPU), median "
                  f"of {runs} run{'s' if runs > 1 else ''}" + (" after one untimed warm pass" if warm else ""),
    }
    if one_thread:
        P1, G1 = min(P, 8), min(G, 8)
        one, _ = ref_run(path, prompt[:P1], G1, isa=isa, threads=1, max_seq=P1 + G1, logits=False, timeout=900)
        log(f"[bench] cpu baseline 1 thread: decode {one['decode_tok_s']:.2f} prefill {one['prompt_tok_s']:.2f} tok/s")
        cb["one_thread"] = {"decode_tok_s": round(one["decode_tok_s"], 3), "prefill_tok_s": round(one["prompt_tok_s"], 3),
                            "sample": f"{P1} prompt + {G1} decode tokens"}
    return cb


def model_path(w, tag):
    need = 8.5e9 if w.wtype == "q8_0" and w.dim >= 4096 else 4.5e9
    d = "/dev/shm" if shutil.disk_usage("/dev/shm").free > 2 * need else tempfile.gettempdir()
    return os.path.join(d, f"qmh_bench_{tag}_{w.name}_{os.getpid()}.qlm")


def measure(q, w, P, K, W, detail=False):
    """Prefill, decode and the forward loop of one config; with detail, the c5a extras too."""
    import numpy as np

    path = model_path(w, "m")
    threads = min(len(os.sched_getaffinity(0)), CPU_SHARE)
    t0 = time.time()
    q.gen_model(path, w.config(), w.wtype, seed=w.seed, threads=threads)
    gen_s = time.time() - t0
    max_seq = min(P + max(K, W), w.max_seq)
    K = min(K, max_seq - P)
    out = {"workload": w.name, "prompt": P, "decode_steps": K, "max_seq": max_seq}
    try:
        t0 = time.time()
        m = q.Model.load(path, max_seq=max_seq)
        load_s = time.time() - t0
        prompt = q.prompt_ids(P, w.vocab_size)
        m.time_prefill(prompt[:4], 0, "last")  # warm the launch paths
        pf_all = statistics.median(m.time_prefill(prompt, 0, "all") for _ in range(3))
        pf_last = statistics.median(m.time_prefill(prompt, 0, "last") for _ in range(3))
        fwd = m.forward(int(prompt[-1]), P - 1)  # logits of the last prompt position
        tok0 = int(np.argmax(fwd))
        if W > 0:
            m.greedy(tok0, P, min(W, K))
        ids, dev_ms = m.time_greedy(tok0, P, K)
        value = K / (dev_ms / 1e3)
        fids, fwd_ms = m.time_forward(tok0, P, K)
        assert list(fids) == list(ids), "forward loop and device greedy loop disagree"
        bpt, wbytes = decode_bytes_per_token(w, list(range(P, P + K)))
        out.update({
            "decode_tok_s": round(value, 2), "ms_per_step": round(dev_ms / K, 4),
            "decode_bytes_per_token": int(bpt), "decode_hbm_frac": round(value * bpt / (HBM_PEAK_GBS * 1e9), 4),
            "decode_roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / bpt, 1),
            "forward_tok_s": round(K / (fwd_ms / 1e3), 2),
            "prefill_tok_s": round(P / (pf_all / 1e3), 2), "prefill_ms": round(pf_all, 3),
            "prefill_last_logits_tok_s": round(P / (pf_last / 1e3), 2),
            "greedy_ids_head": [int(x) for x in ids[:8]],
        })
        log(f"[bench] {w.name}: prefill {P} in {pf_all:.2f} ms (all logits) / {pf_last:.2f} ms (last), decode "
            f"{value:.1f} tok/s ({out['decode_hbm_frac']:.3f} of HBM), forward loop {out['forward_tok_s']:.1f} tok/s")
        if detail:
            flops = prefill_flops(w, P, P)
            ach = flops / (pf_all * 1e-3)
            valu_ms = prefill_valu_floor_s(w, P, P) * 1e3
            out["prefill_roofline"] = {
                "bound": "mfma", "unit": "TOP/s", "achieved": round(ach / 1e12, 2), "peak": INT8_PEAK_TOPS,
                "frac": round(ach / 1e12 / INT8_PEAK_TOPS, 4), "flops": int(flops),
                "valu_floor_ms": round(valu_ms, 3), "frac_of_valu_floor": round(valu_ms / pf_all, 4),
                "note": "int8 MFMA block dots and f16 MFMA scale products (both exact) + the bitwise f32 epilogue "
                        "on the VALU (3 ops per row, token, block), whose floor bounds this path more tightly than "
                        "the int8 peak; flops counted as the reference's P forwards, every position's logits "
                        "included",
            }
            # the same flops over the FP32-MFMA peak the north star names (above 1: the exact integer
            # dots run on int8 MFMA, so this is a comparison, not a roofline fraction)
            out["prefill_vs_fp32_mfma_peak"] = round(ach / 1e12 / FP32_MFMA_PEAK_TFS, 4)
            # the same steps sampled on the device with the reference CLI's default sampler
            # (src/main.c:70-72: temperature 0.8, top-k 0, top-p 0.95, seed 42); wall clock, synchronous
            with q.Sampler(w.vocab_size, 0.8, 0, 0.95, 42) as smp:
                m.sample(smp, tok0, P, min(W, 8))
                t0 = time.perf_counter()
                m.sample(smp, tok0, P, K)
                out["sampled_decode_tok_s"] = round(K / (time.perf_counter() - t0), 2)
            # batched decode of 4 and 16 independent sequences (qmh_batch_greedy): informational
            batched = []
            for BB in (4, 16):
                with q.Batch(m, BB) as bt:
                    bt.greedy([tok0] * BB, [P] * BB, 2)
                    _, b_ms = bt.greedy([tok0] * BB, [P] * BB, K)
                batched.append({"sequences": BB, "tok_s_aggregate": round(BB * K / (b_ms / 1e3), 1),
                                "ms_per_step": round(b_ms / K, 3)})
            out["batched_decode"] = batched
            stages = {}
            for st in ("qkv", "wo", "w13", "w2", "output", "attn", "attn_scores", "attn_pv"):
                try:
                    ms, nbytes = m.time_stage(st, 3 * w.n_layers, pos=P + K - 1)
                except q.QmhError:
                    continue  # a head shape or position the one-launch attention does not take
                stages[st] = {"us_per_launch": round(ms * 1e3, 3),
                              "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1) if nbytes else None,
                              "weight_MB": round(nbytes / 1e6, 3)}
            out["stages"] = stages
            ms_w13, bytes_w13 = m.time_stage("w13", 3 * w.n_layers, pos=P + K - 1)
            achieved = bytes_w13 / (ms_w13 * 1e-3) / 1e9
            out["roofline"] = {
                "kernel": "k_matvec<Q4_0> W1|W3 launch (64-row tiles: RMSNorm + W1|W3 + SwiGLU + W2's quantized input)",
                "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": pmc_traffic(f"k_matvec_w13_{w.wtype}_{w.name}_pmc.txt"),
                "bytes_per_launch": int(bytes_w13), "us_per_launch": round(ms_w13 * 1e3, 3)}
            out["setup_s"] = {"generate": round(gen_s, 1), "load": round(load_s, 1)}
            out["kernel_rows"] = kernel_rows(q)
        m.close()
    except BaseException:
        if os.path.exists(path):
            os.remove(path)
        raise
    return out, path


def probe_stream(q, w, grids=(256, 512, 1024), reps=20):
    """The device's read ceiling for the sizes of the decode step's weight streams (the separate probe
    library quillm_amd/libqmhprobe.so, so the token loop's code objects stay as timed): each size alone,
    launches back to back, every launch reading a fresh stretch of a 2 GiB pool (HBM, not the 256 MB
    Infinity Cache); and one layer's four matrices in order, 32 layers back to back."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(ROOT, "quillm_amd", "libqmhprobe.so"))
    lib.qmh_probe_reads.restype = ctypes.c_int
    lib.qmh_probe_reads.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64), ctypes.c_int,
                                    ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
    D, H, kvd = w.dim, w.hidden_dim, w.kvd
    rb = lambda n: row_bytes(w, n)
    mats = {"qkv": (D + 2 * kvd) * rb(D), "wo": D * rb(D), "w13": 2 * H * rb(D), "w2": D * rb(H),
            "output": w.vocab_size * rb(D), "1GiB": 1 << 30}
    pool_bytes = 2 << 30
    pool = q.DeviceBuffer(pool_bytes)
    q._check(q.load_library().qmh_memset(pool.ptr, 1, pool_bytes), "probe fill")
    q.sync()
    out = {"probe": "stream", "kernel": "k_read (16-byte loads, 4 in flight per lane, 256-thread workgroups)",
           "pool_bytes": pool_bytes, "reps": reps, "single": {}}
    for name, nbytes in mats.items():
        n16 = (nbytes + 15) // 16 * 16
        arr = (ctypes.c_uint64 * 1)(n16)
        per = {}
        for g in grids:
            us = (ctypes.c_double * 1)()
            rc = lib.qmh_probe_reads(ctypes.c_void_p(pool.ptr), pool_bytes, arr, 1, reps, g, 0, us)
            if rc:
                raise RuntimeError(f"qmh_probe_reads: {rc}")
            per[str(g)] = round(us[0], 2)
        best = min(per.values())
        out["single"][name] = {"bytes": n16, "us_by_grid": per, "best_us": best,
                               "best_GBps": round(n16 / (best * 1e-6) / 1e9, 1)}
        log(f"[bench] probe stream {name}: {n16 / 1e6:.2f} MB, best {best:.2f} us ({out['single'][name]['best_GBps']} GB/s)")
    seq = [mats[k] for k in ("qkv", "wo", "w13", "w2")]
    arr = (ctypes.c_uint64 * 4)(*[(n + 15) // 16 * 16 for n in seq])
    us = (ctypes.c_double * 1)()
    rc = lib.qmh_probe_reads(ctypes.c_void_p(pool.ptr), pool_bytes, arr, 4, w.n_layers, 512, 1, us)
    if rc:
        raise RuntimeError(f"qmh_probe_reads: {rc}")
    out["layer_sequence"] = {"matrices": ["qkv", "wo", "w13", "w2"], "grid": 512, "layers": w.n_layers,
                             "bytes": int(sum(arr)), "us_per_layer": round(us[0], 2),
                             "GBps": round(sum(arr) / (us[0] * 1e-6) / 1e9, 1)}
    del pool
    return out


def kernel_rows(q, n=4096, gemm_n=512):
    """The reference bench's kernel rows (bench/bench.c:63-123; README.md:163-173) on the device:
    qmh_matvec at n x n for q8_0, q4_0 and f32 weights, and qmh_matmul_nt at gemm_n^3. Device time per
    call from HIP events over back-to-back calls. 'hbm': calls cycle through copies of the matrix
    whose total exceeds the 256 MB Infinity Cache, so the weights come from HBM; 'cached': one matrix
    over and over (the reference bench's own loop). GFLOP/s counts 2*rows*cols per matvec as the
    reference does (README.md:161)."""
    import ctypes

    import numpy as np

    L = q.load_library()
    rs = np.random.default_rng(5)
    x = q.DeviceBuffer.from_array(rs.standard_normal(n).astype(np.float32))
    y = q.DeviceBuffer(4 * n)
    out = {}
    for name, dtype, bb in (("q8_0", 2, 34), ("q4_0", 3, 18), ("f32", 0, None)):
        if bb is None:
            host = rs.standard_normal((n, n)).astype(np.float32) * 0.02
            row_b = 4 * n
        else:
            nb = (n + 31) // 32
            blocks = rs.integers(0, 256, (n, nb, bb), dtype=np.uint8)
            scale = np.float16(0.01).view(np.uint16)
            blocks[:, :, 0], blocks[:, :, 1] = scale & 0xff, scale >> 8
            host = blocks.reshape(n, nb * bb)
            row_b = nb * bb
        mbytes = n * row_b
        copies = max(1, -(-300_000_000 // mbytes))  # past the Infinity Cache
        ws = []
        try:
            for _ in range(copies):
                h = L.qmh_weight_upload(dtype, n, n, np.ascontiguousarray(host).ctypes.data)
                if not h:
                    raise q.QmhError(f"qmh_weight_upload: {q.last_error()}")
                ws.append(h)
            row = {"bytes": mbytes}
            for tag, nw in (("hbm", copies), ("cached", 1)):
                arr = (ctypes.c_void_p * nw)(*ws[:nw])
                ms = ctypes.c_double()
                iters = max(3 * copies, 24)
                q._check(L.qmh_time_matvec(arr, nw, x.ptr, y.ptr, iters, ctypes.byref(ms)), "time_matvec")  # warm
                q._check(L.qmh_time_matvec(arr, nw, x.ptr, y.ptr, iters, ctypes.byref(ms)), "time_matvec")
                us = ms.value * 1e3
                row[tag] = {"us_per_call": round(us, 3), "GBps": round(mbytes / (us * 1e-6) / 1e9, 1),
                            "frac_of_hbm_peak": round(mbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                            "GFLOPs": round(2.0 * n * n / (us * 1e-6) / 1e9, 1)}
            out[f"matvec_{name}_{n}x{n}"] = row
        finally:
            for h in ws:
                L.qmh_weight_free(h)
    M = gemm_n
    A = q.DeviceBuffer.from_array(rs.standard_normal((M, M)).astype(np.float32))
    B = q.DeviceBuffer.from_array(rs.standard_normal((M, M)).astype(np.float32))
    C = q.DeviceBuffer(4 * M * M)
    ms = ctypes.c_double()
    q._check(L.qmh_time_matmul_nt(A.ptr, B.ptr, C.ptr, M, M, M, 5, ctypes.byref(ms)), "time_matmul_nt")
    q._check(L.qmh_time_matmul_nt(A.ptr, B.ptr, C.ptr, M, M, M, 20, ctypes.byref(ms)), "time_matmul_nt")
    flops = 2.0 * M * M * M
    out[f"matmul_nt_f32_{M}^3"] = {
        "us_per_call": round(ms.value * 1e3, 3), "GFLOPs": round(flops / (ms.value * 1e-3) / 1e9, 1),
        "frac_of_valu_floor": round(flops / (ms.value * 1e-3) / VALU_LANE_OPS, 4),
        "note": "the scalar ISA's rounding order (K panels of 256, one serial sum per output per panel): a "
                "multiply and an add per term on the fp32 VALU, so the floor is 2*M*N*K lane operations"}
    return out


def probe_stages(q, w, pos):
    """Stage times of the decode step at position pos (HIP events over 3 x n_layers launches cycling the
    layers), for counter runs of single kernels at a chosen context length."""
    path = model_path(w, "p")
    try:
        q.gen_model(path, w.config(), w.wtype, seed=w.seed, threads=min(len(os.sched_getaffinity(0)), CPU_SHARE))
        out = {"probe": "stages", "workload": w.name, "pos": pos, "stages": {}}
        with q.Model.load(path, max_seq=pos + 1) as m:
            for st in ("qkv", "wo", "w13", "w2", "output", "attn_scores", "attn_pv"):
                ms, nbytes = m.time_stage(st, 3 * w.n_layers, pos=pos)
                out["stages"][st] = round(ms * 1e3, 3)
    finally:
        if os.path.exists(path):
            os.remove(path)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed decode steps (default: the config's 128)")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", default="c5a")
    ap.add_argument("--prefill", type=int, default=None, help="prompt length (default: the config's 512)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the other BASELINE configs")
    ap.add_argument("--probe-stream", action="store_true",
                    help="print the device's read ceiling for the decode step's weight sizes and exit")
    ap.add_argument("--probe-stages", type=int, default=None, metavar="POS",
                    help="print the decode stages' times at position POS and exit")
    ap.add_argument("--probe-copy", action="store_true",
                    help="first run a known-size streaming kernel (fp16->fp32 of 64 Mi halves: 128 MiB read, "
                         "256 MiB written) whose FETCH_SIZE/WRITE_SIZE readings calibrate the counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported by this build "
              "(the token loop runs on one MI355X; multi-GPU sharding is a design note, not a run)", file=sys.stderr)
        sys.exit(2)

    import quillm_amd as q

    w = q.WORKLOADS[args.workload]
    P = args.prefill if args.prefill is not None else w.n_prompt
    K = args.steps if args.steps is not None else w.n_gen
    W = args.warmup
    if not q.available():
        raise SystemExit("no gfx950 device visible")
    q.init(0)
    if args.probe_copy:
        n = 64 << 20
        src, dst = q.DeviceBuffer(2 * n), q.DeviceBuffer(4 * n)
        q._check(q.load_library().qmh_memset(src.ptr, 0x3c, 2 * n), "probe fill")
        for _ in range(3):
            q._check(q.load_library().qmh_fp16_to_fp32(src.ptr, dst.ptr, n, None), "probe copy")
        q.sync()
        del src, dst
        log(f"[bench] probe copy: 3 x k_h2f over {n} halves")
    if args.probe_stream:
        print(json.dumps(probe_stream(q, w)), flush=True)
        return
    if args.probe_stages is not None:
        print(json.dumps(probe_stages(q, w, args.probe_stages)), flush=True)
        return

    head, path = measure(q, w, P, K, W, detail=True)
    out = {
        "metric": "decode tok/s + % HBM roofline, 7B-shape Q4_0 bs=1; prefill tok/s @512",
        "value": head["decode_tok_s"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": head["decode_steps"],
        "warmup": W,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 x q8_0 int8 dot, f32 accumulate" if w.wtype == "q4_0" else "q8_0 x q8_0 int8 dot, f32 accumulate",
        "data": "synthetic: random-init N(0,0.02) weights (seed 1), random prompt ids (seed 1234)",
        "config": {"workload": f"{w.name}: 7B-shape Llama {w.wtype} dim {w.dim} hidden {w.hidden_dim} "
                               f"{w.n_layers} layers {w.n_heads}/{w.n_kv_heads} heads vocab {w.vocab_size}, "
                               f"batch 1, prompt {P}, decode {head['decode_steps']} greedy",
                   "prompt": P, "decode_steps": head["decode_steps"], "max_seq": head["max_seq"]},
    }
    for k in ("prefill_tok_s", "prefill_last_logits_tok_s", "prefill_ms", "prefill_roofline", "forward_tok_s",
              "sampled_decode_tok_s", "batched_decode", "decode_bytes_per_token", "decode_hbm_frac",
              "decode_roofline_tok_s", "roofline", "stages", "kernel_rows", "prefill_vs_fp32_mfma_peak",
              "greedy_ids_head", "setup_s"):
        out[k] = head[k]
    out["timing"] = ("decode: HIP events around K graph replays (device argmax, no host round trip); forward_tok_s: "
                     "host clock around K qmh_model_forward calls with the logits copied to the host and a host "
                     "argmax (the reference bench's loop, bench/bench.c:143-149); prefill: HIP events around the "
                     "batched prefill, median of 3, every position's logits computed on the device (the work of the "
                     "reference's prompt loop) or only the last one's")
    try:
        if not args.no_cpu:
            log(f"[bench] cpu baseline: reference on {w.name}")
            cb = cpu_baseline(path, w, q, P, w.n_gen)
            if cb is not None:
                out["cpu_baseline"] = cb
    finally:
        os.remove(path)
    if not args.no_configs:
        others = {}
        for name in ("c1", "c2", "c3", "c4", "c5a", "c5b"):
            if name == w.name:
                continue
            wc = q.WORKLOADS[name]
            r, p = measure(q, wc, wc.n_prompt, wc.n_gen, W)
            try:
                if not args.no_cpu:
                    # the reference on the config's whole workload, one run (the file is in /dev/shm)
                    cb = cpu_baseline(p, wc, q, wc.n_prompt, wc.n_gen, runs=1, warm=False, one_thread=False)
                    if cb is not None:
                        r["cpu_reference"] = {"decode_tok_s": cb["value"], "prefill_tok_s": cb["prefill_tok_s"],
                                              "threads": cb["cores"], "isa": cb["isa"],
                                              "sample": f"{wc.n_prompt} prompt + {wc.n_gen} greedy, one run"}
            finally:
                os.remove(p)
            others[name] = {k: v for k, v in r.items() if k != "workload"}
        out["configs"] = others
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
