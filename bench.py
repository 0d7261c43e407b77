#!/usr/bin/env python3
"""Decode/prefill benchmark of the quillm token loop on one MI355X.

Workload (BASELINE.json metric): config c5a, a 7B-shaped Llama in Q4_0 (dim 4096, hidden 11008,
32 layers, 32/32 heads, vocab 32000), random-init N(0,0.02) weights from a fixed seed, batch 1:
a 512-token random-id prompt, then greedy decode. One "step" is one decode token (a full
forward + argmax, replayed as one hipGraph, inputs resident in HBM); W untimed warmup steps,
then exactly K timed steps at positions P..P+K-1.

Prints one JSON line: decode tok/s (value), prefill tok/s, fraction of the HBM roofline,
`roofline` for the dominant kernel (the fused RMSNorm + W1|W3 Q4_0 matvec + SwiGLU), and
`cpu_baseline` = the compiled reference (best CPU ISA, all host cores) on a bounded sample.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c5a] [--no-cpu]
"""
import argparse
import json
import os
import shutil
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def decode_bytes_per_token(w, positions):
    """Algorithmic HBM bytes of one decode token, averaged over `positions`: every weight
    stream + K and V reads up to pos + KV writes + norm gains + logits + one embedding row."""
    D, H, L, V, kvd = w.dim, w.hidden_dim, w.n_layers, w.vocab_size, w.kvd
    bb = 18 if w.wtype == "q4_0" else 34 if w.wtype == "q8_0" else None
    nb = lambda n: (n + 31) // 32
    rb = (lambda n: nb(n) * bb) if bb else (lambda n: 4 * n)
    weights = L * ((D + 2 * kvd) * rb(D) + D * rb(D) + 2 * H * rb(D) + D * rb(H)) + V * rb(D)
    kv_read = sum(2 * L * (p + 1) * kvd * 4 for p in positions) / len(positions)
    small = 2 * L * kvd * 4 + (2 * L + 1) * D * 4 + V * 4 + rb(D)
    return weights + kv_read + small, weights


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


def cpu_baseline(path, w, threads, n_prompt, n_gen, q):
    """The compiled reference (oracle/_ref/ref_driver) on a bounded sample of the workload."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from _bind import REF_DRIVER, ref_run

    if not os.path.exists(REF_DRIVER):
        return None
    flags = open("/proc/cpuinfo").read()
    isa = "avx512" if (" avx512f " in flags and " avx512bw " in flags and " avx512vl " in flags) else "avx2"
    prompt = q.prompt_ids(n_prompt, w.vocab_size)
    res, _ = ref_run(path, prompt, n_gen, isa=isa, threads=threads, max_seq=n_prompt + n_gen, logits=False,
                     warm=True, timeout=600)
    return {
        "value": round(res["decode_tok_s"], 3), "unit": "tok/s", "cores": threads, "kind": "reference",
        "isa": res["isa"], "prefill_tok_s": round(res["prompt_tok_s"], 3),
        "sample": f"same {w.name} .qlm file; {n_prompt} prompt tokens (sequential qm_model_forward) + {n_gen} "
                  f"greedy decode steps, max_seq {n_prompt + n_gen}, QUILLM isa {res['isa']}, {threads} threads",
        "tokens": res["tokens"],
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed decode steps (default: the config's 128)")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", default="c5a")
    ap.add_argument("--prefill", type=int, default=None, help="prompt length (default: the config's 512)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-prompt", type=int, default=None, help="CPU sample prompt (default: the same P)")
    ap.add_argument("--cpu-gen", type=int, default=None, help="CPU sample decode steps (default: the same K)")
    ap.add_argument("--model-dir", default=None)
    ap.add_argument("--probe-copy", action="store_true",
                    help="first run a known-size streaming kernel (fp16->fp32 of 64 Mi halves: 128 MiB read, "
                         "256 MiB written) whose FETCH_SIZE/WRITE_SIZE readings calibrate the counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported by this build "
              "(the token loop runs on one MI355X; multi-GPU sharding is a design note, not a run)", file=sys.stderr)
        sys.exit(2)

    import numpy as np

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

    # synthetic model file (generated on this host: it does not travel)
    need = 8.5e9 if w.wtype == "q8_0" else 4.5e9
    d = args.model_dir
    if d is None:
        d = "/dev/shm" if shutil.disk_usage("/dev/shm").free > 2 * need else tempfile.gettempdir()
    path = os.path.join(d, f"qmh_bench_{w.name}_{os.getpid()}.qlm")
    threads = min(os.cpu_count() or 1, 16)
    t0 = time.time()
    q.gen_model(path, w.config(), w.wtype, seed=w.seed, threads=threads)
    gen_s = time.time() - t0
    log(f"[bench] generated {w.name} ({os.path.getsize(path) / 1e9:.2f} GB) in {gen_s:.1f}s")
    try:
        max_seq = P + max(K, W)
        t0 = time.time()
        m = q.Model.load(path, max_seq=max_seq)
        load_s = time.time() - t0
        log(f"[bench] loaded to device in {load_s:.1f}s (max_seq {max_seq})")
        prompt = q.prompt_ids(P, w.vocab_size)

        # prefill: P tokens at positions 0..P-1 (warm the graph first)
        m.prefill(prompt[:4], 0)
        q.sync()
        t0 = time.perf_counter()
        last = m.prefill(prompt, 0, want_logits=False)
        q.sync()
        prefill_s = time.perf_counter() - t0
        fwd = m.forward(int(prompt[-1]), P - 1)  # logits of the last prompt position
        tok0 = int(np.argmax(fwd))
        del last
        log(f"[bench] prefill {P} tok in {prefill_s * 1e3:.1f} ms")

        # decode: W warmup steps, then K timed steps from the same start (positions P..P+K-1)
        if W > 0:
            m.greedy(tok0, P, W)
        q.sync()
        t0 = time.perf_counter()
        ids, dev_ms = m.time_greedy(tok0, P, K)
        q.sync()
        wall_s = time.perf_counter() - t0
        ms_per_step = dev_ms / K
        value = K / (dev_ms / 1e3)
        log(f"[bench] decode {K} steps: {dev_ms:.2f} ms device ({wall_s * 1e3:.2f} ms wall), {value:.1f} tok/s")

        # the same steps sampled on the device with the reference CLI's default sampler
        # (src/main.c:70-72: temperature 0.8, top-k 0, top-p 0.95, seed 42); wall clock, synchronous
        with q.Sampler(w.vocab_size, 0.8, 0, 0.95, 42) as smp:
            m.sample(smp, tok0, P, min(W, 8))
            t0 = time.perf_counter()
            m.sample(smp, tok0, P, K)
            sampled_s = time.perf_counter() - t0
        log(f"[bench] sampled decode {K} steps: {sampled_s * 1e3:.2f} ms wall, {K / sampled_s:.1f} tok/s")

        # batched decode of 4 and 16 independent sequences (qmh_batch_greedy) over the same positions:
        # informational, the metric stays batch 1
        batched = []
        for BB in (4, 16):
            with q.Batch(m, BB) as bt:
                bt.greedy([tok0] * BB, [P] * BB, 2)
                _, b_ms = bt.greedy([tok0] * BB, [P] * BB, K)
            batched.append({"sequences": BB, "tok_s_aggregate": round(BB * K / (b_ms / 1e3), 1),
                            "ms_per_step": round(b_ms / K, 3)})
            log(f"[bench] batched decode B={BB}: {b_ms / K:.3f} ms per step, "
                f"{BB * K / (b_ms / 1e3):.1f} tok/s aggregate")

        # dominant kernel: fused RMSNorm + W1|W3 matvec + SwiGLU, cycling the layers
        stages = {}
        for st in ("qkv", "wo", "w13", "w2", "output", "attn_scores", "attn_pv"):
            ms, nbytes = m.time_stage(st, 3 * w.n_layers, pos=P + K - 1)
            stages[st] = {"us_per_launch": round(ms * 1e3, 3),
                          "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1) if nbytes else None,
                          "weight_MB": round(nbytes / 1e6, 3)}
        ms_w13, bytes_w13 = m.time_stage("w13", 3 * w.n_layers, pos=P + K - 1)
        achieved = bytes_w13 / (ms_w13 * 1e-3) / 1e9
        m.close()
    finally:
        pass

    positions = list(range(P, P + K))
    bpt, wbytes = decode_bytes_per_token(w, positions)
    out = {
        "metric": "decode tok/s + % HBM roofline, 7B-shape Q4_0 bs=1; prefill tok/s @512",
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 x q8_0 int8 dot, f32 accumulate" if w.wtype == "q4_0" else "q8_0 x q8_0 int8 dot, f32 accumulate",
        "data": "synthetic: random-init N(0,0.02) weights (seed 1), random prompt ids (seed 1234)",
        "config": {"workload": f"{w.name}: 7B-shape Llama {w.wtype} dim {w.dim} hidden {w.hidden_dim} "
                               f"{w.n_layers} layers {w.n_heads}/{w.n_kv_heads} heads vocab {w.vocab_size}, "
                               f"batch 1, prompt {P}, decode {K} greedy",
                   "prompt": P, "decode_steps": K, "max_seq": P + max(K, W)},
        "prefill_tok_s": round(P / prefill_s, 2),
        "sampled_decode_tok_s": round(K / sampled_s, 2),
        "batched_decode": batched,
        "decode_bytes_per_token": int(bpt),
        "decode_hbm_frac": round(value * bpt / (HBM_PEAK_GBS * 1e9), 4),
        "decode_roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / bpt, 1),
        "roofline": {"kernel": "k_matvec<Q4_0> W1|W3 launch (64-row tiles: RMSNorm + W1|W3 + SwiGLU + W2's quantized input)",
                     "bound": "hbm",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": pmc_traffic(f"k_matvec_w13_{w.wtype}_{w.name}_pmc.txt") if w.name in ("c5a", "c5b") else None,
                     "bytes_per_launch": int(bytes_w13), "us_per_launch": round(ms_w13 * 1e3, 3)},
        "stages": stages,
        "greedy_ids_head": [int(x) for x in ids[:8]],
        "setup_s": {"generate": round(gen_s, 1), "load": round(load_s, 1)},
    }
    if not args.no_cpu:
        cpu_threads = min(os.cpu_count() or 1, 16)
        cp = P if args.cpu_prompt is None else args.cpu_prompt
        cg = K if args.cpu_gen is None else args.cpu_gen
        log(f"[bench] cpu baseline: reference, {cpu_threads} threads, {cp}+{cg} tokens")
        cb = cpu_baseline(path, w, cpu_threads, cp, cg, q)
        if cb is not None:
            out["cpu_baseline"] = {k: v for k, v in cb.items() if k != "tokens"}
    try:
        os.remove(path)
    except OSError:
        pass
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
