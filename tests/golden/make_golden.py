#!/usr/bin/env python3
"""Writes the whole-model golden fixtures for the BASELINE configs -- TEST INFRASTRUCTURE.

For each config: generate the synthetic .qlm with the library's seeded generator, run the
compiled reference (oracle/_ref/ref_driver, built from the reference's src/ by
oracle/Makefile) on the scalar ISA over the config's prompt and greedy decode, and record

  * xxh64 of the generated .qlm file (pins the generator on the machine that replays it),
  * the prompt ids and the greedy ids (tokens[0] = argmax after the last prompt position,
    tokens[k] = argmax after the forward at position P+k-1 fed tokens[k-1]),
  * xxh64 of the float32 logits bytes at every position (P prompt + G decode positions),
  * the top-5 (id, logit) of the last position, for diagnosis when a hash differs.

The scalar ISA is the reference's bit-exact order (serial float sums, no FMA) that the
device path reproduces; the AVX-512 kernels sum in another order and pick different greedy
ids on random weights within a few steps. Run here, where the reference sources are:

  python tests/golden/make_golden.py [--configs c3,c4,c5a,c5b] [--threads 7]

Every config is recorded at its full prompt and decode length. c5b (7.2 GB of Q8_0 weights)
takes the longest: the scalar reference runs at about 0.3 tok/s on it here (~40 min).
"""
import argparse
import json
import os
import sys
import time

import numpy as np
import xxhash

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

SHORT: dict = {}


def file_xxh64(path: str) -> str:
    h = xxhash.xxh64()
    with open(path, "rb") as f:
        while True:
            b = f.read(1 << 24)
            if not b:
                break
            h.update(b)
    return h.hexdigest()


def row_hashes(logits: np.ndarray) -> list:
    return [xxhash.xxh64(np.ascontiguousarray(r).tobytes()).hexdigest() for r in logits]


def main():
    import quillm_amd as q
    from _bind import ref_run

    ap = argparse.ArgumentParser()
    ap.add_argument("--configs", default="c1,c2,c3,c4,c5a,c5b")
    ap.add_argument("--threads", type=int, default=7)
    ap.add_argument("--dir", default="/dev/shm")
    args = ap.parse_args()
    for name in args.configs.split(","):
        w = q.WORKLOADS[name]
        P, G = SHORT.get(name, (w.n_prompt, w.n_gen))
        path = os.path.join(args.dir, f"golden_{name}.qlm")
        t0 = time.time()
        q.gen_model(path, w.config(), w.wtype, seed=w.seed, threads=args.threads)
        fh = file_xxh64(path)
        prompt = q.prompt_ids(P, w.vocab_size)
        print(f"[golden] {name}: generated in {time.time() - t0:.1f}s, reference {P}+{G} ...", flush=True)
        t0 = time.time()
        res, lg = ref_run(path, prompt, G, isa="scalar", threads=args.threads, max_seq=P + G, timeout=1e5)
        lg = lg.reshape(P + G, w.vocab_size)
        top = np.argsort(-lg[-1], kind="stable")[:5]
        out = {
            "config": name, "wtype": w.wtype, "seed": w.seed, "prompt_seed": 1234,
            "dims": [w.dim, w.hidden_dim, w.n_layers, w.n_heads, w.n_kv_heads, w.vocab_size, w.max_seq],
            "n_prompt": P, "n_gen": G, "max_seq": P + G,
            "reference": {"driver": "oracle/_ref/ref_driver", "isa": res["isa"], "threads": args.threads},
            "qlm_xxh64": fh,
            "prompt": [int(t) for t in prompt],
            "tokens": [int(t) for t in res["tokens"]],
            "logits_xxh64": row_hashes(lg),
            "last_top5": [[int(i), float(lg[-1, i])] for i in top],
        }
        with open(os.path.join(HERE, f"{name}_scalar.json"), "w") as f:
            json.dump(out, f, indent=0)
            f.write("\n")
        os.remove(path)
        print(f"[golden] {name}: {time.time() - t0:.1f}s, tokens {out['tokens'][:8]}...", flush=True)


if __name__ == "__main__":
    main()
