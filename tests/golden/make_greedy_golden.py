"""Writes tests/golden/greedy_27b.json: the CPU oracle's greedy decode of the synthetic
Bonsai-27B-shape model -- a prefill of uniform-random ids, then greedy tokens.

The oracle (oracle/, a C restatement of the reference's AVX2 path) runs every position through
forward_single_token (forward.rs:204-375); greedy = argmax with the lowest index on ties
(simd_exp.rs:551-598).  Stored per decode step: the token, the top-1 minus top-2 logit margin
and the top-8 (index, logit) pairs, so a GPU mismatch can be told apart from a near tie.

Usage: python tests/golden/make_greedy_golden.py [--prefill 1024] [--decode 256] [--threads N]
Takes several minutes on 8 cores (about 3.6 GB of weights per token).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

SEED = 0xDA1A0004
PROMPT_SEED = 4


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--prefill", type=int, default=1024)
    ap.add_argument("--decode", type=int, default=256)
    ap.add_argument("--threads", type=int, default=0)
    ap.add_argument("--out", default=os.path.join(os.path.dirname(os.path.abspath(__file__)), "greedy_27b.json"))
    a = ap.parse_args()
    import oracle
    import daiza_amd as dz  # Config only (no library call)
    cfg = dz.Config.bonsai27b(max_ctx=a.prefill + a.decode + 8)
    t0 = time.time()
    om = oracle.Model(cfg, SEED, nthreads=a.threads)
    print("model %.1f s" % (time.time() - t0), flush=True)
    prompt = np.random.default_rng(PROMPT_SEED).integers(0, cfg.vocab, a.prefill).astype(np.uint32)
    t0 = time.time()
    tok = None
    for i, t in enumerate(prompt):
        last = i == len(prompt) - 1
        tok, logits = om.forward(int(t), want_logits=last)
        if i % 128 == 0:
            print("prefill %d/%d %.1f s" % (i, len(prompt), time.time() - t0), flush=True)
    steps = []
    for i in range(a.decode):
        order = np.argsort(-logits, kind="stable")[:8]
        steps.append({"token": int(tok), "margin": float(logits[order[0]] - logits[order[1]]),
                      "top": [[int(j), float(logits[j])] for j in order]})
        tok, logits = om.forward(int(tok), want_logits=True)
        if i % 32 == 0:
            print("decode %d/%d %.1f s" % (i, a.decode, time.time() - t0), flush=True)
    om.close()
    out = {
        "what": "CPU-oracle greedy decode, synthetic Bonsai-27B shape (daiza_synth.h)",
        "seed": SEED,
        "prompt": {"generator": "numpy default_rng(%d).integers(0, vocab, n)" % PROMPT_SEED, "n": a.prefill},
        "decode": a.decode,
        "tokens": [s["token"] for s in steps],
        "steps": steps,
    }
    with open(a.out, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print("wrote %s (%.1f s)" % (a.out, time.time() - t0), flush=True)


if __name__ == "__main__":
    main()
