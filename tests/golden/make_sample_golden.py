"""Writes tests/golden/sample_27b.json: the CPU oracle's sampled decode of the synthetic
Bonsai-27B-shape model (BASELINE config 4 shape) with the reference's default sampling
(T 0.7, top-k 20, top-p 0.95; Daiza-engine/src/math/sampling.rs:39 and 144-247).

The oracle (oracle/, a C restatement of the reference's AVX2 path) runs the prompt's first n - 1 ids
through forward_single_token (forward.rs:204-375); then, from the prompt's last id, each step forwards
the current id and draws the next with sample_top_k_top_p_into and one LcgRng (sampling.rs:9-19), as
the decode loop of engine.rs:850-862 does.  Stored per step: the drawn id, the uniform draw r, the
smallest distance between r and a cumulative probability of the renormalised top-p set (in float64),
and the gap between the k-th and (k+1)-th logit, so that a GPU mismatch can be told apart from a
draw that lands next to a boundary.  The final generator state is stored too.

Usage: python tests/golden/make_sample_golden.py [--prefill 64] [--decode 48] [--threads N]
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
TEMP, TOP_K, TOP_P = 0.7, 20, 0.95
RNG_SEED = 0xC0FFEE


def diagnostics(logits, state):
    """The draw's uniform r and its distance to the nearest cumulative boundary, in float64."""
    s = (state * 6364136223846793005 + 1442695040888963407) & ((1 << 64) - 1)
    r = ((s >> 40) & 0xFFFFFF) / float(1 << 24)
    order = np.argsort(-logits, kind="stable")
    top = logits[order[:TOP_K]].astype(np.float64) / TEMP
    p = np.exp(top - top[0])
    p /= p.sum()
    cum = np.cumsum(p)
    cut = int(np.argmax(cum >= TOP_P)) + 1 if (cum >= TOP_P).any() else TOP_K
    q = p[:cut] / p[:cut].sum()
    return r, float(np.min(np.abs(np.cumsum(q) - r))), float(logits[order[TOP_K - 1]] - logits[order[TOP_K]])


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--prefill", type=int, default=64)
    ap.add_argument("--decode", type=int, default=48)
    ap.add_argument("--threads", type=int, default=0)
    ap.add_argument("--out", default=os.path.join(os.path.dirname(os.path.abspath(__file__)), "sample_27b.json"))
    a = ap.parse_args()
    import oracle
    import daiza_amd as dz  # Config only (no library call)
    cfg = dz.Config.bonsai27b(max_ctx=a.prefill + a.decode + 8)
    t0 = time.time()
    om = oracle.Model(cfg, SEED, nthreads=a.threads)
    print("model %.1f s" % (time.time() - t0), flush=True)
    prompt = np.random.default_rng(PROMPT_SEED).integers(0, cfg.vocab, a.prefill).astype(np.uint32)
    t0 = time.time()
    for t in prompt[:-1]:
        om.forward(int(t), want_logits=False)
    print("prefill %.1f s" % (time.time() - t0), flush=True)
    rng = oracle.Rng(RNG_SEED)
    tok = int(prompt[-1])
    steps = []
    for i in range(a.decode):
        _, logits = om.forward(tok, want_logits=True)
        r, dist, gap = diagnostics(logits, rng.state.value)
        tok = int(oracle.sample_top_k_top_p(logits, TEMP, TOP_K, TOP_P, rng))
        steps.append({"token": tok, "r": r, "boundary_distance": dist, "kth_gap": gap})
        if i % 16 == 0:
            print("decode %d/%d %.1f s" % (i, a.decode, time.time() - t0), flush=True)
    om.close()
    out = {
        "what": "CPU-oracle sampled decode, synthetic Bonsai-27B shape (daiza_synth.h)",
        "seed": SEED,
        "prompt": {"generator": "numpy default_rng(%d).integers(0, vocab, n)" % PROMPT_SEED, "n": a.prefill},
        "sampling": {"temperature": TEMP, "top_k": TOP_K, "top_p": TOP_P, "rng_seed": RNG_SEED},
        "decode": a.decode,
        "tokens": [s["token"] for s in steps],
        "final_rng_state": rng.state.value,
        "steps": steps,
    }
    with open(a.out, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print("wrote %s (%.1f s)" % (a.out, time.time() - t0), flush=True)


if __name__ == "__main__":
    main()
