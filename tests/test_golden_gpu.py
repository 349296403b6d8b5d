"""Full-size greedy decode against the committed CPU-oracle golden.

tests/golden/greedy_27b.json holds the oracle's greedy continuation of the synthetic
Bonsai-27B-shape model after a 1024-token uniform-random prompt (tests/golden/make_greedy_golden.py).
The GPU runs the same prompt through dz_forward_batch and decodes greedily on the device; the
bar is token identity for every stored step, and the first step's top logits within 1e-3.
"""
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "greedy_27b.json")


@pytest.fixture(scope="module")
def golden():
    with open(GOLDEN) as f:
        return json.load(f)


def test_greedy_27b_matches_oracle(dz, golden):
    g = golden
    n_prompt, n_dec = g["prompt"]["n"], g["decode"]
    cfg = dz.Config.bonsai27b(max_ctx=n_prompt + n_dec + 8)
    prompt = np.random.default_rng(4).integers(0, cfg.vocab, n_prompt).astype(np.uint32)
    print("golden: seed %#x, prompt %d, decode %d" % (g["seed"], n_prompt, n_dec), flush=True)
    model = dz.Model.synthetic(cfg, g["seed"])
    ctx = dz.Context(model)
    try:
        last = ctx.forward_batch(prompt)
        top = g["steps"][0]["top"]
        want = np.array([v for _, v in top], np.float64)
        got = last[[i for i, _ in top]].astype(np.float64)
        assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 1e-3
        first = int(np.argmax(last))
        toks = [first] + list(ctx.decode_greedy(first, n_dec - 1))
        ref = g["tokens"]
        mism = [i for i in range(n_dec) if toks[i] != ref[i]]
        if mism:
            i = mism[0]
            pytest.fail("first mismatch at decode step %d: gpu %d, oracle %d (oracle top1-top2 margin %.3g)"
                        % (i, toks[i], ref[i], g["steps"][i]["margin"]))
    finally:
        ctx.close()
        model.close()


GOLDEN_SAMPLE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "sample_27b.json")


def test_sampled_27b_matches_oracle(dz):
    """The in-kernel sampled decode (dz_decode_sample, T 0.7, top-k 20, top-p 0.95) against the CPU
    oracle's sampled loop on the full 27B shape (tests/golden/make_sample_golden.py): the generator
    state after the run exactly, and every drawn id up to the first step whose draw lies within 1e-4
    of a cumulative-probability boundary (such a draw is not fixed by logits that agree to 1e-4; the
    golden's steps 0-44 are all farther from one)."""
    with open(GOLDEN_SAMPLE) as f:
        g = json.load(f)
    n_prompt, n_dec, sp = g["prompt"]["n"], g["decode"], g["sampling"]
    cfg = dz.Config.bonsai27b(max_ctx=n_prompt + n_dec + 8)
    prompt = np.random.default_rng(4).integers(0, cfg.vocab, n_prompt).astype(np.uint32)
    model = dz.Model.synthetic(cfg, g["seed"])
    ctx = dz.Context(model)
    try:
        assert ctx.token_kernel
        ctx.forward_batch(prompt[:-1])
        rng = dz.LcgRng(sp["rng_seed"])
        got = [int(t) for t in ctx.decode_sample(int(prompt[-1]), n_dec,
                                                 dz.SamplingParams(sp["temperature"], sp["top_k"], sp["top_p"]), rng)]
        assert rng.state.value == g["final_rng_state"]
        lim = next((i for i, s in enumerate(g["steps"]) if s["boundary_distance"] < 1e-4), n_dec)
        assert lim >= 40
        mism = [i for i in range(lim) if got[i] != g["tokens"][i]]
        if mism:
            i = mism[0]
            pytest.fail("first mismatch at step %d: gpu %d, oracle %d (draw %.6f, %.3g from a boundary)"
                        % (i, got[i], g["tokens"][i], g["steps"][i]["r"], g["steps"][i]["boundary_distance"]))
        print("identical through step %d of %d; all %d: %s" % (lim, n_dec, n_dec, got == g["tokens"]), flush=True)
    finally:
        ctx.close()
        model.close()
