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
