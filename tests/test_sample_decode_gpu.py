"""dz_decode_sample: the sampled decode loop of Engine::generate_inner (engine.rs:850-862) with
sample_top_k_top_p_into (Daiza-engine/src/math/sampling.rs:144-247) and its LcgRng
(sampling.rs:9-19), on the GPU against the same loop over the oracle (oracle forward, oracle
sampler): the same tokens draw for draw and the same generator state at the end.

For a top_k up to 32 the draws run inside the one token-kernel launch of the loop (per-workgroup
top-k lists from the lm_head phase, merged in two levels at the next token's start); a top_k up to 64
(or DAIZA_PTK_SAMPLE=0) takes a launch per token with the top-k over the vocabulary (vocabulary
248320: 61 slices), the softmax over the k, the top-p cut and the draw in kernels between the
launches; a top_k above 64 and the graph path sample on the host from each forward's logits.  Bar:
identical tokens and generator state; the logits after the loop within 1e-3 normwise.
"""
import os

import numpy as np
import pytest

from conftest import normwise_rel

pytestmark = pytest.mark.gpu

SEED = 0xDA1A0071


def _oracle_loop(oracle, om, first, n, t, k, p, seed):
    rng = oracle.Rng(seed)
    tok, out = first, []
    for _ in range(n):
        _, lg = om.forward(tok)
        tok = int(oracle.sample_top_k_top_p(lg, t, k, p, rng))
        out.append(tok)
    return out, rng.state.value, lg


@pytest.fixture(scope="module")
def big_vocab(dz):
    cfg = dz.Config.small(n_layers=4, max_ctx=160, vocab=248320)
    return cfg, dz.Model.synthetic(cfg, SEED)


@pytest.mark.parametrize("t,k,p,n", [(0.7, 20, 0.95, 64), (0.8, 32, 0.9, 16), (1.3, 64, 0.9, 24),
                                     (0.5, 1, 0.95, 8), (0.9, 100, 0.8, 12), (0.7, 20, 0.95, 1),
                                     (2.0, 32, 1.0, 12), (0.05, 7, 0.5, 10)])
def test_decode_sample_matches_oracle_loop(dz, oracle, big_vocab, t, k, p, n):
    cfg, m = big_vocab
    ctx = dz.Context(m)
    assert ctx.token_kernel
    om = oracle.Model(cfg, SEED)
    first = 7
    rng = dz.LcgRng(0xC0FFEE + k)
    got = ctx.decode_sample(first, n, dz.SamplingParams(t, k, p), rng)
    want, state, lg = _oracle_loop(oracle, om, first, n, t, k, p, 0xC0FFEE + k)
    assert [int(x) for x in got] == want
    assert rng.state.value == state
    assert ctx.pos == n
    assert normwise_rel(ctx.logits(), lg) < 1e-3


def test_decode_sample_in_kernel_matches_launch_per_token(dz, big_vocab, monkeypatch):
    """The in-kernel draws against the launch-per-token path (DAIZA_PTK_SAMPLE=0) on two contexts of
    one model: the same tokens and generator states over a sampled call, a greedy call and a second
    sampled call with other parameters, which continue each other's positions and generator."""
    cfg, m = big_vocab
    a, b = dz.Context(m), dz.Context(m)
    ra, rb = dz.LcgRng(1234), dz.LcgRng(1234)

    def both(fn):
        x = fn(a, ra)
        monkeypatch.setenv("DAIZA_PTK_SAMPLE", "0")
        try:
            y = fn(b, rb)
        finally:
            monkeypatch.delenv("DAIZA_PTK_SAMPLE")
        assert [int(v) for v in x] == [int(v) for v in y]
        assert ra.state.value == rb.state.value
        return x

    t1 = both(lambda c, r: c.decode_sample(5, 12, dz.SamplingParams(0.9, 32, 0.9), r))
    t2 = both(lambda c, r: c.decode_greedy(int(t1[-1]), 3))
    both(lambda c, r: c.decode_sample(int(t2[-1]), 9, dz.SamplingParams(1.1, 7, 0.8), r))
    assert a.pos == b.pos == 24
    assert normwise_rel(a.logits(), b.logits()) < 1e-6


def test_decode_sample_greedy_temperature_and_errors(dz, big_vocab):
    """temperature 0 is the greedy loop with no draw; ids past the vocabulary and runs past max_ctx
    are refused before any launch."""
    cfg, m = big_vocab
    a, b = dz.Context(m), dz.Context(m)
    rng = dz.LcgRng(5)
    got = a.decode_sample(3, 10, dz.SamplingParams(0.0, 20, 0.95), rng)
    assert rng.state.value == 5
    assert np.array_equal(got, b.decode_greedy(3, 10))
    with pytest.raises(dz.DaizaError) as e:
        a.decode_sample(cfg.vocab, 4, dz.SamplingParams(0.7, 20, 0.95), rng)
    assert e.value.code == dz.DZ_ERR_TENSOR
    with pytest.raises(dz.DaizaError) as e:
        a.decode_sample(3, cfg.max_ctx, dz.SamplingParams(0.7, 20, 0.95), rng)
    assert e.value.code == dz.DZ_ERR_TENSOR
    assert a.pos == 10 and rng.state.value == 5


def test_decode_sample_graph_path(dz, oracle, monkeypatch):
    """The per-kernel graph path (DAIZA_PTK=0) samples on the host from each forward's logits: the same
    loop, draw for draw."""
    cfg = dz.Config.small(n_layers=4, max_ctx=64)
    m = dz.Model.synthetic(cfg, SEED + 1)
    monkeypatch.setenv("DAIZA_PTK", "0")
    ctx = dz.Context(m)
    monkeypatch.delenv("DAIZA_PTK")
    assert not ctx.token_kernel
    om = oracle.Model(cfg, SEED + 1)
    rng = dz.LcgRng(77)
    got = ctx.decode_sample(11, 16, dz.SamplingParams(0.8, 20, 0.9), rng)
    want, state, _ = _oracle_loop(oracle, om, 11, 16, 0.8, 20, 0.9, 77)
    assert [int(x) for x in got] == want and rng.state.value == state


def test_decode_sample_exact_ties(dz, oracle):
    """An lm_head whose rows 8192..12287 are byte copies of rows 0..4095 (vocabulary 12289, four
    device slices): every logit of the first slice has an exact twin in the third, so the device
    top-k must order equal values by lower index, as the oracle's sampler does, for the draws (and
    the chosen ids) to agree."""
    from named_tensors import named_tensors
    cfg = dz.Config.small(n_layers=4, max_ctx=64, vocab=12289)
    seed = SEED + 7
    om = oracle.Model(cfg, seed)
    t = named_tensors(oracle, om, cfg, seed)
    row = (cfg.hidden // 128) * 18
    w = t["output.weight"][1].copy()
    w[8192 * row:12288 * row] = w[0:4096 * row]
    t["output.weight"] = (dz.GGUF_Q1_0, w)
    m = dz.Model.from_tensors(cfg, t)
    ctx = dz.Context(m)
    assert ctx.token_kernel
    for k, temp in ((20, 0.7), (64, 1.5)):
        ctx.reset()
        o2 = oracle.Model(cfg, seed)
        o2.q1(3, -1)[0][:] = w  # the oracle's own lm_head buffer, written in place
        rng = dz.LcgRng(99 + k)
        got = ctx.decode_sample(3, 24, dz.SamplingParams(temp, k, 0.95), rng)
        want, state, _ = _oracle_loop(oracle, o2, 3, 24, temp, k, 0.95, 99 + k)
        assert [int(x) for x in got] == want, k
        assert rng.state.value == state
