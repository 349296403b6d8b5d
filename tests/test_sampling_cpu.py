"""Speculative-verify sampling on the host (no GPU): the oracle's restatement of LcgRng,
sample_top_k_top_p_into, softmax_pair_single, sample_bonus and leviathan_check
(sampling.rs:9-19,144-247; simd_exp.rs:605-767; engine.rs:1791-1866) pinned by known answers and
closed forms, then the library's sampler (libdaiza_hip.so host code) against it draw for draw.
"""
import ctypes

import numpy as np
import pytest


def _lcg_seq(seed, n):
    s, out = seed, []
    for _ in range(n):
        s = (s * 6364136223846793005 + 1442695040888963407) & (2**64 - 1)
        out.append(((s >> 40) & 0xFFFFFF) / float(1 << 24))
    return out


def _trunc_dist(logits, temperature, top_k, top_p):
    """float64 closed form of the distribution sample_top_k_top_p_into draws from: softmax of the
    temperature-scaled top k (descending), cut after the first index whose cumulative mass
    reaches top_p, renormalised."""
    x = np.asarray(logits, np.float64) / temperature
    order = np.argsort(-x, kind="stable")[:top_k]
    p = np.exp(x[order] - x[order].max())
    p /= p.sum()
    c = np.cumsum(p)
    cut = int(np.argmax(c >= top_p)) + 1 if np.any(c >= top_p) else len(p)
    p = p[:cut] / p[:cut].sum()
    return order[:cut], p


@pytest.fixture(scope="module")
def dzl():
    import daiza_amd
    return daiza_amd


def test_lcg_matches_closed_form(oracle, dzl):
    want = _lcg_seq(0xC0FFEE, 50)
    r1, r2 = oracle.Rng(0xC0FFEE), dzl.LcgRng(0xC0FFEE)
    for w in want:
        assert r1.next_f32() == np.float32(w)
        assert r2.next_f32() == np.float32(w)


def test_oracle_softmax_pieces(oracle):
    rng = np.random.default_rng(0)
    for n in (5, 8, 1000, 248320):
        t = (rng.standard_normal(n) * 3).astype(np.float32)
        d = (rng.standard_normal(n) * 3).astype(np.float32)
        pt = np.exp(t.astype(np.float64) - t.max())
        pt /= pt.sum()
        pd = np.exp(d.astype(np.float64) - d.max())
        pd /= pd.sum()
        # f32 sums over n/8 terms per lane (the reference's own rounding): relative error grows with n
        tol = 1e-5 if n <= 1000 else 2e-4
        assert np.allclose(oracle.softmax(t), pt, rtol=tol, atol=1e-12)
        for idx in (0, n // 3, n - 1):
            p, q = oracle.softmax_pair_single(t, d, idx)
            assert abs(p - pt[idx]) <= tol * pt[idx] + 1e-12
            assert abs(q - pd[idx]) <= tol * pd[idx] + 1e-12


def test_oracle_sample_greedy_and_top1(oracle):
    x = np.array([0.5, 2.0, -1.0, 2.0, 1.9], np.float32)
    r = oracle.Rng(1)
    assert oracle.sample_top_k_top_p(x, 0.0, 20, 0.95, r) == 1  # argmax, lowest index on ties
    assert r.state.value == 1                                      # greedy draws nothing
    for _ in range(20):
        assert oracle.sample_top_k_top_p(x, 0.7, 1, 0.95, r) in (1, 3)  # top-1: one of the tied maxima
    assert r.state.value != 1


@pytest.mark.parametrize("temperature,top_k,top_p", [(0.7, 20, 0.95), (1.3, 5, 0.5), (0.7, 50, 1.0)])
def test_oracle_sample_follows_closed_form(oracle, temperature, top_k, top_p):
    """Each draw is the first index whose cumulative truncated probability reaches u (u = the
    LcgRng value), over float64 probabilities; exact except within 1e-5 of a boundary."""
    rng = np.random.default_rng(7)
    logits = (rng.standard_normal(300) * 2).astype(np.float32)
    idx, p = _trunc_dist(logits, temperature, top_k, top_p)
    c = np.cumsum(p)
    seed = 12345
    r = oracle.Rng(seed)
    us = _lcg_seq(seed, 400)
    checked = 0
    for u in us:
        got = oracle.sample_top_k_top_p(logits, temperature, top_k, top_p, r)
        if np.min(np.abs(c - u)) < 1e-5:
            continue
        j = int(np.argmax(c >= u)) if u <= c[-1] else 0
        assert got == idx[j]
        checked += 1
    assert checked > 350


def test_oracle_bonus_and_leviathan_closed_cases(oracle):
    rng = np.random.default_rng(3)
    t = (rng.standard_normal(1000) * 2).astype(np.float32)
    # p == q: the residual has no mass -> sample from the target with the same draw
    r1, r2 = oracle.Rng(9), oracle.Rng(9)
    assert oracle.sample_bonus(t, t, 0.7, 20, 0.95, r1) == oracle.sample_top_k_top_p(t, 0.7, 20, 0.95, r2)
    assert r1.state.value == r2.state.value
    # q == p: p/q = 1 > u always -> accept
    r = oracle.Rng(5)
    assert all(oracle.leviathan_check(t, t, int(k), 0.7, r) for k in range(0, 1000, 37))
    # draft puts all mass on a token the target gives ~0 -> reject
    d = np.full(1000, -50.0, np.float32)
    d[int(np.argmin(t))] = 50.0
    assert not oracle.leviathan_check(t, d, int(np.argmin(t)), 0.7, r)
    # greedy: argmax comparison, no draw
    s0 = r.state.value
    assert oracle.leviathan_check(t, None, int(np.argmax(t)), 0.0, r)
    assert not oracle.leviathan_check(t, None, int(np.argmin(t)), 0.0, r)
    assert r.state.value == s0
    # residual distribution: a bonus is never a token with p <= q
    p, q = oracle.softmax(t), oracle.softmax(d * 0.01)
    d2 = (d * 0.01).astype(np.float32)
    r = oracle.Rng(11)
    for _ in range(50):
        b = oracle.sample_bonus(t, d2, 1.0, 1000, 1.0, r)
        assert p[b] > q[b]


@pytest.mark.parametrize("temperature,top_k,top_p", [(0.7, 20, 0.95), (1.0, 3, 0.9), (0.0, 20, 0.95)])
def test_library_sampler_matches_oracle(oracle, dzl, temperature, top_k, top_p):
    rng = np.random.default_rng(21)
    params = dzl.SamplingParams(temperature, top_k, top_p)
    for trial in range(40):
        n = int(rng.integers(2, 5000))
        t = (rng.standard_normal(n) * 2).astype(np.float32)
        d = (t + rng.standard_normal(n).astype(np.float32) * 0.5).astype(np.float32)
        tok = int(rng.integers(0, n))
        seed = int(rng.integers(0, 2**63))
        ro, rl = oracle.Rng(seed), dzl.LcgRng(seed)
        assert dzl.sample_top_k_top_p(t, params, rl) == oracle.sample_top_k_top_p(t, temperature, top_k, top_p, ro)
        assert dzl.leviathan_check(t, d, tok, params, rl) == oracle.leviathan_check(t, d, tok, temperature, ro)
        if temperature > 0:
            assert dzl.sample_bonus(t, d, params, rl) == oracle.sample_bonus(t, d, temperature, top_k, top_p, ro)
        assert rl.state.value == ro.state.value, trial


@pytest.mark.parametrize("top_k", [3, 20, 64])
def test_library_sampler_exact_ties(oracle, dzl, top_k):
    """Logits with many exactly equal values straddling the top-k boundary: the library's sampler
    keeps the k best by value and, among equal values, by lower index, as the oracle and the device
    top-k do, so the draws and the generator state agree."""
    rng = np.random.default_rng(5)
    params = dzl.SamplingParams(0.8, top_k, 0.97)
    for trial in range(30):
        n = int(rng.integers(top_k + 1, 3000))
        t = rng.integers(-3, 4, n).astype(np.float32) * 0.5  # seven distinct values
        seed = int(rng.integers(0, 2**63))
        ro, rl = oracle.Rng(seed), dzl.LcgRng(seed)
        for _ in range(4):
            assert dzl.sample_top_k_top_p(t, params, rl) == oracle.sample_top_k_top_p(t, 0.8, top_k, 0.97, ro), trial
        assert rl.state.value == ro.state.value
