"""GPU parity of speculative verify: k drafts in one n-token forward with
per-token DeltaNet rollback records, the accepted prefix kept afterwards, and Leviathan acceptance
with bonus sampling in the reference's order (engine.rs:1255-1470, 1791-1866).

The reference verifies sequentially, forwarding each accepted draft with forward_single_token.
The oracle side of these tests does exactly that; the GPU side runs dz_verify_forward +
dz_verify_commit (or dz_spec_verify).  Bar: logits and states within 1e-3 normwise relative error,
identical accept counts, bonus tokens and generator states.
"""
import numpy as np
import pytest

from conftest import normwise_rel

pytestmark = pytest.mark.gpu

SEED = 0xDA1A0007


def _ids(cfg, n, seed):
    return [int(t) for t in np.random.default_rng(seed).integers(0, cfg.vocab, n)]


def _gpu(dz, cfg, prompt):
    m = dz.Model.synthetic(cfg, SEED)
    ctx = dz.Context(m)
    last = ctx.forward_batch(np.array(prompt, np.uint32))
    return m, ctx, last


def _oracle(oracle, cfg, prompt):
    om = oracle.Model(cfg, SEED)
    lg = None
    for t in prompt:
        _, lg = om.forward(t)
    return om, lg


def _compare_states(ctx, om, cfg, tol=1e-3):
    for layer in range(cfg.n_layers):
        if (layer + 1) % cfg.full_attn_interval:
            sg, cg, hg = ctx.get_ssm_state(layer)
            so, co, ho = om.get_ssm_state(layer)
            assert hg == ho, layer
            assert normwise_rel(sg, so) < tol, layer
            assert normwise_rel(cg, co) < tol, layer
        else:
            kg, vg = ctx.get_kv(layer, ctx.pos)
            ko, vo = om.get_kv(layer)
            assert ko.shape[1] == ctx.pos
            assert normwise_rel(kg, ko) < tol and normwise_rel(vg, vo) < tol, layer


def test_verify_forward_logits(dz, oracle):
    cfg = dz.Config.small(n_layers=8, max_ctx=96)
    prompt = _ids(cfg, 12, 1)
    draft = _ids(cfg, 8, 2)
    m, ctx, _ = _gpu(dz, cfg, prompt)
    om, _ = _oracle(oracle, cfg, prompt)
    p0 = ctx.pos
    per = ctx.verify_forward(draft)
    assert ctx.pos == p0  # nothing kept yet
    for i, t in enumerate(draft):
        _, olg = om.forward(t)
        assert normwise_rel(per[i], olg) < 1e-3, i


@pytest.mark.parametrize("a", [0, 1, 3, 4, 5, 8])
def test_verify_commit_prefix(dz, oracle, a):
    """Keeping a of 8 drafts leaves the context exactly where forwarding those a drafts would."""
    cfg = dz.Config.small(n_layers=8, max_ctx=96)
    prompt = _ids(cfg, 12, 1)
    draft = _ids(cfg, 8, 3)
    m, ctx, last = _gpu(dz, cfg, prompt)
    om, olg = _oracle(oracle, cfg, prompt)
    ctx.verify_forward(draft, want_logits=False)
    ctx.verify_commit(a)
    for t in draft[:a]:
        _, olg = om.forward(t)
    assert ctx.pos == om.pos == len(prompt) + a
    _compare_states(ctx, om, cfg)
    # the context's logits are those after the last kept draft
    lg = ctx.logits()
    assert normwise_rel(lg, olg) < 1e-3
    # and the next forward continues from there
    am, lg = ctx.forward_single_token(77)
    oam, olg = om.forward(77)
    assert normwise_rel(lg, olg) < 1e-3 and am == oam


def test_verify_commit_equals_batch_forward(dz):
    """The replayed DeltaNet updates reproduce the scan's state bit for bit."""
    cfg = dz.Config.small(n_layers=4, max_ctx=64)
    prompt = _ids(cfg, 6, 4)
    draft = _ids(cfg, 8, 5)
    m1, c1, _ = _gpu(dz, cfg, prompt)
    m2, c2, _ = _gpu(dz, cfg, prompt)
    c1.verify_forward(draft, want_logits=False)
    c1.verify_commit(5)
    c2.forward_batch(np.array(draft[:5], np.uint32))
    for layer in range(cfg.n_layers):
        if (layer + 1) % cfg.full_attn_interval:
            s1, r1, h1 = c1.get_ssm_state(layer)
            s2, r2, h2 = c2.get_ssm_state(layer)
            assert np.array_equal(s1, s2) and np.array_equal(r1, r2) and h1 == h2, layer
    assert normwise_rel(c1.logits(), c2.logits()) < 1e-6


def _reference_step(oracle, om, target, draft, draft_logits, T, top_k, top_p, rng, eos=-1):
    """engine.rs:1255-1470: sequential Leviathan verify, forwarding each accepted draft."""
    acc, bonus = 0, None
    for i, dt in enumerate(draft):
        ok = oracle.leviathan_check(target, None if T <= 0 else draft_logits[i], dt, T, rng)
        if not ok:
            bonus = int(np.argmax(target)) if T <= 0 else oracle.sample_bonus(target, draft_logits[i], T, top_k,
                                                                              top_p, rng)
            return acc, bonus
        acc += 1
        if dt == eos:
            return acc, None
        _, target = om.forward(dt)
    return acc, oracle.sample_top_k_top_p(target, T, top_k, top_p, rng)


@pytest.mark.parametrize("case", ["all_accept", "reject_at_3", "random_drafts", "greedy", "eos", "wide_top_k"])
def test_spec_verify_matches_sequential_reference(dz, oracle, case):
    """The vocabulary-wide sampling runs on the device for top_k <= 64 and on the host beyond
    (wide_top_k); both must follow the reference draw for draw."""
    cfg = dz.Config.small(n_layers=8, max_ctx=96)
    prompt = _ids(cfg, 10, 6)
    T, top_k, top_p = (0.0, 20, 0.95) if case == "greedy" else (0.7, 100 if case == "wide_top_k" else 20, 0.95)
    k = 8
    m, ctx, _ = _gpu(dz, cfg, prompt)
    om, olg = _oracle(oracle, cfg, prompt)
    # drafts: the target's own greedy continuation (probe model), with draft logits equal to the
    # target's (p = q, always accepted at T > 0), changed from position 3 on for the rejecting case
    probe, plg = _oracle(oracle, cfg, prompt)
    draft, dlog = [], []
    for i in range(k):
        t = int(np.argmax(plg))
        dlog.append(plg.copy())
        draft.append(t)
        _, plg = probe.forward(t)
    dlog = np.array(dlog, np.float32)
    eos = -1
    if case == "reject_at_3":
        rng = np.random.default_rng(8)
        draft[3] = int(np.argmin(dlog[3]))
        dlog[3] = rng.standard_normal(cfg.vocab).astype(np.float32) * 0.1
        dlog[3][draft[3]] = 30.0
    elif case in ("random_drafts", "wide_top_k"):
        draft = _ids(cfg, k, 9)
        dlog = np.random.default_rng(10).standard_normal((k, cfg.vocab)).astype(np.float32)
    elif case == "eos":
        eos = draft[2]
    params = dz.SamplingParams(T, top_k, top_p)
    rg, ro = dz.LcgRng(0xC0FFEE), oracle.Rng(0xC0FFEE)
    na, bonus = ctx.spec_verify(draft, None if T <= 0 else dlog, params, rg, eos_id=eos)
    ona, obonus = _reference_step(oracle, om, olg, draft, dlog, T, top_k, top_p, ro, eos)
    assert (na, bonus) == (ona, obonus), (case, na, bonus, ona, obonus)
    assert rg.state.value == ro.state.value
    if case in ("all_accept", "greedy"):
        assert na == k
    if case == "reject_at_3":
        assert na == 3
    # kept state = the reference's (an accepted EOS is not forwarded)
    assert ctx.pos == om.pos
    _compare_states(ctx, om, cfg)
    if bonus is not None:
        am, lg = ctx.forward_single_token(bonus)
        oam, olg2 = om.forward(bonus)
        assert normwise_rel(lg, olg2) < 1e-3 and am == oam


def test_verify_full_shape_long_context(dz, oracle):
    """BASELINE config 5 shapes: a DeltaNet and an attention layer of the 27B model, k = 8 drafts
    after a 1000-token N(0,1) KV cache and random recurrent state: per-position logits, then 5 kept."""
    cfg = dz.Config.bonsai27b(max_ctx=1024 + 16)
    cfg.n_layers, cfg.vocab, cfg.full_attn_interval = 2, 1024, 2
    m = dz.Model.synthetic(cfg, SEED)
    ctx = dz.Context(m)
    om = oracle.Model(cfg, SEED)
    L = 1000
    rng = np.random.default_rng(11)
    k_ = rng.standard_normal((cfg.n_head_kv, L, cfg.head_dim)).astype(np.float32)
    v_ = rng.standard_normal((cfg.n_head_kv, L, cfg.head_dim)).astype(np.float32)
    st = (rng.standard_normal((cfg.ssm_v_heads, cfg.ssm_state, cfg.ssm_state)) * 0.02).astype(np.float32)
    conv = (rng.standard_normal((4, cfg.qkv_dim)) * 0.1).astype(np.float32)
    ctx.set_pos(L)
    om.set_pos(L)
    ctx.set_kv(1, k_, v_)
    om.set_kv(1, k_, v_)
    ctx.set_ssm_state(0, st, conv, 1)
    om.set_ssm_state(0, st, conv, 1)
    _, lg = ctx.forward_single_token(3)
    _, olg = om.forward(3)
    assert normwise_rel(lg, olg) < 1e-3
    draft = _ids(cfg, 8, 12)
    per = ctx.verify_forward(draft)
    probe = []
    for t in draft:
        _, x = om.forward(t)
        probe.append(x)
    for i in range(8):
        assert normwise_rel(per[i], probe[i]) < 1e-3, i
    ctx.verify_commit(5)
    om2 = oracle.Model(cfg, SEED)
    om2.set_pos(L)
    om2.set_kv(1, k_, v_)
    om2.set_ssm_state(0, st, conv, 1)
    for t in [3] + draft[:5]:
        om2.forward(t, want_logits=False)
    assert ctx.pos == om2.pos
    _compare_states(ctx, om2, cfg)
