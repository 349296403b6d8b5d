"""BASELINE configs 3-5 at their stated sizes on the GPU against the oracle.

- config 3: one gated attention layer of the 27B shape (24 q / 4 kv heads x 256) through the token
  kernel's 27B instance (6 query heads per kv head) at context 4096 and 32768 over an N(0,1) cache;
- config 4: the token kernel's DeltaNet and attention state after full-shape greedy decode steps;
- config 5: dz_spec_verify at vocabulary 248320 (61 slices of the device sampling) after an N(0,1)
  cache of 8192 positions, draw for draw against the reference's sequential loop over the oracle;
- the device sampling's per-row merges across slices (vocabulary 12289 = 4 slices), including an
  exact tie of the target maximum across two slices.
Bar: 1e-3 normwise relative error for logits, hidden and state; identical tokens and draws.
"""
import numpy as np
import pytest

from conftest import normwise_rel
from named_tensors import named_tensors
from test_verify_gpu import _compare_states, _reference_step

pytestmark = pytest.mark.gpu

SEED = 0xDA1A0013


def _attn_only_27b(dz, L):
    cfg = dz.Config.bonsai27b(max_ctx=L + 16)
    cfg.n_layers, cfg.vocab, cfg.full_attn_interval = 1, 1024, 1
    return cfg


@pytest.mark.parametrize("L", [4096, 32768])
def test_config3_token_kernel_long_context(dz, oracle, L):
    """forward_single_token through the token kernel's 27B instance at context L (attention.rs:124-199
    over a growing cache; kv_cache.rs:17-130): logits and the appended K/V rows."""
    cfg = _attn_only_27b(dz, L)
    m = dz.Model.synthetic(cfg, SEED)
    ctx = dz.Context(m)
    assert ctx.token_kernel
    om = oracle.Model(cfg, SEED)
    rng = np.random.default_rng(L)
    k = rng.standard_normal((cfg.n_head_kv, L, cfg.head_dim), dtype=np.float32)
    v = rng.standard_normal((cfg.n_head_kv, L, cfg.head_dim), dtype=np.float32)
    ctx.set_kv(0, k, v)
    om.set_kv(0, k, v)
    del k, v
    ctx.set_pos(L)
    om.set_pos(L)
    for t in (5, 777):
        am, lg = ctx.forward_single_token(t)
        oam, olg = om.forward(t)
        assert normwise_rel(lg, olg) < 1e-3, (L, t)
        assert am == oam
    kg, vg = ctx.get_kv(0, L + 2)
    ko, vo = om.get_kv(0)
    assert ko.shape[1] == L + 2
    assert normwise_rel(kg[:, L:], ko[:, L:]) < 1e-3 and normwise_rel(vg[:, L:], vo[:, L:]) < 1e-3
    assert np.array_equal(kg[:, :8], ko[:, :8])


def test_config4_decode_states_full_shape(dz, oracle):
    """Three DeltaNet layers and one attention layer of the 27B shape: a 16-token batched prefill,
    then 8 greedy tokens in the token kernel; tokens, every DeltaNet state and conv ring, and the KV
    cache against the oracle's forward_single_token sequence."""
    cfg = dz.Config.bonsai27b(max_ctx=64)
    cfg.n_layers, cfg.vocab = 4, 4096
    m = dz.Model.synthetic(cfg, SEED + 1)
    ctx = dz.Context(m)
    assert ctx.token_kernel
    om = oracle.Model(cfg, SEED + 1)
    prompt = [int(t) for t in np.random.default_rng(5).integers(0, cfg.vocab, 16)]
    last = ctx.forward_batch(np.array(prompt, np.uint32))
    for t in prompt:
        first, olg = om.forward(t)
    assert normwise_rel(last, olg) < 1e-3
    got = ctx.decode_greedy(first, 8)
    want, tok = [], first
    for _ in range(8):
        tok, _ = om.forward(tok, want_logits=False)
        want.append(tok)
    assert list(got) == want
    assert ctx.pos == om.pos
    _compare_states(ctx, om, cfg)


def _spec_case(dz, oracle, cfg, seed, prompt_ids, case, k=8, setup=None, model=None, lm_bytes=None):
    """dz_spec_verify vs _reference_step for one case on a fresh context of `cfg` (lm_bytes: the
    lm_head bytes of `model` when they differ from the seed's, given to the oracle models too)."""
    T, top_k, top_p = (0.0, 20, 0.95) if case.startswith("greedy") else (0.7, 20, 0.95)
    m = model if model is not None else dz.Model.synthetic(cfg, seed)
    ctx = dz.Context(m)
    om = oracle.Model(cfg, seed)
    probe = oracle.Model(cfg, seed)
    if lm_bytes is not None:
        for o in (om, probe):
            o.q1(3, -1)[0][:] = lm_bytes  # the oracle's own lm_head buffer, written in place
    if setup:
        setup(ctx, om, probe)
    last = ctx.forward_batch(np.array(prompt_ids, np.uint32))
    for t in prompt_ids:
        _, olg = om.forward(t)
        _, plg = probe.forward(t)
    assert normwise_rel(last, olg) < 1e-3
    draft, dlog = [], []
    for i in range(k):
        t = int(np.argmax(plg))
        dlog.append(plg.copy())
        draft.append(t)
        _, plg = probe.forward(t)
    dlog = np.array(dlog, np.float32)
    if case == "reject_at_3":
        draft[3] = int(np.argmin(dlog[3]))
        dlog[3] = np.random.default_rng(8).standard_normal(cfg.vocab).astype(np.float32) * 0.1
        dlog[3][draft[3]] = 30.0
    elif case == "random_drafts":
        draft = [int(t) for t in np.random.default_rng(9).integers(0, cfg.vocab, k)]
        dlog = np.random.default_rng(10).standard_normal((k, cfg.vocab)).astype(np.float32)
    elif case == "greedy_reject":
        draft[2] = (draft[2] + 1) % cfg.vocab
    params = dz.SamplingParams(T, top_k, top_p)
    rg, ro = dz.LcgRng(0xC0FFEE), oracle.Rng(0xC0FFEE)
    na, bonus = ctx.spec_verify(draft, None if T <= 0 else dlog, params, rg)
    ona, obonus = _reference_step(oracle, om, olg, draft, dlog, T, top_k, top_p, ro)
    assert (na, bonus) == (ona, obonus), (case, na, bonus, ona, obonus)
    assert rg.state.value == ro.state.value
    if case in ("all_accept", "greedy"):
        assert na == k
    if case == "reject_at_3":
        assert na == 3
    if case == "greedy_reject":
        assert na == 2
    assert ctx.pos == om.pos
    _compare_states(ctx, om, cfg)
    return ctx, om, bonus


@pytest.mark.parametrize("case", ["all_accept", "reject_at_3", "random_drafts", "greedy", "greedy_reject"])
def test_config5_spec_verify_full_vocab_ctx8192(dz, oracle, case):
    """BASELINE config 5 at its stated sizes: the 27B layer shapes (one DeltaNet, one attention
    layer), vocabulary 248320, an N(0,1) cache of 8192 positions and seeded recurrent state; k = 8
    drafts verified in one forward, Leviathan at T = 0.7 (engine.rs:1791-1866) or greedy."""
    cfg = dz.Config.bonsai27b(max_ctx=8192 + 32)
    cfg.n_layers, cfg.full_attn_interval = 2, 2
    L = 8192
    rng = np.random.default_rng(21)
    kv_k = rng.standard_normal((cfg.n_head_kv, L, cfg.head_dim), dtype=np.float32)
    kv_v = rng.standard_normal((cfg.n_head_kv, L, cfg.head_dim), dtype=np.float32)
    st = (rng.standard_normal((cfg.ssm_v_heads, cfg.ssm_state, cfg.ssm_state)) * 0.02).astype(np.float32)
    conv = (rng.standard_normal((4, cfg.qkv_dim)) * 0.1).astype(np.float32)

    def setup(ctx, om, probe):
        ctx.set_pos(L)
        ctx.set_kv(1, kv_k, kv_v)
        ctx.set_ssm_state(0, st, conv, 1)
        for o in (om, probe):
            o.set_pos(L)
            o.set_kv(1, kv_k, kv_v)
            o.set_ssm_state(0, st, conv, 1)

    ctx, om, bonus = _spec_case(dz, oracle, cfg, SEED + 2, [3, 99], case, setup=setup)
    if bonus is not None:
        am, lg = ctx.forward_single_token(bonus)
        oam, olg = om.forward(bonus)
        assert normwise_rel(lg, olg) < 1e-3 and am == oam


@pytest.mark.parametrize("case", ["reject_at_3", "greedy"])
def test_config5_spec_verify_64_layers(dz, oracle, case):
    """BASELINE config 5 at the model's own depth: the full 64-layer 27B model (48 Gated DeltaNet +
    16 attention layers, vocabulary 248320), an N(0,1) cache of 8192 positions on every attention
    layer and seeded state and conv rings on every DeltaNet layer; k = 8 drafts in one verify forward
    (the forward bench.py times), Leviathan at T = 0.7 with a rejection, and greedy.  Accept count,
    bonus token, generator state and every layer's state against the reference's sequential loop
    (engine.rs:1255-1470, 1791-1866) over the oracle."""
    cfg = dz.Config.bonsai27b(max_ctx=8192 + 32)
    L = 8192
    rng = np.random.default_rng(64)
    attn = [i for i in range(cfg.n_layers) if (i + 1) % cfg.full_attn_interval == 0]
    assert len(attn) == 16
    kv = {i: (rng.standard_normal((cfg.n_head_kv, L, cfg.head_dim), dtype=np.float32),
              rng.standard_normal((cfg.n_head_kv, L, cfg.head_dim), dtype=np.float32)) for i in attn}
    dn = {}
    for i in range(cfg.n_layers):
        if i not in kv:
            st = (rng.standard_normal((cfg.ssm_v_heads, cfg.ssm_state, cfg.ssm_state)) * 0.02).astype(np.float32)
            conv = (rng.standard_normal((4, cfg.qkv_dim)) * 0.1).astype(np.float32)
            dn[i] = (st, conv, i % 4)
    assert len(dn) == 48

    def setup(ctx, om, probe):
        for o in (ctx, om, probe):
            o.set_pos(L)
            for i, (k, v) in kv.items():
                o.set_kv(i, k, v)
            for i, (st, conv, head) in dn.items():
                o.set_ssm_state(i, st, conv, head)

    _spec_case(dz, oracle, cfg, SEED + 5, [3, 99], case, setup=setup)


def _tie_model(dz, oracle, cfg, seed, prompt):
    """The synthetic model with lm_head row b made a byte copy of the target maximum's row a after
    the prompt, b in another 4096-logit slice than a: an exact tie of the maximum across slices."""
    om = oracle.Model(cfg, seed)
    for t in prompt:
        _, lg = om.forward(t)
    a = int(np.argmax(lg))
    b = (a + 2 * 4096 + 7) % cfg.vocab
    if b // 4096 == a // 4096:
        b = (b + 4096) % cfg.vocab
    t = named_tensors(oracle, om, cfg, seed)
    row = (cfg.hidden // 128) * 18
    w = t["output.weight"][1].copy()
    w[b * row:(b + 1) * row] = w[a * row:(a + 1) * row]
    t["output.weight"] = (dz.GGUF_Q1_0, w)
    return dz.Model.from_tensors(cfg, t), t, a, b


@pytest.mark.parametrize("case", ["all_accept", "reject_at_3", "random_drafts", "greedy", "greedy_tie"])
def test_spec_merges_across_slices(dz, oracle, case):
    """Vocabulary 12289: four slices of 4096 logits (the last holding one), so the per-row maxima,
    rescaled sums, draft-token p/q, argmax and top-k candidates all merge across slices.  greedy_tie
    copies the target maximum's lm_head row into another slice: the exact tie must go to the lower
    index (argmax_avx2, simd_exp.rs:551-598), or the greedy check rejects draft 0."""
    cfg = dz.Config.small(n_layers=4, max_ctx=64, vocab=12289)
    seed = SEED + 3
    prompt = [int(t) for t in np.random.default_rng(4).integers(0, cfg.vocab, 6)]
    if case != "greedy_tie":
        _spec_case(dz, oracle, cfg, seed, prompt, case)
        return
    model, tensors, a, b = _tie_model(dz, oracle, cfg, seed, prompt)
    ctx, om, _ = _spec_case(dz, oracle, cfg, seed, prompt, "greedy", model=model,
                            lm_bytes=tensors["output.weight"][1])
    # the tie itself, on a fresh context after the prompt
    c2 = dz.Context(model)
    lg = c2.forward_batch(np.array(prompt, np.uint32))
    assert lg[a] == lg[b] == lg.max()
