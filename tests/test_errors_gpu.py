"""Error behaviour of the decode and verify entry points (BonsaiError counterparts, lib.rs:42-78):
bad ids, empty batches, a full context and verify misuse are refused on the host with DZ_ERR_TENSOR
before any launch, and the context stays usable with its state unchanged (checked against the
oracle after each refusal)."""
import numpy as np
import pytest

from conftest import normwise_rel

pytestmark = pytest.mark.gpu

SEED = 0xDA1A0009


def _pair(dz, oracle, max_ctx=40):
    cfg = dz.Config.small(n_layers=4, max_ctx=max_ctx)
    m = dz.Model.synthetic(cfg, SEED)
    ctx = dz.Context(m)
    om = oracle.Model(cfg, SEED)
    return cfg, m, ctx, om


def _refused(dz, fn, *args, empty=False):
    """fn(*args) raises DaizaError with DZ_ERR_TENSOR (an empty array may also be refused as a null
    argument, DZ_ERR_MODEL, depending on the pointer numpy gives it)."""
    with pytest.raises(dz.DaizaError) as ei:
        fn(*args)
    ok = (dz.DZ_ERR_TENSOR, dz.DZ_ERR_MODEL) if empty else (dz.DZ_ERR_TENSOR,)
    assert ei.value.code in ok, str(ei.value)


def _still_matches(ctx, om, tok=17):
    am, lg = ctx.forward_single_token(tok)
    oam, olg = om.forward(tok)
    assert am == oam and normwise_rel(lg, olg) < 1e-3
    assert ctx.pos == om.pos


def test_bad_ids_and_empty_batches(dz, oracle):
    cfg, m, ctx, om = _pair(dz, oracle)
    for t in (3, 9):
        ctx.forward_single_token(t)
        om.forward(t)
    p0 = ctx.pos
    _refused(dz, ctx.forward_batch, np.array([1, cfg.vocab, 2], np.uint32))  # id == vocab
    _refused(dz, ctx.forward_batch, np.zeros(0, np.uint32), empty=True)      # empty batch
    _refused(dz, ctx.forward_single_token, cfg.vocab + 5)
    _refused(dz, ctx.decode_greedy, 0xFFFFFFFF, 4)
    assert ctx.pos == p0
    _still_matches(ctx, om)


def test_full_context_is_refused(dz, oracle):
    cfg, m, ctx, om = _pair(dz, oracle, max_ctx=16)
    ids = np.arange(1, 13, dtype=np.uint32)
    ctx.forward_batch(ids)
    for t in ids:
        om.forward(int(t), want_logits=False)
    assert ctx.pos == 12
    _refused(dz, ctx.forward_batch, np.arange(5, dtype=np.uint32))  # 12 + 5 > 16
    _refused(dz, ctx.decode_greedy, 4, 5)
    _refused(dz, ctx.verify_forward, [1, 2, 3, 4, 5])
    assert ctx.pos == 12
    _still_matches(ctx, om)


def test_verify_misuse(dz, oracle):
    cfg, m, ctx, om = _pair(dz, oracle)
    for t in (3, 9, 27):
        ctx.forward_single_token(t)
        om.forward(t)
    _refused(dz, ctx.verify_commit, 2)               # no verify forward pending
    ctx.verify_commit(0)                             # nothing pending, nothing kept: a no-op
    _refused(dz, ctx.verify_forward, [], empty=True)  # no drafts
    ctx.verify_forward([5, 6, 7], want_logits=False)
    _refused(dz, ctx.verify_commit, 4)               # more than the 3 drafts
    _refused(dz, ctx.verify_commit, -1)
    ctx.verify_commit(0)                             # keep none of them
    params = dz.SamplingParams(0.7, 20, 0.95)
    _refused(dz, ctx.spec_verify, [], None, params, dz.LcgRng(1), empty=True)
    _still_matches(ctx, om)
