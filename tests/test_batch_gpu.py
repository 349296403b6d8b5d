"""GPU parity of the n-token forward (forward_batch, forward.rs:394-1407) that prefill runs on
the matrix cores, against the CPU oracle and against the token-by-token decode path.

Bar: per-position logits, SSM states and KV entries within 1e-3 normwise relative error of the
oracle (the batched path sums in a different order, as the reference's own batched path does,
gemm.rs:153-225); greedy continuations after a batched prefill token-identical.
"""
import numpy as np
import pytest

from conftest import normwise_rel

pytestmark = pytest.mark.gpu

SEED = 0xDA1A0005


def _ids(cfg, n, seed):
    return np.random.default_rng(seed).integers(0, cfg.vocab, n).astype(np.uint32)


def _serial(monkeypatch):
    monkeypatch.setenv("DAIZA_BATCH", "0")


def test_batch_logits_vs_oracle_with_offset(dz, oracle):
    """Two decode tokens, then a 37-token batch starting at position 2, then one more token."""
    cfg = dz.Config.small(n_layers=8, max_ctx=96)
    m = dz.Model.synthetic(cfg, SEED)
    ctx = dz.Context(m)
    om = oracle.Model(cfg, SEED)
    for t in (9, 99):
        _, lg = ctx.forward_single_token(t)
        _, olg = om.forward(t)
        assert normwise_rel(lg, olg) < 1e-3
    ids = _ids(cfg, 37, 1)
    per = ctx.forward_batch(ids, per_pos_logits=True)
    assert ctx.pos == 39
    for i, t in enumerate(ids):
        _, olg = om.forward(int(t))
        assert normwise_rel(per[i], olg) < 1e-3, i
    am, lg = ctx.forward_single_token(5)
    oam, olg = om.forward(5)
    assert normwise_rel(lg, olg) < 1e-3
    assert am == oam
    # states after the batch and the token: every DeltaNet layer, every attention layer's cache
    for layer in range(cfg.n_layers):
        if (layer + 1) % cfg.full_attn_interval:
            sg, cg, hg = ctx.get_ssm_state(layer)
            so, co, ho = om.get_ssm_state(layer)
            assert hg == ho
            assert normwise_rel(sg, so) < 1e-3, layer
            assert normwise_rel(cg, co) < 1e-3, layer
        else:
            kg, vg = ctx.get_kv(layer, ctx.pos)
            ko, vo = om.get_kv(layer)
            assert normwise_rel(kg, ko) < 1e-3, layer
            assert normwise_rel(vg, vo) < 1e-3, layer


@pytest.mark.parametrize("n", [1, 3, 4, 5, 130])
def test_batch_matches_serial_path(dz, monkeypatch, n):
    """The batched forward and the token-by-token path agree (chunking at 128 with per-position
    logits included), and the decode that follows gives the same tokens."""
    cfg = dz.Config.small(n_layers=8, max_ctx=160 + 24)
    ids = _ids(cfg, n, 2 + n)
    out = {}
    for mode in ("batch", "serial"):
        if mode == "serial":
            _serial(monkeypatch)
        m = dz.Model.synthetic(cfg, SEED + 1)
        ctx = dz.Context(m)
        ctx.forward_single_token(7)
        out[mode] = ctx.forward_batch(ids, per_pos_logits=True)
        out[mode + "_tok"] = list(ctx.decode_greedy(int(np.argmax(out[mode][-1])), 16))
        out[mode + "_ssm"] = ctx.get_ssm_state(0)
        ctx.close()
        m.close()
    for i in range(n):
        assert normwise_rel(out["batch"][i], out["serial"][i]) < 1e-4, i
    assert out["batch_tok"] == out["serial_tok"]
    assert normwise_rel(out["batch_ssm"][0], out["serial_ssm"][0]) < 1e-4
    assert np.array_equal(out["batch_ssm"][1], out["serial_ssm"][1])  # conv ring: same inputs, same slots
    assert out["batch_ssm"][2] == out["serial_ssm"][2]


def test_batch_full_shape_layers(dz, oracle):
    """BASELINE shapes (hidden 5120, 48 v-heads, 24/4 attention heads): a DeltaNet layer and an
    attention layer over a 64-token batch after 8 decode tokens, against the oracle."""
    cfg = dz.Config.bonsai27b(max_ctx=96)
    cfg.n_layers, cfg.vocab, cfg.full_attn_interval = 2, 512, 2
    m = dz.Model.synthetic(cfg, SEED + 2)
    ctx = dz.Context(m)
    om = oracle.Model(cfg, SEED + 2)
    for t in range(8):
        ctx.forward_single_token(t * 31)
        om.forward(t * 31, want_logits=False)
    ids = _ids(cfg, 64, 3)
    last = ctx.forward_batch(ids)
    for t in ids:
        _, olg = om.forward(int(t))
    assert normwise_rel(last, olg) < 1e-3
    sg, cg, hg = ctx.get_ssm_state(0)
    so, co, ho = om.get_ssm_state(0)
    assert hg == ho and normwise_rel(sg, so) < 1e-3 and normwise_rel(cg, co) < 1e-3
    kg, vg = ctx.get_kv(1, ctx.pos)
    ko, vo = om.get_kv(1)
    assert normwise_rel(kg, ko) < 1e-3 and normwise_rel(vg, vo) < 1e-3
