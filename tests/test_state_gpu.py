"""GPU tests of the boundary's state handling: the real-weights entry (dz_model_create with GGUF
names, both token-embedding formats), the argmax tie rule across lm_head workgroups, KV truncation
(KvCache::truncate keeps every conv ring where it is), the greedy loop's EOS stop, the refusal of a
context whose launch gave up part-way, and state copies between contexts (checkpoint / restore).
Oracle: oracle/oracle.c (the reference's algorithm).
"""
import numpy as np
import pytest

from conftest import normwise_rel
from named_tensors import named_tensors

pytestmark = pytest.mark.gpu

SEED = 0xDA1A0011


def _oracle_greedy(om, first, n):
    out, tok = [], first
    for _ in range(n):
        tok, _ = om.forward(tok, want_logits=False)
        out.append(tok)
    return out


@pytest.mark.parametrize("embd_f16", [1, 0])
def test_model_create_from_named_tensors(dz, oracle, embd_f16):
    """dz_model_create (LoadedWeights::load_all, weights.rs:1308-1379) from the GGUF-named tensors
    of the synthetic model: the same logits as dz_model_create_synth bit for bit, and as the oracle.
    embd_f16 = 0 is the reference's own Q1_0 token embedding (weights.rs:1309)."""
    cfg = dz.Config.small(n_layers=4, max_ctx=32, embd_f16=embd_f16)
    om = oracle.Model(cfg, SEED)
    tensors = named_tensors(oracle, om, cfg, SEED)
    m_named = dz.Model.from_tensors(cfg, tensors)
    m_synth = dz.Model.synthetic(cfg, SEED)
    assert m_named.q1_bytes() == m_synth.q1_bytes()
    c_named, c_synth = dz.Context(m_named), dz.Context(m_synth)
    for t in (5, 2047, 0, 731, 1999, 12):
        a1, l1 = c_named.forward_single_token(t)
        a2, l2 = c_synth.forward_single_token(t)
        ao, lo = om.forward(t)
        assert np.array_equal(l1, l2), t
        assert normwise_rel(l1, lo) < 1e-3, t
        assert a1 == a2 == ao, t
    # the batched forward reads the same embedding
    c_named.reset()
    last = c_named.forward_batch(np.array([5, 2047, 0, 731, 1999, 12], np.uint32))
    assert normwise_rel(last, lo) < 1e-3


def test_model_create_rejects_bad_tables(dz, oracle):
    cfg = dz.Config.small(n_layers=4, max_ctx=32)
    om = oracle.Model(cfg, SEED)
    t = named_tensors(oracle, om, cfg, SEED)
    missing = dict(t)
    del missing["blk.1.ssm_a"]
    with pytest.raises(dz.DaizaError) as e:
        dz.Model.from_tensors(cfg, missing)
    assert e.value.code == dz.DZ_ERR_MODEL
    wrong_type = dict(t)
    wrong_type["output_norm.weight"] = (dz.GGUF_F16, t["output_norm.weight"][1].astype(np.float16))
    with pytest.raises(dz.DaizaError) as e:
        dz.Model.from_tensors(cfg, wrong_type)
    assert e.value.code == dz.DZ_ERR_MODEL
    short = dict(t)
    short["blk.0.ffn_down.weight"] = (dz.GGUF_Q1_0, t["blk.0.ffn_down.weight"][1][:-18])
    with pytest.raises(dz.DaizaError) as e:
        dz.Model.from_tensors(cfg, short)
    assert e.value.code == dz.DZ_ERR_TENSOR


@pytest.fixture(params=["token_kernel", "graph"])
def launch_path(request, monkeypatch):
    monkeypatch.setenv("DAIZA_PTK", "1" if request.param == "token_kernel" else "0")
    return request.param


def test_argmax_ties_take_lowest_index(dz, oracle, launch_path):
    """argmax_avx2 (simd_exp.rs:551-598) keeps the first of equal maxima.  The lm_head holds one row
    pattern R in every row r = 5 (mod 64), its negation -R in every row r = 9 (mod 64), and zero
    scales elsewhere (logit exactly 0).  Rows of one residue take the same lane of every row-block,
    so their logits are bit-identical on the device (a lane's lookups run in a lane-dependent order),
    and the maximum is shared by 32 rows spread over every lm_head workgroup: row 5 or row 9 wins."""
    cfg = dz.Config.small(n_layers=4, max_ctx=32)
    om = oracle.Model(cfg, SEED)
    t = named_tensors(oracle, om, cfg, SEED)
    V, H = cfg.vocab, cfg.hidden
    out = t["output.weight"][1].reshape(V, H // 128, 18).copy()
    pat = out[0].copy()
    neg = pat.copy()
    neg[:, 2:] ^= 0xFF  # flip the 16 sign bytes of every block, keep the f16 scale
    out[:] = 0  # zero scales (and signs): logit 0
    out[5::64] = pat
    out[9::64] = neg
    t["output.weight"] = (dz.GGUF_Q1_0, out.reshape(-1))
    m = dz.Model.from_tensors(cfg, t)
    ctx = dz.Context(m)
    assert ctx.token_kernel == (launch_path == "token_kernel")
    for tok in (3, 1500, 77):
        am, lg = ctx.forward_single_token(tok)
        a, b = lg[5::64], lg[9::64]
        assert np.all(a == a[0]) and np.all(b == b[0])
        rest = np.delete(lg, np.r_[5:V:64, 9:V:64])
        assert np.all(rest == 0)
        assert a[0] != b[0]
        want = 5 if a[0] > b[0] else 9
        assert am == want, (tok, am, a[0], b[0])
    # the device greedy loop's own pick (every workgroup's candidates merged on the device)
    got = ctx.decode_greedy(5, 3)
    assert all(int(x) in (5, 9) for x in got)
    assert int(np.argmax(ctx.logits())) == int(got[-1])


@pytest.mark.parametrize("d", [1, 2, 3])
def test_kv_truncate_keeps_conv_rings(dz, oracle, d):
    """KvCache::truncate (kv_cache.rs:119-130) drops cached positions only; each DeltaNet layer's
    conv ring head (SsmState::conv_head) stays where it was, whatever the truncation."""
    cfg = dz.Config.small(n_layers=4, max_ctx=64)
    m = dz.Model.synthetic(cfg, SEED)
    ctx = dz.Context(m)
    om = oracle.Model(cfg, SEED)
    toks = [9, 8, 7, 6, 5, 4, 3, 2, 1]
    for t in toks:
        ctx.forward_single_token(t, want_logits=False)
        om.forward(t, want_logits=False)
    heads_before = [ctx.get_ssm_state(l)[2] for l in range(3)]
    n = len(toks) - d
    ctx.kv_truncate(n)
    om.kv_truncate(n)
    assert ctx.pos == om.pos == n
    assert [ctx.get_ssm_state(l)[2] for l in range(3)] == heads_before
    for t in (100, 200):
        am, lg = ctx.forward_single_token(t)
        oam, olg = om.forward(t)
        assert normwise_rel(lg, olg) < 1e-3 and am == oam
    for l in range(3):
        sg, cg, hg = ctx.get_ssm_state(l)
        so, co, ho = om.get_ssm_state(l)
        assert hg == ho and normwise_rel(sg, so) < 1e-3 and normwise_rel(cg, co) < 1e-5, l
    kg, vg = ctx.get_kv(3, ctx.pos)
    ko, vo = om.get_kv(3)
    assert ko.shape[1] == ctx.pos
    assert normwise_rel(kg, ko) < 1e-5 and normwise_rel(vg, vo) < 1e-5


def test_decode_greedy_eos_stop(dz, oracle, launch_path):
    """engine.rs:850-871: the loop ends on a sampled eos_token_id before forwarding it."""
    cfg = dz.Config.small(n_layers=4, max_ctx=96)
    m = dz.Model.synthetic(cfg, SEED + 1)
    ctx = dz.Context(m)
    om = oracle.Model(cfg, SEED + 1)
    prompt = [3, 1, 4, 1, 5]
    ctx.forward_batch(np.array(prompt, np.uint32))
    for t in prompt:
        first, _ = om.forward(t, want_logits=False)
    seq = _oracle_greedy(om, first, 40)
    j = next(i for i in range(6, 40) if seq[i] not in seq[:i])  # a token that first appears at step j
    eos = seq[j]
    p0 = ctx.pos
    got = ctx.decode_greedy_eos(first, 40, eos)
    assert list(got) == seq[: j + 1]
    assert ctx.pos == p0 + j + 1
    # the context holds the logits of the last forward, and the eos id was not forwarded
    om2 = oracle.Model(cfg, SEED + 1)
    for t in prompt + [first] + seq[: j]:
        _, olg = om2.forward(t)
    assert om2.pos == ctx.pos
    assert normwise_rel(ctx.logits(), olg) < 1e-3
    am, lg = ctx.forward_single_token(11)
    oam, olg = om2.forward(11)
    assert normwise_rel(lg, olg) < 1e-3 and am == oam
    # no EOS within n: n forwards, like dz_decode_greedy; first == eos: nothing runs
    got = ctx.decode_greedy_eos(am, 4, -1)
    assert len(got) == 4 and ctx.pos == om2.pos + 4
    p1 = ctx.pos
    assert len(ctx.decode_greedy_eos(eos, 4, eos)) == 0 and ctx.pos == p1


def test_failed_wait_poisons_context(dz, oracle, monkeypatch, tmp_path):
    """A launch whose bounded waits give up (forced from the host with a tiny spin limit, so every
    kernel still exits normally) fails with DZ_ERR_DEVICE and leaves the context refusing forwards
    until dz_ctx_reset; after the reset it matches the oracle again."""
    cfg = dz.Config.small(n_layers=4, max_ctx=64)
    m = dz.Model.synthetic(cfg, SEED + 2)
    ctx = dz.Context(m)
    assert ctx.token_kernel
    ctx.forward_single_token(1, want_logits=False)
    monkeypatch.setenv("DAIZA_PTK_SPIN", "1")
    with pytest.raises(dz.DaizaError) as e:
        ctx.decode_greedy(2, 8)
    assert e.value.code == dz.DZ_ERR_DEVICE
    monkeypatch.delenv("DAIZA_PTK_SPIN")
    for call in (lambda: ctx.forward_single_token(3), lambda: ctx.decode_greedy(3, 2),
                 lambda: ctx.forward_batch(np.array([1, 2], np.uint32)), lambda: ctx.verify_forward([1, 2]),
                 lambda: ctx.save(str(tmp_path / "poisoned.dzss"))):
        with pytest.raises(dz.DaizaError) as e:
            call()
        assert e.value.code == dz.DZ_ERR_DEVICE
    import os
    assert not os.path.exists(str(tmp_path / "poisoned.dzss")) or os.path.getsize(str(tmp_path / "poisoned.dzss")) == 0
    ctx.reset()
    om = oracle.Model(cfg, SEED + 2)
    for t in (1, 2, 3):
        am, lg = ctx.forward_single_token(t)
        oam, olg = om.forward(t)
        assert normwise_rel(lg, olg) < 1e-3 and am == oam


@pytest.mark.parametrize("embd_f16", [1, 0])
def test_model_from_gguf_file(dz, oracle, tmp_path, embd_f16):
    """A GGUF file of the synthetic model (tests/gguf_writer.py) through GgufFile::open,
    Config::from_metadata and LoadedWeights::load_all (dz_gguf_open, dz_gguf_config,
    dz_model_create_gguf): the same logits as dz_model_create_synth bit for bit, and as the oracle."""
    from gguf_writer import model_metadata, model_tensors, write_gguf
    cfg = dz.Config.small(n_layers=4, max_ctx=32, embd_f16=embd_f16)
    om = oracle.Model(cfg, SEED)
    path = str(tmp_path / "model.gguf")
    write_gguf(path, model_metadata(cfg) + [("general.alignment", 10, 64)],
               model_tensors(named_tensors(oracle, om, cfg, SEED), cfg), alignment=64)
    g = dz.GgufFile(path)
    gcfg, eos = g.config(max_ctx=32)
    for name, _ in dz.Config._fields_:
        assert getattr(gcfg, name) == pytest.approx(getattr(cfg, name)), name
    m_file = g.model(gcfg)
    g.close()
    m_synth = dz.Model.synthetic(cfg, SEED)
    c_file, c_synth = dz.Context(m_file), dz.Context(m_synth)
    for t in (5, 2047, 0, 731):
        a1, l1 = c_file.forward_single_token(t)
        a2, l2 = c_synth.forward_single_token(t)
        ao, lo = om.forward(t)
        assert np.array_equal(l1, l2), t
        assert normwise_rel(l1, lo) < 1e-3 and a1 == a2 == ao, t


def test_copy_state_checkpoint_restore(dz, oracle, launch_path):
    """ModelState::clone through dz_ctx_copy_state: a checkpoint taken into a spare context after a
    prefill and 4 greedy tokens; the original runs 5 more tokens, is restored from the checkpoint and
    runs the same 5 again with bit-identical logits; the checkpoint's own continuation agrees, and the
    oracle given the same tokens agrees within 1e-3."""
    cfg = dz.Config.small(n_layers=8, max_ctx=96)
    m = dz.Model.synthetic(cfg, SEED + 5)
    a = dz.Context(m)
    prompt = [int(t) for t in np.random.default_rng(11).integers(0, cfg.vocab, 10)]
    lg = a.forward_batch(np.array(prompt, np.uint32))
    first = int(np.argmax(lg))
    toks = [int(t) for t in a.decode_greedy(first, 4)]
    slot = dz.Context(m)
    slot.forward_batch(np.array([1, 2, 3], np.uint32))  # some other state, replaced by the copy
    slot.copy_state_from(a)
    assert slot.pos == a.pos == 14
    assert np.array_equal(slot.logits(), a.logits())
    for l in range(cfg.n_layers):
        if cfg.is_full_attention(l):
            ka, va = a.get_kv(l, a.pos)
            ks, vs = slot.get_kv(l, slot.pos)
            assert np.array_equal(ka, ks) and np.array_equal(va, vs)
        else:
            sa, ca, ha = a.get_ssm_state(l)
            ss, cs, hs = slot.get_ssm_state(l)
            assert np.array_equal(sa, ss) and np.array_equal(ca, cs) and ha == hs

    def run(ctx, n=5):
        out, t = [], toks[-1]
        for _ in range(n):
            t, lgt = ctx.forward_single_token(t)
            out.append(lgt)
        return out

    cont = run(a)
    a.copy_state_from(slot)  # restore
    assert a.pos == 14
    again = run(a)
    from_slot = run(slot)
    for i in range(5):
        assert np.array_equal(again[i], cont[i]) and np.array_equal(from_slot[i], cont[i]), i
    om = oracle.Model(cfg, SEED + 5)
    for t in prompt + [first] + toks[:-1]:
        om.forward(t)
    _, olg = om.forward(toks[-1])
    assert normwise_rel(cont[0], olg) < 1e-3


def test_copy_state_across_shapes_and_paths(dz, oracle, monkeypatch):
    """A copy into a context with a larger max_ctx, from the token kernel to the per-kernel graph
    path, continues like the source; copies between different model shapes, or of a position that
    does not fit the destination, are refused and leave the destination unchanged."""
    cfg = dz.Config.small(n_layers=4, max_ctx=64)
    m = dz.Model.synthetic(cfg, SEED + 6)
    a = dz.Context(m)
    assert a.token_kernel
    a.forward_batch(np.array([7, 8, 9, 10, 11], np.uint32))
    big = dz.Config.small(n_layers=4, max_ctx=128)
    monkeypatch.setenv("DAIZA_PTK", "0")
    mb = dz.Model.synthetic(big, SEED + 6)  # the same weights, a longer cache
    b = dz.Context(mb)
    monkeypatch.delenv("DAIZA_PTK")
    assert not b.token_kernel
    b.copy_state_from(a)
    assert b.pos == 5
    ta, la = a.forward_single_token(12)
    tb, lb = b.forward_single_token(12)
    assert ta == tb and normwise_rel(lb, la) < 1e-5
    # refusals
    other = dz.Context(dz.Model.synthetic(dz.Config.small(n_layers=8, max_ctx=64), SEED))
    with pytest.raises(dz.DaizaError) as e:
        other.copy_state_from(a)
    assert e.value.code == dz.DZ_ERR_MODEL
    small = dz.Context(dz.Model.synthetic(dz.Config.small(n_layers=4, max_ctx=8), SEED))
    small.forward_single_token(3)
    long_ctx = dz.Context(m)
    long_ctx.forward_batch(np.arange(20, dtype=np.uint32))
    with pytest.raises(dz.DaizaError) as e:
        small.copy_state_from(long_ctx)
    assert e.value.code == dz.DZ_ERR_TENSOR
    assert small.pos == 1
