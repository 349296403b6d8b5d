"""GPU parity of the decode path against the CPU oracle.

Small hybrid stacks (hidden 512, same per-head shapes as Bonsai-27B) run in seconds on the
oracle, so every output is compared elementwise; full-size layers (configs 2 and 3) are
compared for one step.  Bar: 1e-3 normwise relative error for hidden state, SSM state and
logits; greedy tokens identical.
"""
import numpy as np
import pytest

from conftest import normwise_rel

pytestmark = pytest.mark.gpu

SEED = 0xDA1A0004
K_STATE, K_CONV, K_KV, K_X = 65, 66, 67, 64


def _pair(dz, oracle, cfg, seed=SEED):
    m = dz.Model.synthetic(cfg, seed)
    ctx = dz.Context(m)
    om = oracle.Model(cfg, seed)
    return m, ctx, om


def test_small_forward_logits_and_argmax(dz, oracle):
    cfg = dz.Config.small(n_layers=4, max_ctx=64)
    m, ctx, om = _pair(dz, oracle, cfg)
    toks = [5, 17, 2047, 0, 999, 1234, 7, 7, 42, 1000]
    for i, t in enumerate(toks):
        am, lg = ctx.forward_single_token(t)
        oam, olg = om.forward(t)
        err = normwise_rel(lg, olg)
        assert err < 1e-3, (i, err)
        assert am == oam, (i, am, oam, err)
    assert ctx.pos == om.pos == len(toks)


def test_f16_embedding_subnormal_rows(dz, oracle):
    """Tokens whose f16 embedding row holds subnormal halves: the row converts with the
    reference's f16_to_f32 (tensor/tensor.rs:62-76, quant.rs:39-74) on the GPU as in the oracle."""
    cfg = dz.Config.small(n_layers=1, max_ctx=16)
    toks = []
    for t in range(cfg.vocab):
        row = oracle.synth_embd_row_f16(SEED, t, cfg.hidden)
        if np.any(((row & 0x7C00) == 0) & ((row & 0x3FF) != 0)):
            toks.append(t)
        if len(toks) == 3:
            break
    assert toks, "no token with a subnormal embedding element in this vocabulary"
    for t in toks:
        m, ctx, om = _pair(dz, oracle, cfg)
        _, lg = ctx.forward_single_token(t)
        _, olg = om.forward(t)
        assert normwise_rel(lg, olg) < 1e-4, t


def test_small_decode_greedy_tokens(dz, oracle):
    cfg = dz.Config.small(n_layers=8, max_ctx=128)
    m, ctx, om = _pair(dz, oracle, cfg, seed=SEED + 1)
    prompt = [3, 1, 4, 1, 5, 9, 2, 6]
    last = ctx.forward_batch(prompt)
    for t in prompt:
        oam, olg = om.forward(t)
    assert normwise_rel(last, olg) < 1e-3
    n = 48
    got = ctx.decode_greedy(oam, n)
    want = []
    tok = oam
    for _ in range(n):
        tok, _ = om.forward(tok, want_logits=False)
        want.append(tok)
    assert list(got) == want


def test_small_batch_per_position_logits(dz, oracle):
    cfg = dz.Config.small(n_layers=4, max_ctx=64)
    m, ctx, om = _pair(dz, oracle, cfg, seed=SEED + 2)
    ids = [11, 22, 33, 44, 55]
    per = ctx.forward_batch(ids, per_pos_logits=True)
    for i, t in enumerate(ids):
        _, olg = om.forward(t)
        assert normwise_rel(per[i], olg) < 1e-3


@pytest.mark.parametrize("full", [False, True])
def test_deltanet_step(dz, oracle, full):
    # one Gated DeltaNet step with random recurrent and conv state
    if full:
        cfg = dz.Config.bonsai27b(max_ctx=64)
        cfg.n_layers, cfg.vocab = 1, 64
    else:
        cfg = dz.Config.small(n_layers=1, max_ctx=64)
    m, ctx, om = _pair(dz, oracle, cfg, seed=SEED + 3)
    nvh, hd = cfg.ssm_v_heads, cfg.ssm_state
    state = oracle.synth_normal(SEED, K_STATE, 0, nvh * hd * hd, sigma=0.02).reshape(nvh, hd, hd)
    conv = oracle.synth_normal(SEED, K_CONV, 0, 4 * cfg.qkv_dim, sigma=0.1).reshape(4, cfg.qkv_dim)
    for pos, head in ((0, 0), (7, 2)):
        ctx.set_pos(pos)
        om.set_pos(pos)
        ctx.set_ssm_state(0, state, conv, head)
        om.set_ssm_state(0, state, conv, head)
        h = oracle.synth_normal(SEED, K_X, pos, cfg.hidden)
        for step in range(3):
            hg = ctx.mixer_step(0, h)
            ho = om.mixer_step(0, h)
            assert normwise_rel(hg, ho) < 1e-3, step
            sg, cg, headg = ctx.get_ssm_state(0)
            so, co, heado = om.get_ssm_state(0)
            assert headg == heado
            assert normwise_rel(sg, so) < 1e-3
            assert normwise_rel(cg, co) < 1e-5
            h = ho


@pytest.mark.parametrize("ctxlen", [1, 100, 300, 4096, 5000, 32768])
def test_attention_step(dz, oracle, ctxlen):
    # one gated attention step over an N(0,1) KV cache of length ctxlen
    cfg = dz.Config.bonsai27b(max_ctx=ctxlen + 8)
    cfg.n_layers, cfg.vocab, cfg.full_attn_interval = 1, 64, 1
    m, ctx, om = _pair(dz, oracle, cfg, seed=SEED + 4)
    kvn = cfg.n_head_kv * (ctxlen - 1) * cfg.head_dim
    k = oracle.synth_normal(SEED, K_KV, 0, kvn).reshape(cfg.n_head_kv, ctxlen - 1, cfg.head_dim)
    v = oracle.synth_normal(SEED, K_KV, 1, kvn).reshape(cfg.n_head_kv, ctxlen - 1, cfg.head_dim)
    ctx.set_kv(0, k, v)
    om.set_kv(0, k, v)
    ctx.set_pos(ctxlen - 1)
    om.set_pos(ctxlen - 1)
    h = oracle.synth_normal(SEED, K_X, 9, cfg.hidden)
    for step in range(2):
        hg = ctx.mixer_step(0, h)
        ho = om.mixer_step(0, h)
        assert normwise_rel(hg, ho) < 1e-3, step
        h = ho
    kg, vg = ctx.get_kv(0, ctxlen + 1)
    ko, vo = om.get_kv(0)
    assert ko.shape[1] == ctxlen + 1
    assert normwise_rel(kg[:, -2:], ko[:, -2:]) < 1e-3
    assert normwise_rel(vg[:, -2:], vo[:, -2:]) < 1e-3


@pytest.fixture
def graph_path(monkeypatch):
    """Contexts created while this fixture is active replay the per-kernel token graph."""
    monkeypatch.setenv("DAIZA_PTK", "0")


def test_token_kernel_is_default_for_supported_shapes(dz):
    for cfg in (dz.Config.small(n_layers=4, max_ctx=64), dz.Config.bonsai27b(max_ctx=64)):
        if cfg.n_layers == 64:
            cfg.n_layers = 4  # a 4-layer stack of the 27B shapes: same kernel instance, less memory
        m = dz.Model.synthetic(cfg, SEED)
        ctx = dz.Context(m)
        assert ctx.token_kernel, cfg.hidden
        ctx.close()
        m.close()


def test_graph_path_matches_oracle(dz, oracle, graph_path):
    cfg = dz.Config.small(n_layers=4, max_ctx=64)
    m, ctx, om = _pair(dz, oracle, cfg, seed=SEED + 7)
    assert not ctx.token_kernel
    for t in [5, 17, 2047, 0, 999, 1234]:
        am, lg = ctx.forward_single_token(t)
        oam, olg = om.forward(t)
        assert normwise_rel(lg, olg) < 1e-3
        assert am == oam
    got = ctx.decode_greedy(am, 24)
    want, tok = [], am
    for _ in range(24):
        tok, _ = om.forward(tok, want_logits=False)
        want.append(tok)
    assert list(got) == want


@pytest.mark.parametrize("L", [300, 3000, 5000])
def test_token_kernel_long_context(dz, oracle, L):
    """The token kernel's attention chunks at long contexts (several rounds of cache reads per wave:
    up to 10 positions per wave at L = 5000) against the oracle: N(0,1) cache of length L."""
    cfg = dz.Config.small(n_layers=4, max_ctx=L + 16)
    m, ctx, om = _pair(dz, oracle, cfg, seed=SEED + 11)
    assert ctx.token_kernel
    kvn = cfg.n_head_kv * L * cfg.head_dim
    k = oracle.synth_normal(SEED, K_KV, 2, kvn).reshape(cfg.n_head_kv, L, cfg.head_dim)
    v = oracle.synth_normal(SEED, K_KV, 3, kvn).reshape(cfg.n_head_kv, L, cfg.head_dim)
    ctx.set_kv(3, k, v)
    om.set_kv(3, k, v)
    ctx.set_pos(L)
    om.set_pos(L)
    for t in (5, 1234, 77):
        am, lg = ctx.forward_single_token(t)
        oam, olg = om.forward(t)
        assert normwise_rel(lg, olg) < 1e-3, t
        assert am == oam


def test_token_kernel_and_graph_agree(dz, monkeypatch):
    """The two launch paths compute the same per-position logits (small stack, 20 tokens)."""
    cfg = dz.Config.small(n_layers=8, max_ctx=64)
    ids = np.random.default_rng(3).integers(0, cfg.vocab, 20).astype(np.uint32)
    out = {}
    for path in ("1", "0"):
        monkeypatch.setenv("DAIZA_PTK", path)
        m = dz.Model.synthetic(cfg, SEED + 9)
        ctx = dz.Context(m)
        assert ctx.token_kernel == (path == "1")
        out[path] = ctx.forward_batch(ids, per_pos_logits=True)
        out[path + "g"] = ctx.decode_greedy(int(np.argmax(out[path][-1])), 16)
        ctx.close()
        m.close()
    for i in range(len(ids)):
        assert normwise_rel(out["1"][i], out["0"][i]) < 1e-5, i
    assert list(out["1g"]) == list(out["0g"])


def test_traced_token_kernel_matches(dz, tmp_path, monkeypatch):
    """DAIZA_PTK_TRACE runs the traced instances (ptk_trace.hip), a kernel of their own beside the
    production one: the same greedy and sampled tokens and generator state, the same logits, and a
    trace file of n_tok x phases x workgroups x slots stamps: every workgroup stamps each token's
    selection (phase 0) and lm_head (the last phase), in that order, token after token."""
    cfg = dz.Config.small(n_layers=8, max_ctx=96)
    m = dz.Model.synthetic(cfg, SEED + 11)
    a, b = dz.Context(m), dz.Context(m)
    assert a.token_kernel and b.token_kernel
    prompt = np.random.default_rng(5).integers(0, cfg.vocab, 12).astype(np.uint32)
    first = int(np.argmax(a.forward_batch(prompt)))
    b.forward_batch(prompt)
    path = tmp_path / "trace.bin"
    ra, rb = dz.LcgRng(31), dz.LcgRng(31)
    sp = dz.SamplingParams(0.9, 20, 0.9)
    ga = a.decode_greedy(first, 6)
    sa = a.decode_sample(int(ga[-1]), 5, sp, ra)
    monkeypatch.setenv("DAIZA_PTK_TRACE", str(path))
    try:
        gb = b.decode_greedy(first, 6)
        sb = b.decode_sample(int(gb[-1]), 5, sp, rb)
    finally:
        monkeypatch.delenv("DAIZA_PTK_TRACE")
    assert list(ga) == list(gb) and list(sa) == list(sb)
    assert ra.state.value == rb.state.value
    assert normwise_rel(a.logits(), b.logits()) < 1e-6
    data = path.read_bytes()
    off = 0
    for n_expect in (6, 5):
        n, ppt, G, S = np.frombuffer(data[off:off + 16], np.int32)
        assert n == n_expect and S == 8
        off += 16
        t = np.frombuffer(data[off:off + 8 * n * ppt * G * S], np.uint64).reshape(n, ppt, G, S)
        off += 8 * n * ppt * G * S
        ends = np.stack([t[:, 0, :, 0], t[:, ppt - 1, :, 0]], axis=1).astype(np.int64)  # [token][S, LM][wg]
        assert (ends > 0).all()
        seq = ends.transpose(2, 0, 1).reshape(G, 2 * n)  # per workgroup: S0, LM0, S1, LM1, ...
        assert (np.diff(seq, axis=1) > 0).all()
    assert off == len(data)
