"""DZSS session snapshots on the GPU (dz_ctx_save / dz_ctx_load; Session::save_to_disk and
load_from_disk, session_persist.rs:70-312, format v1).

The file layout is checked by a reader and a writer written here from the format's description
(independent of the library): header fields, history, per-layer blocks (KV as [seq][kv head][dim],
DeltaNet state, conv ring and head), system prompt.  A context restored from a file continues exactly
as the uninterrupted one (bit-identical logits: same kernels, same state) and as the oracle given the
same state (1e-3 normwise); a refused file leaves the context as it was."""
import struct

import numpy as np
import pytest

from conftest import normwise_rel

pytestmark = pytest.mark.gpu

SEED = 0xDA1A0055


def read_dzss(path, cfg):
    """The DZSS v1 file as Python data: (header dict, history, blocks, system prompt or None)."""
    b = open(path, "rb").read()
    assert len(b) >= 128 and b[:4] == b"DZSS"
    ver, h, pos, nh, nb = struct.unpack_from("<IQQQI", b, 4)
    hdr = dict(version=ver, cfg_hash=h, pos=pos, n_history=nh, n_blocks=nb, think=b[36], has_sys=b[37])
    assert b[38:128] == bytes(90)
    off = 128
    hist = np.frombuffer(b, np.uint32, nh, off).copy()
    off += 4 * nh
    blocks = []
    for l in range(nb):
        kind = b[off]
        off += 1
        if kind == 0:
            per_tok, n = struct.unpack_from("<QQ", b, off)
            off += 16
            k = np.frombuffer(b, np.float32, per_tok * n, off).reshape(n, cfg.n_head_kv, cfg.head_dim)
            off += 4 * per_tok * n
            v = np.frombuffer(b, np.float32, per_tok * n, off).reshape(n, cfg.n_head_kv, cfg.head_dim)
            off += 4 * per_tok * n
            blocks.append((0, k.transpose(1, 0, 2).copy(), v.transpose(1, 0, 2).copy()))
        else:
            assert kind == 1
            (sn,) = struct.unpack_from("<Q", b, off)
            off += 8
            st = np.frombuffer(b, np.float32, sn, off).reshape(cfg.ssm_v_heads, cfg.ssm_state, cfg.ssm_state).copy()
            off += 4 * sn
            (cn,) = struct.unpack_from("<Q", b, off)
            off += 8
            conv = np.frombuffer(b, np.float32, cn, off).copy()
            off += 4 * cn
            (head,) = struct.unpack_from("<Q", b, off)
            off += 8
            blocks.append((1, st, conv, head))
    sys_prompt = None
    if hdr["has_sys"]:
        (n,) = struct.unpack_from("<Q", b, off)
        sys_prompt = b[off + 8:off + 8 + n].decode()
        off += 8 + n
    assert off == len(b), "trailing bytes"
    return hdr, hist, blocks, sys_prompt


def write_dzss(path, cfg_hash, pos, history, blocks, think=False, system_prompt=None, n_blocks=None, version=1):
    """A DZSS v1 file from Python data, laid out as save_to_disk writes it (blocks as read_dzss
    returns them: KV in the cache's [kv head][seq][dim])."""
    hdr = bytearray(128)
    hdr[:4] = b"DZSS"
    struct.pack_into("<IQQQI", hdr, 4, version, cfg_hash, pos, len(history), len(blocks) if n_blocks is None else n_blocks)
    hdr[36] = int(think)
    hdr[37] = int(system_prompt is not None)
    out = [bytes(hdr), np.asarray(history, np.uint32).tobytes()]
    for blk in blocks:
        if blk[0] == 0:
            k, v = blk[1], blk[2]
            out += [b"\0", struct.pack("<QQ", k.shape[0] * k.shape[2], k.shape[1]),
                    np.ascontiguousarray(k.transpose(1, 0, 2), np.float32).tobytes(),
                    np.ascontiguousarray(v.transpose(1, 0, 2), np.float32).tobytes()]
        else:
            st, conv, head = blk[1], blk[2], blk[3]
            out += [b"\1", struct.pack("<Q", st.size), np.asarray(st, np.float32).tobytes(),
                    struct.pack("<Q", conv.size), np.asarray(conv, np.float32).tobytes(), struct.pack("<Q", head)]
    if system_prompt is not None:
        sp = system_prompt.encode()
        out += [struct.pack("<Q", len(sp)), sp]
    with open(path, "wb") as f:
        f.write(b"".join(out))


def _state_blocks(ctx, cfg):
    out = []
    for l in range(cfg.n_layers):
        if cfg.is_full_attention(l):
            k, v = ctx.get_kv(l, ctx.pos)
            out.append((0, k, v))
        else:
            st, conv, head = ctx.get_ssm_state(l)
            out.append((1, st, conv.reshape(-1), head))
    return out


@pytest.fixture(scope="module")
def small(dz):
    cfg = dz.Config.small(n_layers=8, max_ctx=96)
    return cfg, dz.Model.synthetic(cfg, SEED)


def test_save_matches_the_format_and_restores_exactly(dz, oracle, small, tmp_path):
    cfg, m = small
    ctx = dz.Context(m)
    prompt = [int(t) for t in np.random.default_rng(1).integers(0, cfg.vocab, 12)]
    lg = ctx.forward_batch(np.array(prompt, np.uint32))
    toks = ctx.decode_greedy(int(np.argmax(lg)), 5)
    history = prompt + [int(np.argmax(lg))] + [int(t) for t in toks[:-1]]
    p = str(tmp_path / "s.dzss")
    ctx.save(p, history=history, think_enabled=True, system_prompt="You are terse. é")

    hdr, hist, blocks, sp = read_dzss(p, cfg)
    assert hdr == dict(version=1, cfg_hash=dz.session_cfg_hash(cfg), pos=ctx.pos, n_history=len(history),
                       n_blocks=cfg.n_layers, think=1, has_sys=1)
    assert list(hist) == history and sp == "You are terse. é"
    for l, (want, got) in enumerate(zip(_state_blocks(ctx, cfg), blocks)):
        assert want[0] == got[0], l
        for a, b in zip(want[1:], got[1:]):
            assert np.array_equal(np.asarray(a), np.asarray(b)), l

    # uninterrupted continuation vs the restored context
    nxt = int(toks[-1])
    ref = []
    t = nxt
    for _ in range(4):
        am, lgt = ctx.forward_single_token(t)
        ref.append(lgt)
        t = am
    c2 = dz.Context(m)
    c2.forward_batch(np.array([7, 8, 9], np.uint32))  # some other state, replaced by the load
    h2, think, sp2 = c2.load(p)
    assert list(h2) == history and think and sp2 == "You are terse. é"
    assert c2.pos == hdr["pos"]
    t = nxt
    for i in range(4):
        am, lgt = c2.forward_single_token(t)
        assert np.array_equal(lgt, ref[i]), i
        t = am

    # the oracle given the file's state agrees with the restored context
    om = oracle.Model(cfg, SEED)
    om.set_pos(hdr["pos"])
    for l, blk in enumerate(blocks):
        if blk[0] == 0:
            om.set_kv(l, blk[1], blk[2])
        else:
            om.set_ssm_state(l, blk[1], blk[2].reshape(cfg.ssm_conv_kernel, cfg.qkv_dim), blk[3])
    c3 = dz.Context(m)
    c3.load(p)
    am, lgt = c3.forward_single_token(nxt)
    oam, olg = om.forward(nxt)
    assert normwise_rel(lgt, olg) < 1e-3 and am == oam


def test_load_of_a_file_written_from_python(dz, oracle, small, tmp_path):
    """A file laid out by write_dzss (seeded state, ring head 2, no system prompt) restores that state
    exactly, and the next forward matches the oracle on it."""
    cfg, m = small
    rng = np.random.default_rng(3)
    pos = 20
    blocks = []
    for l in range(cfg.n_layers):
        if cfg.is_full_attention(l):
            blocks.append((0, rng.standard_normal((cfg.n_head_kv, pos, cfg.head_dim), dtype=np.float32),
                           rng.standard_normal((cfg.n_head_kv, pos, cfg.head_dim), dtype=np.float32)))
        else:
            blocks.append((1, (rng.standard_normal((cfg.ssm_v_heads, cfg.ssm_state, cfg.ssm_state)) * 0.02)
                           .astype(np.float32),
                           (rng.standard_normal(cfg.ssm_conv_kernel * cfg.qkv_dim) * 0.1).astype(np.float32), 2))
    p = str(tmp_path / "py.dzss")
    write_dzss(p, dz.session_cfg_hash(cfg), pos, [1, 2, 3], blocks)
    ctx = dz.Context(m)
    hist, think, sp = ctx.load(p)
    assert list(hist) == [1, 2, 3] and not think and sp is None and ctx.pos == pos
    om = oracle.Model(cfg, SEED)
    om.set_pos(pos)
    for l, blk in enumerate(blocks):
        if blk[0] == 0:
            k, v = ctx.get_kv(l, pos)
            assert np.array_equal(k, blk[1]) and np.array_equal(v, blk[2])
            om.set_kv(l, blk[1], blk[2])
        else:
            st, conv, head = ctx.get_ssm_state(l)
            assert np.array_equal(st, blk[1]) and np.array_equal(conv.reshape(-1), blk[2]) and head == 2
            om.set_ssm_state(l, blk[1], blk[2].reshape(cfg.ssm_conv_kernel, cfg.qkv_dim), 2)
    am, lg = ctx.forward_single_token(11)
    oam, olg = om.forward(11)
    assert normwise_rel(lg, olg) < 1e-3 and am == oam
    # saving it again gives the same bytes
    p2 = str(tmp_path / "py2.dzss")
    c2 = dz.Context(m)
    c2.load(p)
    c2.save(p2, history=[1, 2, 3])
    assert open(p, "rb").read() == open(p2, "rb").read()


def test_fresh_context_writes_empty_conv_history(dz, small, tmp_path):
    """A state that has seen no token has an empty conv history in the reference (conv_len 0); such a
    file loads as zero rings."""
    cfg, m = small
    ctx = dz.Context(m)
    p = str(tmp_path / "fresh.dzss")
    ctx.save(p)
    hdr, hist, blocks, sp = read_dzss(p, cfg)
    assert hdr["pos"] == 0 and hdr["n_history"] == 0 and hdr["has_sys"] == 0
    for l, blk in enumerate(blocks):
        if blk[0] == 0:
            assert blk[1].shape[1] == 0
        else:
            assert blk[2].size == 0 and blk[3] == 0 and not blk[1].any()
    c2 = dz.Context(m)
    c2.forward_batch(np.array([4, 5], np.uint32))
    c2.load(p)
    assert c2.pos == 0
    a = dz.Context(m)
    am1, lg1 = a.forward_single_token(9)
    am2, lg2 = c2.forward_single_token(9)
    assert np.array_equal(lg1, lg2)


def test_refused_files_leave_the_context_unchanged(dz, small, tmp_path):
    cfg, m = small
    ctx = dz.Context(m)
    ctx.forward_batch(np.array([5, 6, 7, 8], np.uint32))
    p = str(tmp_path / "ok.dzss")
    ctx.save(p, history=[5, 6, 7, 8])
    good = open(p, "rb").read()
    other = dz.Config.small(n_layers=4, max_ctx=96)
    cases = {
        "magic": b"DZSX" + good[4:],
        "version": good[:4] + struct.pack("<I", 2) + good[8:],
        "cfg_hash": good[:8] + struct.pack("<Q", dz.session_cfg_hash(other)) + good[16:],
        "blocks": good[:32] + struct.pack("<I", 7) + good[36:],
        "kind": None,
        "truncated": good[:-40],
        "short_header": good[:100],
    }
    # first block kind byte (layer 0 is DeltaNet: kind 1) turned into 0
    kind_off = 128 + 4 * 4
    cases["kind"] = good[:kind_off] + b"\0" + good[kind_off + 1:]
    assert good[kind_off] == 1
    state0 = _state_blocks(ctx, cfg)
    for name, blob in cases.items():
        q = tmp_path / (name + ".dzss")
        q.write_bytes(blob)
        with pytest.raises(dz.DaizaError):
            ctx.load(str(q))
        assert ctx.pos == 4, name
    with pytest.raises(dz.DaizaError):
        ctx.load(p, context_length=4096)  # another Config::context_length: another cfg_hash
    with pytest.raises(dz.DaizaError):
        ctx.load(str(tmp_path / "missing.dzss"))
    for a, b in zip(state0, _state_blocks(ctx, cfg)):
        for x, y in zip(a[1:], b[1:]):
            assert np.array_equal(np.asarray(x), np.asarray(y))
    # too small a history buffer is refused before the context changes
    with pytest.raises(dz.DaizaError):
        ctx.load(p, history_cap=2)
    assert ctx.pos == 4


def test_history_length_is_bounded_before_allocation(dz, small, tmp_path):
    """A header whose n_history is 2^62 (or anything beyond the bytes that follow it) is refused
    with DZ_ERR_MODEL before any allocation, and the context is left as it was."""
    cfg, m = small
    ctx = dz.Context(m)
    ctx.forward_batch(np.array([5, 6, 7], np.uint32))
    p = str(tmp_path / "ok.dzss")
    ctx.save(p, history=[5, 6, 7])
    good = open(p, "rb").read()
    for name, nh in (("huge", 2 ** 62), ("past_2_32", 2 ** 32 + 1), ("past_the_file", len(good) // 4)):
        q = tmp_path / (name + ".dzss")
        q.write_bytes(good[:24] + struct.pack("<Q", nh) + good[32:])
        with pytest.raises(dz.DaizaError) as e:
            ctx.load(str(q))
        assert e.value.code == dz.DZ_ERR_MODEL, name
        assert ctx.pos == 3, name
    am0, lg0 = ctx.forward_single_token(9)
    c2 = dz.Context(m)
    c2.load(p)
    am1, lg1 = c2.forward_single_token(9)
    assert np.array_equal(lg0, lg1)


def test_full_context_round_trip(dz, small, tmp_path):
    """A context filled to max_ctx saves and restores (position max_ctx is a valid, full state;
    forwards there are refused), and a refused forward leaves the restored state intact."""
    cfg, m = small
    ctx = dz.Context(m)
    rng = np.random.default_rng(5)
    ctx.forward_batch(rng.integers(0, cfg.vocab, cfg.max_ctx).astype(np.uint32))
    assert ctx.pos == cfg.max_ctx
    p = str(tmp_path / "full.dzss")
    ctx.save(p, history=list(range(cfg.max_ctx)))
    c2 = dz.Context(m)
    c2.forward_batch(np.array([1, 2], np.uint32))
    hist = c2.load(p)[0]
    assert c2.pos == cfg.max_ctx and list(hist) == list(range(cfg.max_ctx))
    for a, b in zip(_state_blocks(ctx, cfg), _state_blocks(c2, cfg)):
        for x, y in zip(a[1:], b[1:]):
            assert np.array_equal(np.asarray(x), np.asarray(y))
    with pytest.raises(dz.DaizaError) as e:
        c2.forward_single_token(3)
    assert e.value.code == dz.DZ_ERR_TENSOR
    c2.save(str(tmp_path / "again.dzss"), history=list(range(cfg.max_ctx)))
    assert open(p, "rb").read() == open(str(tmp_path / "again.dzss"), "rb").read()
