"""CPU tests of the GGUF reader (dz_gguf_*, host code of libdaiza_hip.so; no GPU call): the
committed tests/golden/tiny.gguf against hand-derived expected values, round trips of files written
by tests/gguf_writer.py, Config::from_metadata (model/config.rs:76-160), and malformed files.
Reference: GgufFile::open (gguf/parser.rs:40-119), metadata.rs, tensor_info.rs:41-201."""
import os
import struct

import numpy as np
import pytest

from gguf_writer import ARR, F32, F64, I32, STR, U8, U16, U32, U64, I8, I16, I64, BOOL, model_metadata, write_gguf

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def dz():
    import daiza_amd
    if not os.path.exists(daiza_amd.LIB_PATH):
        pytest.fail("libdaiza_hip.so is not built; run __graft_entry__.build()")
    return daiza_amd


def test_tiny_golden_file(dz):
    """tests/golden/tiny.gguf (tests/golden/make_tiny_gguf.py): header 704 bytes (11 metadata entries,
    3 tensor infos) padded to the u64 alignment 64; tensors at 704, 896, 1920."""
    g = dz.GgufFile(os.path.join(HERE, "golden", "tiny.gguf"))
    t = g.tensors()
    assert [x[0] for x in t] == ["blk.0.ffn_up.weight", "output_norm.weight", "token_embd.weight"]
    assert [x[1] for x in t] == [41, 0, 1]
    assert [x[2] for x in t] == [(256, 4), (256,), (256, 3)]
    assert [x[3] for x in t] == [704, 896, 1920]
    assert [x[4] for x in t] == [144, 1024, 1536]
    assert np.array_equal(g.tensor_bytes(0), ((7 * np.arange(144) + 3) & 0xFF).astype(np.uint8))
    assert np.array_equal(g.tensor_bytes(1).view(np.float32), (0.5 + np.arange(256) / 256.0).astype(np.float32))
    assert np.array_equal(g.tensor_bytes(2).view(np.float16), ((np.arange(768) % 17) - 8).astype(np.float16))
    cfg, eos = g.config(max_ctx=77)
    assert (cfg.n_layers, cfg.hidden, cfg.max_ctx) == (2, 256, 77)
    assert cfg.rms_eps == pytest.approx(1e-5)
    assert cfg.ffn == 17408 and cfg.vocab == 248320 and eos == 248046  # absent keys keep the defaults
    assert cfg.embd_f16 == 1  # token_embd.weight is F16
    g.close()


def test_every_metadata_type_and_alignment(dz, tmp_path):
    md = [("general.architecture", STR, "qwen35"), ("general.alignment", U64, 128),
          ("a.u8", U8, 200), ("a.i8", I8, -5), ("a.u16", U16, 60000), ("a.i16", I16, -300), ("a.u32", U32, 7),
          ("a.i32", I32, -7), ("a.f32", F32, 1.5), ("a.bool", BOOL, False), ("a.u64", U64, 1 << 40),
          ("a.i64", I64, -(1 << 40)), ("a.f64", F64, 2.5),
          ("a.arr_u8", ARR, (U8, [1, 2, 3])), ("a.arr_str", ARR, (STR, ["x", "yy", ""])),
          ("a.arr_f32", ARR, (F32, [0.5, -1.0])), ("a.empty", ARR, (I32, []))]
    rng = np.random.default_rng(0)
    q = rng.integers(0, 256, 18 * 3 * 5, dtype=np.uint8)  # 5 rows x 384 columns of Q1_0
    f = rng.standard_normal(33).astype(np.float32)
    tensors = [("m.q", 41, (384, 5), q.tobytes()), ("m.f", 0, (33,), f.tobytes()),
               ("m.other", 8, (32,), bytes(34))]  # Q8_0: not sized by this path
    p = str(tmp_path / "a.gguf")
    data = write_gguf(p, md, tensors, alignment=128)
    g = dz.GgufFile(p)
    t = g.tensors()
    assert [x[2] for x in t] == [(384, 5), (33,), (32,)]
    assert all(x[3] % 128 == 0 for x in t)
    assert t[0][4] == q.size and t[1][4] == 132 and t[2][4] == 0
    assert np.array_equal(g.tensor_bytes(0), q)
    assert np.array_equal(g.tensor_bytes(1).view(np.float32), f)
    assert g.tensor_bytes(2) is None
    assert data[t[0][3]:t[0][3] + q.size] == q.tobytes()


def test_u32_alignment_is_ignored_like_the_reference(dz, tmp_path):
    """GgufFile::open reads general.alignment with Metadata::get_u64, which returns None for a u32
    value: the data section then starts at a multiple of 32 whatever the u32 key says."""
    q = np.arange(18 * 4, dtype=np.uint8)
    md = [("general.architecture", STR, "qwen35"), ("general.alignment", U32, 256)]
    p = str(tmp_path / "b.gguf")
    write_gguf(p, md, [("m.q", 41, (128, 4), q.tobytes())], alignment=32)
    g = dz.GgufFile(p)
    (name, ty, dims, off, nb), = g.tensors()
    assert off % 32 == 0 and off % 256 != 0
    assert np.array_equal(g.tensor_bytes(0), q)


def test_config_from_metadata(dz, tmp_path):
    cfg = dz.Config.small(n_layers=8, max_ctx=100)
    p = str(tmp_path / "c.gguf")
    write_gguf(p, model_metadata(cfg, eos=42), [("token_embd.weight", 41, (cfg.hidden, cfg.vocab),
                                                 bytes(cfg.vocab * cfg.hidden // 128 * 18))])
    g = dz.GgufFile(p)
    got, eos = g.config(max_ctx=100)
    for name, _ in dz.Config._fields_:
        want = 0 if name == "embd_f16" else getattr(cfg, name)  # a Q1_0 token embedding
        assert getattr(got, name) == pytest.approx(want), name
    assert eos == 42
    # string tokens (real files) leave the default vocabulary, as the reference reads them
    p2 = str(tmp_path / "d.gguf")
    md = [m for m in model_metadata(cfg) if m[0] != "tokenizer.ggml.tokens"]
    md.append(("tokenizer.ggml.tokens", ARR, (STR, ["<a>", "<b>"])))
    write_gguf(p2, md, [])
    assert dz.GgufFile(p2).config()[0].vocab == 248320
    p3 = str(tmp_path / "e.gguf")
    write_gguf(p3, [("general.architecture", STR, "llama")], [])
    with pytest.raises(dz.DaizaError) as e:
        dz.GgufFile(p3).config()
    assert e.value.code == dz.DZ_ERR_MODEL


def test_malformed_files_are_refused(dz, tmp_path):
    good = open(os.path.join(HERE, "golden", "tiny.gguf"), "rb").read()
    cases = {
        "magic": b"GGUG" + good[4:],
        "version": good[:4] + (2).to_bytes(4, "little") + good[8:],
        "truncated_header": good[:300],
        "truncated_data": good[:-100],
        "empty": b"",
    }
    for name, blob in cases.items():
        p = tmp_path / (name + ".gguf")
        p.write_bytes(blob)
        with pytest.raises(dz.DaizaError) as e:
            dz.GgufFile(str(p))
        assert e.value.code == dz.DZ_ERR_MODEL, name
    with pytest.raises(dz.DaizaError):
        dz.GgufFile(str(tmp_path / "missing.gguf"))


def _one_tensor_file(dims, ty, offset=0):
    """A GGUF v3 file whose single tensor info declares `dims` of type `ty` at `offset`, followed
    by 64 data bytes: the declared size is whatever the dims say."""
    def s(x):
        b = x.encode()
        return struct.pack("<Q", len(b)) + b
    out = bytearray(b"GGUF") + struct.pack("<IQQ", 3, 1, 1)
    out += s("general.architecture") + struct.pack("<I", STR) + s("qwen35")
    out += s("t") + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
    out += struct.pack("<IQ", ty, offset)
    out += bytes((-len(out)) % 32) + bytes(64)
    return bytes(out)


def test_sizes_that_overflow_are_refused(dz, tmp_path):
    """Declared tensor sizes are computed without wrapping: an F32 tensor of 2^62 - 2 elements
    (4 x that is 2^64 - 8, which wraps below the file size), an element count whose dims product
    passes 2^64, and an offset near 2^64 are refused, where the reference fails on its slice bounds;
    a tensor that fits is read."""
    cases = {
        "f32_bytes_wrap": _one_tensor_file([2 ** 62 - 2], 0),
        "dims_product_wraps": _one_tensor_file([2 ** 33, 2 ** 33], 1),
        "offset_wraps": _one_tensor_file([4], 0, offset=2 ** 64 - 8),
        "past_the_end": _one_tensor_file([17], 0),
    }
    for name, blob in cases.items():
        p = tmp_path / (name + ".gguf")
        p.write_bytes(blob)
        with pytest.raises(dz.DaizaError) as e:
            dz.GgufFile(str(p))
        assert e.value.code == dz.DZ_ERR_MODEL, name
    p = tmp_path / "fits.gguf"
    p.write_bytes(_one_tensor_file([16], 0))
    (name, ty, dims, off, nb), = dz.GgufFile(str(p)).tensors()
    assert (name, ty, nb) == ("t", 0, 64)
