"""CPU tests of the DZSS session format's host pieces (no GPU call): the oracle's SipHash against the
published SipHash-2-4 vectors, then dz_session_cfg_hash (libdaiza_hip.so) against the oracle's
SipHash-1-3 with zero keys over the ten configuration words of cfg_hash (session_persist.rs:52-66).

Rust's DefaultHasher is SipHash-1-3 with keys (0, 0); usize::hash writes the 8 little-endian bytes of
the value, so the hashed message is the 80-byte concatenation of the ten words.  No Rust toolchain is
in the image, so no hash written by the reference itself is available: the pin is the published 2-4
vectors (round function, word packing, length byte, finalisation) plus the c/d round counts."""
import os
import struct

import numpy as np
import pytest

# SipHash-2-4, key 00 01 .. 0f, message 00 01 .. (n-1): the first vectors of the reference
# implementation's vectors.h (Aumasson and Bernstein, github.com/veorq/SipHash)
SIPHASH24_VECTORS = {0: 0x726fdb47dd0e0e31, 1: 0x74f839c593dc67fd, 2: 0x0d6c8009d9a94f5a,
                     3: 0x85676696d7fb7e2d, 8: 0x93f5f5799a932462, 15: 0xa129ca6149be45e5}
K0 = int.from_bytes(bytes(range(8)), "little")
K1 = int.from_bytes(bytes(range(8, 16)), "little")


def test_siphash24_published_vectors(oracle):
    for n, want in SIPHASH24_VECTORS.items():
        assert oracle.siphash(2, 4, K0, K1, bytes(range(n))) == want, n


def test_siphash_round_counts_matter(oracle):
    """1-3 differs from 2-4 and from 1-4 on the same input: the round counts are really applied."""
    m = bytes(range(80))
    hs = {oracle.siphash(c, d, 0, 0, m) for c, d in ((1, 3), (2, 4), (1, 4), (2, 3))}
    assert len(hs) == 4


@pytest.fixture(scope="module")
def dz():
    import daiza_amd
    if not os.path.exists(daiza_amd.LIB_PATH):
        pytest.fail("libdaiza_hip.so is not built; run __graft_entry__.build()")
    return daiza_amd


def _words(cfg, context_length):
    return struct.pack("<10Q", cfg.n_layers, cfg.hidden, cfg.n_head, cfg.n_head_kv, cfg.head_dim,
                       cfg.full_attn_interval, cfg.ssm_state, cfg.ssm_v_heads, cfg.ssm_conv_kernel, context_length)


def test_cfg_hash_is_siphash13_of_the_config_words(dz, oracle):
    for cfg, cl in ((dz.Config.bonsai27b(max_ctx=4096), 262144), (dz.Config.small(n_layers=8), 262144),
                    (dz.Config.bonsai27b(max_ctx=64), 32768)):
        assert dz.session_cfg_hash(cfg, cl) == oracle.siphash(1, 3, 0, 0, _words(cfg, cl))
    a = dz.Config.bonsai27b(max_ctx=4096)
    b = dz.Config.bonsai27b(max_ctx=77)  # max_ctx is not one of the hashed fields
    assert dz.session_cfg_hash(a) == dz.session_cfg_hash(b)
    for field in ("n_layers", "hidden", "n_head", "n_head_kv", "head_dim", "full_attn_interval", "ssm_state",
                  "ssm_v_heads", "ssm_conv_kernel"):
        c = dz.Config.bonsai27b(max_ctx=4096)
        setattr(c, field, getattr(c, field) + 1)
        assert dz.session_cfg_hash(c) != dz.session_cfg_hash(a), field
    assert dz.session_cfg_hash(a, 262143) != dz.session_cfg_hash(a)
