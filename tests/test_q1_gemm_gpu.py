"""GPU parity of the N-column Q1_0 product (matvec_batch_into_slice, weights.rs:475-682) that
prefill and speculative verify run on the matrix cores.

Bar: every column within 1e-3 normwise relative error of the reference quad kernel
(quant.rs:614-740) applied to that column, and in practice ~1e-7: the weights are exact f16
operands and the activations are carried at f32 width (three f16 parts, 33 significant bits), so
only the f32 accumulation order differs; a full-mantissa input through unit scales comes back bit
for bit.  Closed forms pin the sign convention and the scale handling independently of the oracle.
Cases with n <= 16 run the raw form (each K tile packed in LDS with its own scale per token), the
others the packed form (one scale per token, packed by a separate pass).
"""
import numpy as np
import pytest

from conftest import normwise_rel

pytestmark = pytest.mark.gpu

SEED = 0xDA1A0006
K_GATE = 18  # DZ_K_FFN_GATE stream of daiza_synth.h
K_X = 64     # DZ_K_X


def _xs(oracle, n, cols, layer=0):
    return np.stack([oracle.synth_normal(SEED, K_X, layer, cols, i0=i * cols) for i in range(n)])


@pytest.mark.parametrize("rows,cols,n", [
    (64, 512, 1), (64, 512, 32), (100, 384, 5), (3, 128, 33), (257, 1152, 17),
    (17408, 5120, 8), (5120, 6144, 64), (1030, 5120, 100),
])
def test_batch_vs_oracle(dz, oracle, rows, cols, n):
    aos = oracle.synth_q1_0(SEED, K_GATE, 0, rows, cols)
    m = dz.Q1_0Matrix(aos, rows, cols)
    x = _xs(oracle, n, cols)
    y = m.matvec_batch(x)
    for i in range(n):
        ref = oracle.matvec(aos, rows, cols, x[i])
        err = normwise_rel(y[i], ref)
        assert err < 1e-5, (i, err)


def test_batch_accumulate(dz, oracle):
    rows, cols, n = 5120, 17408, 9
    aos = oracle.synth_q1_0(SEED, K_GATE, 1, rows, cols)
    m = dz.Q1_0Matrix(aos, rows, cols)
    x = _xs(oracle, n, cols, layer=1)
    y0 = _xs(oracle, n, rows, layer=2)
    y = y0.copy()
    m.matvec_add_batch_into_slice(x, n, y)
    for i in range(n):
        ref = oracle.matvec(aos, rows, cols, x[i], y=y0[i].copy(), accumulate=True)
        assert normwise_rel(y[i], ref) < 1e-5


def test_batch_matches_gemv(dz, oracle):
    # the same matrix through the LUT GEMV and the matrix-core product
    rows, cols, n = 6144, 5120, 3
    aos = oracle.synth_q1_0(SEED, K_GATE, 2, rows, cols)
    m = dz.Q1_0Matrix(aos, rows, cols)
    x = _xs(oracle, n, cols, layer=3)
    yb = m.matvec_batch(x)
    for i in range(n):
        assert normwise_rel(yb[i], m.matvec(x[i])) < 1e-5


def _aos_const(rows, cols, sign_byte, scale_bits):
    blk = np.zeros((rows, cols // 128, 18), np.uint8)
    blk[:, :, 0] = scale_bits & 0xFF
    blk[:, :, 1] = scale_bits >> 8
    blk[:, :, 2:] = sign_byte
    return blk.reshape(-1)


@pytest.mark.parametrize("sign_byte,sgn", [(0xFF, 1.0), (0x00, -1.0)])
def test_all_ones_all_zeros(dz, sign_byte, sgn):
    # bits all 1 => y = scale * sum(x); all 0 => y = -scale * sum(x)  (quant.rs:136-141)
    rows, cols, n = 70, 1024, 4
    m = dz.Q1_0Matrix(_aos_const(rows, cols, sign_byte, 0x2E66), rows, cols)  # scale = f16 0.1
    rng = np.random.default_rng(1)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    y = m.matvec_batch(x)
    scale = float(np.float16(0.1))
    want = sgn * scale * x.astype(np.float64).sum(1)
    for i in range(n):
        assert np.allclose(y[i], want[i], rtol=1e-5, atol=1e-5 * np.abs(x[i]).sum() * scale)


def test_basis_columns_and_scales(dz, oracle):
    # x = e_k picks column k of the dequantised matrix; includes negative and subnormal f16 scales
    # (the matrix cores take the f16 scale as is; the GEMV path converts it exactly too)
    rows, cols = 64, 512
    aos = oracle.synth_q1_0(SEED, K_GATE, 4, rows, cols).copy().reshape(rows, cols // 128, 18)
    specials = [0x0001, 0x03FF, 0x8200, 0xBC00, 0x3C00, 0x7BFF]
    for r in range(rows):
        v = specials[r % len(specials)]
        aos[r, r % 4, 0] = v & 0xFF
        aos[r, r % 4, 1] = v >> 8
    aos = aos.reshape(-1)
    m = dz.Q1_0Matrix(aos, rows, cols)
    ks = [0, 1, 7, 8, 127, 128, 200, 300, 511]
    x = np.zeros((len(ks), cols), np.float32)
    for i, k in enumerate(ks):
        x[i, k] = 1.0
    y = m.matvec_batch(x)
    # the exact (IEEE) dequantised columns
    blk = aos.reshape(rows, cols // 128, 18)
    sc = (blk[:, :, 0].astype(np.uint16) | (blk[:, :, 1].astype(np.uint16) << 8)).view(np.float16).astype(np.float32)
    for i, k in enumerate(ks):
        g, b, j = k // 128, (k % 128) // 8, k % 8
        bit = (blk[:, g, 2 + b] >> j) & 1
        want = np.where(bit == 1, sc[:, g], -sc[:, g])
        assert np.array_equal(y[i], want), k


@pytest.mark.parametrize("n", [1, 5, 8, 9, 16, 17, 40])
def test_activations_carried_at_f32_width(dz, n):
    """x = v_i e_k with v_i an f32 whose 24-bit significand has its low bits set, through a
    matrix of unit scales: every output is exactly +-v_i, which a product carrying fewer than 24
    significant bits of the activation (a two-part f16 split keeps 22) would round.  All three
    forms: paired (n <= 8), raw (9..16), packed (> 16)."""
    rows, cols = 128, 1024
    rng = np.random.default_rng(n)
    blk = np.empty((rows, cols // 128, 18), np.uint8)
    blk[:, :, 2:] = rng.integers(0, 256, (rows, cols // 128, 16), dtype=np.uint8)
    blk[:, :, 0], blk[:, :, 1] = 0x00, 0x3C  # f16 1.0
    m = dz.Q1_0Matrix(blk.reshape(-1), rows, cols)
    ks = rng.integers(0, cols, n)
    # significands 1.m with the lowest mantissa bits set; magnitudes over a wide range
    mant = rng.integers(0, 1 << 23, n, dtype=np.int64) | 0x3
    expo = rng.integers(-20, 21, n)
    v = np.ldexp((1.0 + mant / float(1 << 23)), expo).astype(np.float32)
    assert np.all(v.astype(np.float64) == (1.0 + mant / float(1 << 23)) * np.ldexp(1.0, expo))
    x = np.zeros((n, cols), np.float32)
    x[np.arange(n), ks] = v
    y = m.matvec_batch(x)
    for i in range(n):
        k = ks[i]
        g, b, j = k // 128, (k % 128) // 8, k % 8
        bit = (blk[:, g, 2 + b] >> j) & 1
        want = np.where(bit == 1, v[i], -v[i]).astype(np.float32)
        assert np.array_equal(y[i], want), (n, i)


def test_wide_dynamic_range(dz, oracle):
    # per-token power-of-two scaling: rows of very different magnitude keep their own precision
    rows, cols = 256, 2048
    aos = oracle.synth_q1_0(SEED, K_GATE, 5, rows, cols)
    m = dz.Q1_0Matrix(aos, rows, cols)
    x = _xs(oracle, 4, cols, layer=6)
    x[0] *= 3.0e4
    x[1] *= 1.0e-6
    x[2, ::7] *= 100.0
    y = m.matvec_batch(x)
    for i in range(4):
        ref = oracle.matvec(aos, rows, cols, x[i])
        assert normwise_rel(y[i], ref) < 1e-5, i


def test_tiles_of_different_magnitude(dz, oracle):
    # within one token, K tiles 2^20 apart: the raw form scales each tile on its own (n <= 16), the
    # packed form (n = 17) scales the row; both stay within the bar of the reference
    rows, cols = 128, 2048
    aos = oracle.synth_q1_0(SEED, K_GATE, 6, rows, cols)
    m = dz.Q1_0Matrix(aos, rows, cols)
    for n in (2, 17):
        x = _xs(oracle, n, cols, layer=7)
        x[:, :512] *= 1024.0
        x[:, 1536:] *= 1.0 / 1024.0
        y = m.matvec_batch(x)
        for i in range(n):
            ref = oracle.matvec(aos, rows, cols, x[i])
            assert normwise_rel(y[i], ref) < 1e-5, (n, i)
