"""CPU tests that pin the oracle (oracle/oracle.c) before it is trusted as the GPU's checker.

The reference holds no golden vectors for this path and its Rust sources cannot be built here,
so every oracle function is pinned by something other than itself: hand-derived known answers,
numpy's IEEE conversions, closed forms, invariants, float64 brute force, and an independent
float64 restatement of the whole decode step (tests/npref.py).
"""
import math
import struct

import numpy as np
import pytest

import npref

SEED = 0xDA1A0001


def f32_bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


# ---------------------------------------------------------------- f16 -> f32 (quant.rs:39-108)

def test_f16_normals_zero_inf_match_ieee(oracle):
    """Every half that is not subnormal or NaN converts exactly as IEEE binary16 does."""
    L = oracle.lib()
    allbits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    exp = (allbits >> 10) & 0x1F
    mant = allbits & 0x3FF
    sel = allbits[~((exp == 0) & (mant != 0)) & ~((exp == 31) & (mant != 0))]
    ieee = sel.view(np.float16).astype(np.float32).view(np.uint32)
    got = np.array([L.or_f16_to_f32_bits(int(b)) for b in sel], np.uint32)
    assert np.array_equal(got, ieee)


@pytest.mark.parametrize("half,expect", [
    # subnormals, worked by hand through quant.rs:50-61: e starts at 1 and grows with each shift
    (0x0001, 0x3D800000),  # 10 shifts: e = 11, exponent 112 + 11 = 123 -> 2^-4 (IEEE: 2^-24)
    (0x8001, 0xBD800000),
    (0x0003, 0x3D400000),  # 9 shifts: e = 10, mantissa 0b1 << 9 -> 1.5 * 2^-5
    (0x0200, 0x39000000),  # 1 shift: e = 2 -> 2^-13 (IEEE: 2^-15)
    (0x03FF, 0x397FC000),  # 1 shift: e = 2, mantissa 0x3FE
    # Inf / NaN keep the payload shifted into place, no quieting (quant.rs:64-67)
    (0x7C00, 0x7F800000), (0xFC00, 0xFF800000),
    (0x7C01, 0x7F802000), (0x7DFF, 0x7FBFE000), (0xFE00, 0xFFC00000),
    (0x0000, 0x00000000), (0x8000, 0x80000000),
    (0x7BFF, 0x477FE000), (0x3C00, 0x3F800000),
])
def test_f16_known_answers(oracle, half, expect):
    assert oracle.lib().or_f16_to_f32_bits(half) == expect


def test_f16_subnormal_closed_form(oracle):
    """All 2046 subnormal halves: quirk value == IEEE value * 2^(20 - 2p), p = leading bit."""
    L = oracle.lib()
    bits = np.array([m | s for s in (0, 0x8000) for m in range(1, 1024)], np.uint16)
    got = np.array([L.or_f16_to_f32(int(b)) for b in bits], np.float64)
    assert np.array_equal(got, npref.f16_ref_quirk(bits))


def test_f16_fast_subnormals(oracle):
    """quant.rs:86-108: exponent field 0 gives f32 exponent 0 with the mantissa kept, i.e. the
    f32 denormal (sign | mant << 13) -- about mant * 2^-136, not the +-0 its comment promises."""
    L = oracle.lib()
    for b in list(range(0, 1024, 7)) + [0x8001, 0x83FF]:
        want = ((b & 0x8000) << 16) | ((b & 0x3FF) << 13)
        assert f32_bits(L.or_f16_to_f32_fast(b)) == want
    assert f32_bits(L.or_f16_to_f32_fast(0x0007)) == 0x0000E000
    for b in range(0x0400, 0x10000, 97):
        if (b & 0x7C00) == 0:
            continue
        assert f32_bits(L.or_f16_to_f32_fast(b)) == f32_bits(L.or_f16_to_f32(b))


def test_f32_to_f16_matches_numpy(oracle):
    """The generator's f32 -> f16 (round to nearest even) against numpy, incl. ties and overflow."""
    L = oracle.lib()
    rng = np.random.default_rng(3)
    xs = np.concatenate([rng.normal(0, 1, 3000) * 0.02, rng.normal(0, 1, 1000) * 1e4,
                         rng.normal(0, 1, 1000) * 1e-6,
                         [0.0, -0.0, 65504.0, 65520.0, 65519.99, 1e9, -1e9, 2.0 ** -25, 2.0 ** -24,
                          3 * 2.0 ** -25, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11]]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    got = np.array([L.or_f32_to_f16(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- dequant (quant.rs:161-194)

def _blocks(scales, sign_bytes):
    out = bytearray()
    for sc, sb in zip(scales, sign_bytes):
        out += struct.pack("<H", sc) + bytes(sb)
    return np.frombuffer(bytes(out), np.uint8).copy()


def test_dequant_all_sign_bytes_and_scales(oracle):
    """All 256 sign bytes in every position, against numpy's unpackbits and the closed form
    w = bit ? +s : -s (quant.rs:136-141), s via the reference's f16_to_f32."""
    scales = [0x2A1F, 0x0001, 0x03FF, 0x0000, 0x8000, 0x7BFF, 0xFBFF, 0x7C00, 0x3C00, 0x1400]
    for sc in scales:
        rows = 16  # 16 rows x 1 block: byte value b sits at position (b % 16) of row b // 16
        sb = [[(r * 16 + (p + r) % 16) % 256 for p in range(16)] for r in range(rows)]
        aos = _blocks([sc] * rows, sb)
        got = oracle.dequant_rows(aos, rows, 128)
        s = float(npref.f16_ref_quirk(np.array([sc], np.uint16))[0])
        bits = np.unpackbits(np.array(sb, np.uint8), axis=1, bitorder="little")
        want = np.where(bits == 1, np.float32(s), np.float32(-s)).astype(np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), hex(sc)


def test_dequant_negative_zero(oracle):
    """(bit*2-1) * +0.0 gives -0.0 for a clear bit and +0.0 for a set bit."""
    aos = _blocks([0x0000], [[0x0F] * 16])
    got = oracle.dequant_rows(aos, 1, 128).view(np.uint32)[0]
    assert got[0] == 0 and got[4] == 0x80000000


def test_dequant_nan_scale(oracle):
    aos = _blocks([0x7E00], [[0xAA] * 16])
    got = oracle.dequant_rows(aos, 1, 128)
    assert np.isnan(got).all()


# ---------------------------------------------------------------- GEMV (quant.rs:614-740, weights.rs:123-465)

def _rand_q1(rng, rows, cols, scale_sigma=0.02):
    g = cols // 128
    aos = np.empty((rows, g, 18), np.uint8)
    sc = np.abs(rng.normal(0, 1, (rows, g)) * scale_sigma).astype(np.float16)
    aos[:, :, 0:2] = sc.view(np.uint8).reshape(rows, g, 2)
    aos[:, :, 2:] = rng.integers(0, 256, (rows, g, 16), dtype=np.uint8)
    return aos.reshape(-1)


@pytest.mark.parametrize("rows,cols", [(8, 256), (64, 1024), (1031, 640), (2050, 5120)])
def test_gemv_vs_float64(oracle, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    aos = _rand_q1(rng, rows, cols)
    x = rng.normal(0, 1, cols).astype(np.float32)
    W = npref.dequant_ieee(aos, rows, cols)
    want = W @ x.astype(np.float64)
    y = oracle.matvec(aos, rows, cols, x)
    # f32 accumulation over cols/8 terms per lane: error well below 1e-5 relative (norm-wise)
    assert np.linalg.norm(y - want) / np.linalg.norm(want) < 2e-6
    bound = np.abs(W) @ np.abs(x) * (cols * 1.2e-7)
    assert np.all(np.abs(y - want) <= bound)


@pytest.mark.parametrize("rows", [4, 5, 6, 7, 128, 1027, 2048 + 3])
def test_gemv_scalar_statement_bit_exact(oracle, rows):
    """The AVX2 quad kernel + work-stealing chunks and the lane-by-lane scalar statement agree
    bit for bit (both follow the reference FMA order; tails use triple/dual/single)."""
    cols = 640
    rng = np.random.default_rng(rows)
    aos = _rand_q1(rng, rows, cols)
    x = rng.normal(0, 1, cols).astype(np.float32)
    a = oracle.matvec(aos, rows, cols, x, nthreads=1)
    b = oracle.matvec_scalar(aos, rows, cols, x)
    if rows >= 1024:
        c = oracle.matvec(aos, rows, cols, x, nthreads=8)
        assert np.array_equal(a.view(np.uint32), c.view(np.uint32))
        # 128-row chunks make every chunk a whole number of quads, as in the reference
        assert np.array_equal(a[: rows // 4 * 4].view(np.uint32), b[: rows // 4 * 4].view(np.uint32))
    else:
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_gemv_sign_invariants(oracle):
    """All-ones sign bits give s*sum(x); all-zeros give -s*sum(x)."""
    rows, cols = 8, 512
    rng = np.random.default_rng(11)
    x = rng.normal(0, 1, cols).astype(np.float32)
    for fill, sgn in ((0xFF, 1.0), (0x00, -1.0)):
        aos = _rand_q1(rng, rows, cols).reshape(rows, cols // 128, 18)
        aos[:, :, 2:] = fill
        sc = np.ascontiguousarray(aos[:, :, 0:2]).view(np.float16)[..., 0].astype(np.float64)
        want = sgn * (sc * x.astype(np.float64).reshape(-1, 128).sum(1)).sum(1)
        y = oracle.matvec(aos.reshape(-1), rows, cols, x)
        assert np.allclose(y, want, rtol=1e-5, atol=1e-6)


def test_gemv_basis_columns_exact(oracle):
    """x = e_k picks column k of the IEEE dequant exactly (every other product is a signed zero)."""
    rows, cols = 12, 384
    rng = np.random.default_rng(5)
    aos = _rand_q1(rng, rows, cols)
    W = npref.dequant_ieee(aos, rows, cols).astype(np.float32)
    for k in (0, 1, 7, 8, 127, 128, 200, 383):
        x = np.zeros(cols, np.float32)
        x[k] = 1.0
        y = oracle.matvec(aos, rows, cols, x)
        assert np.array_equal(y, W[:, k]), k


def test_gemv_linearity_and_accumulate(oracle):
    rows, cols = 256, 1024
    rng = np.random.default_rng(6)
    aos = _rand_q1(rng, rows, cols)
    x1 = rng.normal(0, 1, cols).astype(np.float32)
    x2 = rng.normal(0, 1, cols).astype(np.float32)
    y1, y2 = oracle.matvec(aos, rows, cols, x1), oracle.matvec(aos, rows, cols, x2)
    y12 = oracle.matvec(aos, rows, cols, (2 * x1 + x2).astype(np.float32))
    assert np.linalg.norm(y12 - (2 * y1 + y2)) / np.linalg.norm(y12) < 1e-6
    base = rng.normal(0, 1, rows).astype(np.float32)
    acc = oracle.matvec(aos, rows, cols, x1, y=base.copy(), accumulate=True)
    assert np.array_equal(acc, (base + y1).astype(np.float32))


# ---------------------------------------------------------------- transcendental glue (simd_exp.rs)

def test_exp_ps_accuracy_and_clamp(oracle):
    x = np.linspace(-87.0, 87.0, 40000).astype(np.float32)  # whole 8-lane vectors
    y = oracle.vec_op("or_exp_ps", x)
    rel = np.abs(y.astype(np.float64) / np.exp(x.astype(np.float64)) - 1.0)
    assert rel.max() < 5e-6  # degree-5 Taylor on |r| <= ln2/2
    big = np.array([88.0, 100.0, 1e30, np.inf, -88.0, -100.0, -np.inf, 0.0], np.float32)
    yb = oracle.vec_op("or_exp_ps", big)
    assert yb[0] == yb[1] == yb[2] == yb[3]          # clamp at +88
    assert yb[4] == yb[5] == yb[6] and yb[4] > 0      # clamp at -88, no underflow to 0
    assert yb[7] == 1.0
    assert oracle.lib().or_exp_fast(0.5) == oracle.vec_op("or_exp_ps", np.full(8, 0.5, np.float32))[0]


def test_sigmoid_silu_accuracy(oracle):
    x = np.linspace(-30, 30, 8000).astype(np.float32)
    s = oracle.vec_op("or_sigmoid_ps", x).astype(np.float64)
    ref = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    assert np.max(np.abs(s - ref) / ref) < 2e-5  # rcp + one Newton step
    si = oracle.vec_op("or_silu_ps", x).astype(np.float64)
    assert np.allclose(si, x * ref, rtol=2e-5, atol=1e-30)
    assert abs(oracle.lib().or_sigmoid_fast(0.0) - 0.5) < 1e-7
    # swiglu = silu(g) * u
    g = np.linspace(-6, 6, 37).astype(np.float32)
    u = np.linspace(2, -2, 37).astype(np.float32)
    gg = g.copy()
    oracle.lib().or_swiglu(oracle._f(gg), oracle._f(u), gg.size)
    assert np.allclose(gg, g / (1 + np.exp(-g.astype(np.float64))) * u, rtol=2e-5, atol=1e-7)


def test_rmsnorm_and_l2norm(oracle):
    rng = np.random.default_rng(8)
    for n in (5120, 256, 128, 37):
        x = rng.normal(0, 3, n).astype(np.float32)
        w = rng.uniform(0.8, 1.2, n).astype(np.float32)
        y = np.empty_like(x)
        oracle.lib().or_rmsnorm_into(oracle._f(x), oracle._f(y), oracle._f(w), n, 1e-6)
        want = npref.rmsnorm(x.astype(np.float64), w.astype(np.float64), 1e-6)
        assert np.allclose(y, want, rtol=3e-6, atol=0)
        # constant input c with unit weights -> c / sqrt(c^2 + eps)
        c = np.full(n, 0.25, np.float32)
        one = np.ones(n, np.float32)
        oracle.lib().or_rmsnorm_into(oracle._f(c), oracle._f(y), oracle._f(one), n, 1e-6)
        assert np.allclose(y, 0.25 / math.sqrt(0.0625 + 1e-6), rtol=1e-6)
        z = x.copy()
        oracle.lib().or_l2norm_inplace(oracle._f(z), n, 1e-6)
        assert abs(np.linalg.norm(z.astype(np.float64)) - 1.0) < 1e-5
        assert np.allclose(z, x / np.linalg.norm(x.astype(np.float64)), rtol=1e-5)


def test_argmax_ties_and_nan(oracle):
    L = oracle.lib()
    x = np.array([1.0, 3.0, 3.0, -1.0, 3.0], np.float32)
    assert L.or_argmax(oracle._f(x), x.size) == 1
    x = np.array([np.nan, 2.0, np.nan, 2.0], np.float32)
    assert L.or_argmax(oracle._f(x), x.size) == 1
    x = np.full(1000, -np.inf, np.float32)
    assert L.or_argmax(oracle._f(x), x.size) == 0
    x = np.arange(10000, dtype=np.float32)
    x[7777] = 1e9
    assert L.or_argmax(oracle._f(x), x.size) == 7777


# ---------------------------------------------------------------- RoPE (rope.rs)

def test_rope_freqs_and_identity(oracle):
    import ctypes
    L = oracle.lib()
    fr = np.empty(32, np.float32)
    L.or_rope_freqs(64, 1.0e7, oracle._f(fr))
    want = 1.0 / np.power(1.0e7, np.arange(0, 64, 2) / 64.0)
    assert np.allclose(fr, want, rtol=2e-6)
    assert fr[0] == 1.0
    co, si = np.empty(64, np.float32), np.empty(64, np.float32)
    L.or_rope_cos_sin(0, oracle._f(fr), 64, oracle._f(co), oracle._f(si))
    assert np.all(co == 1.0) and np.all(si == 0.0)
    x = np.random.default_rng(1).normal(0, 1, 256).astype(np.float32)
    y = x.copy()
    L.or_rope_partial(oracle._f(y), 64, oracle._f(co), oracle._f(si))
    assert np.array_equal(x, y)
    del ctypes


def test_rope_quirk_basis_kat(oracle):
    """Pairs (i, i+32) rotate as [[c, s], [s, c]] (rope.rs:205-208, both '+'), dims >= 64 untouched."""
    L = oracle.lib()
    fr = np.empty(32, np.float32)
    L.or_rope_freqs(64, 1.0e7, oracle._f(fr))
    co, si = np.empty(64, np.float32), np.empty(64, np.float32)
    pos = 1000
    L.or_rope_cos_sin(pos, oracle._f(fr), 64, oracle._f(co), oracle._f(si))
    th = np.float32(pos) * fr
    assert np.allclose(co[:32], np.cos(th.astype(np.float64)), atol=2e-7)
    assert np.allclose(si[:32], np.sin(th.astype(np.float64)), atol=2e-7)
    assert np.array_equal(co[:32], co[32:]) and np.array_equal(si[:32], si[32:])
    for i in (0, 5, 31):
        for j, partner in ((i, i + 32), (i + 32, i)):
            x = np.zeros(256, np.float32)
            x[j] = 1.0
            x[100] = 7.0
            L.or_rope_partial(oracle._f(x), 64, oracle._f(co), oracle._f(si))
            assert x[j] == co[i % 32] and x[partner] == si[i % 32] and x[100] == 7.0


# ---------------------------------------------------------------- DeltaNet scan (ssm.rs:153-180, 378-418)

def _scan(oracle, S, q, k, v, a, al, be, dt):
    S = np.ascontiguousarray(S, np.float32).copy()
    y = np.empty(128, np.float32)
    f = oracle._f
    oracle.lib().or_ssm_scan_vhead(f(S), f(y), f(np.ascontiguousarray(q, np.float32)),
                                   f(np.ascontiguousarray(k, np.float32)), f(np.ascontiguousarray(v, np.float32)),
                                   a, al, be, dt, 128)
    return S, y


def test_scan_vs_float64(oracle):
    rng = np.random.default_rng(9)
    S0 = rng.normal(0, 0.02, (128, 128))
    q, k, v = rng.normal(0, 0.1, 128), rng.normal(0, 0.1, 128), rng.normal(0, 1, 128)
    a, al, be, dt = -0.7, 0.3, -0.4, 0.05
    S, y = _scan(oracle, S0, q, k, v, a, al, be, dt)
    decay = np.exp(a * np.log1p(np.exp(al + dt)))
    beta = 1 / (1 + np.exp(-be))
    Sd = S0 * decay
    Sw = Sd + np.outer((v - Sd @ k) * beta, k)
    assert np.allclose(S, Sw, rtol=1e-5, atol=1e-7)
    assert np.allclose(y, Sw @ q, rtol=1e-4, atol=1e-7)


def test_scan_closed_cases(oracle):
    rng = np.random.default_rng(10)
    S0 = rng.normal(0, 0.02, (128, 128)).astype(np.float32)
    q, k, v = rng.normal(0, 0.1, 128), rng.normal(0, 0.1, 128), rng.normal(0, 1, 128)
    # beta -> 0 (b = -100 saturates the sigmoid): S = decay * S, y = S q
    S, y = _scan(oracle, S0, q, k, v, -0.5, 0.2, -100.0, 0.0)
    decay = np.float32(np.exp(np.float32(-0.5) * np.float32(np.log1p(np.exp(0.2)))))
    assert np.allclose(S, S0 * decay, rtol=2e-6)
    assert np.allclose(y, (S0 * decay).astype(np.float64) @ q, rtol=1e-4, atol=1e-8)
    # decay = 1 (ssm_a = 0) and S = 0: S = beta v k^T, y = beta v (k . q)
    Z = np.zeros((128, 128), np.float32)
    S, y = _scan(oracle, Z, q, k, v, 0.0, 0.2, 0.3, 0.0)
    beta = 1 / (1 + np.exp(-0.3))
    assert np.allclose(S, beta * np.outer(v, k), rtol=2e-5, atol=1e-9)
    assert np.allclose(y, beta * v * (k @ q), rtol=1e-4, atol=1e-8)


def test_lcg_known_answers(oracle):
    """sampling.rs:9-19: 64-bit LCG, top 24 bits of state >> 40, divided by 2^24."""
    import ctypes
    st = ctypes.c_uint64(0xC0FFEE)
    s = 0xC0FFEE
    for _ in range(20):
        s = (s * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        want = ((s >> 40) & 0xFFFFFF) / float(1 << 24)
        assert oracle.lib().or_lcg_next(ctypes.byref(st)) == np.float32(want)
    assert st.value == s


# ---------------------------------------------------------------- synthetic generator (daiza_synth.h)

def test_synth_deterministic_and_distributed(oracle):
    a = oracle.synth_q1_0(SEED, 18, 3, 512, 1024)
    b = oracle.synth_q1_0(SEED, 18, 3, 512, 1024)
    c = oracle.synth_q1_0(SEED, 18, 4, 512, 1024)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    # a row range generated alone equals the same rows of the whole matrix
    part = oracle.synth_q1_0(SEED, 18, 3, 100, 1024, r0=200)
    rb = 8 * 18
    assert np.array_equal(part, a[200 * rb:300 * rb])
    blk = a.reshape(-1, 18)
    bits = np.unpackbits(blk[:, 2:])
    assert abs(bits.mean() - 0.5) < 0.005
    sc = np.ascontiguousarray(blk[:, :2]).view(np.float16)[:, 0].astype(np.float64)
    assert np.all(sc >= 0)
    assert abs(sc.mean() - 0.02 * math.sqrt(2 / math.pi)) < 0.0005  # E|N(0,1)| * 0.02
    x = oracle.synth_normal(SEED, 64, 0, 200000)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    x2 = oracle.synth_normal(SEED, 64, 0, 1000, i0=500)
    assert np.array_equal(x2, x[500:1500])


# ---------------------------------------------------------------- whole decode step vs float64

@pytest.fixture(scope="module")
def small_pair(oracle):
    import daiza_amd as dz
    cfg = dz.Config.small(n_layers=4, max_ctx=64)
    om = oracle.Model(cfg, SEED, nthreads=4)
    yield cfg, om
    om.close()


def test_decode_tokens_vs_float64(oracle, small_pair):
    """Six tokens through the 4-layer hybrid stack (3 DeltaNet + 1 attention layer): logits, SSM
    state and KV cache against the float64 restatement."""
    cfg, om = small_pair
    om.new_ctx()
    ref = npref.NpDecoder(om, cfg, SEED)
    for t in (5, 17, 2047, 0, 999, 5):
        am, lo = om.forward(t)
        want = ref.forward(t)
        err = np.linalg.norm(lo - want) / np.linalg.norm(want)
        assert err < 1e-5, err
        if np.sort(want)[-1] - np.sort(want)[-2] > 1e-3 * np.abs(want).max():
            assert am == int(np.argmax(want))
    for l in range(cfg.n_layers):
        if cfg.is_full_attention(l):
            k, v = om.get_kv(l)
            assert k.shape[1] == 6
            assert np.allclose(k, ref.K[l], rtol=1e-4, atol=1e-5)
            assert np.allclose(v, ref.V[l], rtol=1e-4, atol=1e-5)
        else:
            st, conv, head = om.get_ssm_state(l)
            assert head == ref.head[l]
            assert np.abs(st - ref.S[l]).max() < 1e-5 * max(1.0, np.abs(ref.S[l]).max()) * 10
            assert np.allclose(conv, ref.ring[l], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("layer,conv_head", [(0, 0), (1, 3), (2, 1)])
def test_deltanet_step_seeded_state(oracle, small_pair, layer, conv_head):
    """One DeltaNet step from a seeded state (S ~ N(0, 0.02), conv ~ N(0, 0.1))
    for several ring heads, so that a wrong tap order or ring index shows."""
    cfg, om = small_pair
    om.new_ctx()
    rng = np.random.default_rng(layer)
    hd = cfg.ssm_state
    S0 = rng.normal(0, 0.02, (cfg.ssm_v_heads, hd, hd)).astype(np.float32)
    conv0 = rng.normal(0, 0.1, (cfg.ssm_conv_kernel, cfg.qkv_dim)).astype(np.float32)
    h = rng.normal(0, 1, cfg.hidden).astype(np.float32)
    om.set_ssm_state(layer, S0, conv0, conv_head)
    om.set_pos(7)
    out = om.mixer_step(layer, h)
    ref = npref.NpDecoder(om, cfg, SEED)
    ref.S[layer] = S0.astype(np.float64).copy()
    ref.ring[layer] = conv0.astype(np.float64).copy()
    ref.head[layer] = conv_head
    ref.pos = 7
    want = ref.mixer_step(layer, h)
    assert np.linalg.norm(out - want) / np.linalg.norm(want - h) < 1e-5
    st, conv, head = om.get_ssm_state(layer)
    assert head == (conv_head + 1) % 4
    assert np.abs(st - ref.S[layer]).max() < 1e-6
    assert np.allclose(conv, ref.ring[layer], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("ctx", [0, 1, 50])
def test_attention_step_seeded_kv(oracle, small_pair, ctx):
    """One attention step with ctx cached N(0,1) positions (BASELINE config 3 at small length);
    ctx 0 is the first token, whose output is its own v (softmax over one key)."""
    cfg, om = small_pair
    om.new_ctx()
    layer = 3
    rng = np.random.default_rng(100 + ctx)
    k0 = rng.normal(0, 1, (cfg.n_head_kv, ctx, cfg.head_dim)).astype(np.float32)
    v0 = rng.normal(0, 1, (cfg.n_head_kv, ctx, cfg.head_dim)).astype(np.float32)
    h = rng.normal(0, 1, cfg.hidden).astype(np.float32)
    om.set_kv(layer, k0, v0)
    om.set_pos(ctx)
    out = om.mixer_step(layer, h)
    ref = npref.NpDecoder(om, cfg, SEED)
    ref.K[layer] = k0.astype(np.float64)
    ref.V[layer] = v0.astype(np.float64)
    ref.pos = ctx
    want = ref.mixer_step(layer, h)
    assert np.linalg.norm(out - want) / np.linalg.norm(want - h) < 1e-5
    k, v = om.get_kv(layer)
    assert k.shape[1] == ctx + 1
    assert np.allclose(k[:, -1], ref.K[layer][:, -1], rtol=1e-5, atol=1e-6)
