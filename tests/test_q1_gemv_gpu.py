"""GPU parity of the Q1_0 GEMV and dequant against the CPU oracle.

Bar: dequantised weights bit-exact with the reference's dequantize_q1_0_row_into
(quant.rs:161-194, including its f16_to_f32 at quant.rs:39-74); GEMV outputs within 1e-3
normwise relative error of the reference quad kernel (quant.rs:614-740), in practice ~1e-6.
"""
import numpy as np
import pytest

from conftest import normwise_rel

pytestmark = pytest.mark.gpu

SEED = 0xDA1A0001
K_GATE = 18  # DZ_K_FFN_GATE stream of daiza_synth.h
K_X = 64     # DZ_K_X


def _mat(dz, oracle, rows, cols, layer=0, seed=SEED):
    aos = oracle.synth_q1_0(seed, K_GATE, layer, rows, cols)
    return aos, dz.Q1_0Matrix(aos, rows, cols)


@pytest.mark.parametrize("rows,cols", [(64, 512), (100, 384), (3, 128), (257, 1152), (1030, 5120)])
def test_dequant_bit_exact(dz, oracle, rows, cols):
    aos, m = _mat(dz, oracle, rows, cols)
    got = m.dequant_rows(0, rows)
    ref = oracle.dequant_rows(aos, rows, cols)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_special_scales(dz, oracle):
    # scales: subnormal halves, +-0, max normal, +-inf; reference semantics bit for bit
    rows, cols = 8, 1024
    aos, _ = _mat(dz, oracle, rows, cols)
    aos = aos.copy().reshape(rows, cols // 128, 18)
    specials = [0x0001, 0x03FF, 0x0200, 0x0000, 0x8000, 0x7BFF, 0x7C00, 0xFC00, 0x8001, 0x3C00]
    k = 0
    for r in range(rows):
        for g in range(cols // 128):
            v = specials[k % len(specials)]
            aos[r, g, 0] = v & 0xFF
            aos[r, g, 1] = v >> 8
            k += 1
    aos = aos.reshape(-1)
    m = dz.Q1_0Matrix(aos, rows, cols)
    got = m.dequant_rows(0, rows)
    ref = oracle.dequant_rows(aos, rows, cols)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(17408, 5120), (5120, 17408), (100, 384), (64, 512), (1, 128), (6144, 6144)])
def test_matvec_vs_oracle(dz, oracle, rows, cols):
    aos, m = _mat(dz, oracle, rows, cols)
    x = oracle.synth_normal(SEED, K_X, 0, cols)
    y = m.matvec(x)
    ref = oracle.matvec(aos, rows, cols, x)
    err = normwise_rel(y, ref)
    assert err < 1e-3, err
    assert err < 1e-5, "GEMV drifted far from the reference order: %g" % err


def test_matvec_add(dz, oracle):
    rows, cols = 5120, 6144
    aos, m = _mat(dz, oracle, rows, cols)
    x = oracle.synth_normal(SEED, K_X, 1, cols)
    y0 = oracle.synth_normal(SEED, K_X, 2, rows)
    y = y0.copy()
    m.matvec_add_into_slice(x, y)
    ref = oracle.matvec(aos, rows, cols, x, y=y0.copy(), accumulate=True)
    assert normwise_rel(y, ref) < 1e-5


def test_matvec_multi(dz, oracle):
    cols = 5120
    shapes = [10240, 48, 48, 6144]  # DeltaNet in-proj entries (ssm.rs:449-463)
    aoss, mats, outs = [], [], []
    for i, r in enumerate(shapes):
        a, m = _mat(dz, oracle, r, cols, layer=i)
        aoss.append(a)
        mats.append(m)
        outs.append(np.zeros(r, np.float32))
    x = oracle.synth_normal(SEED, K_X, 3, cols)
    dz.Q1_0Matrix.matvec_multi_into_slice(x, mats, outs)
    for a, r, o in zip(aoss, shapes, outs):
        ref = oracle.matvec(a, r, cols, x)
        assert normwise_rel(o, ref) < 1e-5


def ieee_dequant(aos, rows, cols):
    """w = bit ? +scale : -scale with the IEEE f16 scale (numpy's own conversion)."""
    blk = aos.reshape(rows, cols // 128, 18)
    scale = blk[:, :, :2].copy().view(np.float16)[:, :, 0].astype(np.float32)
    bits = np.unpackbits(blk[:, :, 2:], axis=2, bitorder="little").astype(np.float32)
    return ((bits * 2.0 - 1.0) * scale[:, :, None]).reshape(rows, cols)


def test_matvec_basis_columns_exact(dz, oracle):
    # x = e_k: every table entry is +-1 or +-0, so y must equal column k of the dequantised matrix.
    # The GEMV converts scales exactly (like the quad kernel's _mm256_cvtph_ps), so the
    # comparison uses IEEE f16 scales, not the dequant path's f16_to_f32 (quant.rs:39-74).
    rows, cols = 192, 1536
    aos, m = _mat(dz, oracle, rows, cols)
    W = ieee_dequant(aos, rows, cols)
    for k in (0, 7, 8, 511, 512, 1000, 1535):
        x = np.zeros(cols, np.float32)
        x[k] = 1.0
        y = m.matvec(x)
        assert np.array_equal(y, W[:, k]), k


def test_matvec_subnormal_scales_exact_conversion(dz, oracle):
    # The GEMV converts scales exactly (as _mm256_cvtph_ps in the quad kernel): subnormal
    # scales must give the IEEE value, matching the oracle's quad kernel.
    rows, cols = 64, 512
    aos, _ = _mat(dz, oracle, rows, cols)
    a3 = aos.copy().reshape(rows, cols // 128, 18)
    a3[:, :, 0] = 0x01
    a3[:, :, 1] = 0x02  # 0x0201: subnormal half
    aos2 = a3.reshape(-1)
    m = dz.Q1_0Matrix(aos2, rows, cols)
    x = oracle.synth_normal(SEED, K_X, 4, cols)
    y = m.matvec(x)
    ref = oracle.matvec(aos2, rows, cols, x)
    assert normwise_rel(y, ref) < 1e-5


def _hip():
    import ctypes
    h = ctypes.CDLL("libamdhip64.so")
    h.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    h.hipFree.argtypes = [ctypes.c_void_p]
    h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    h.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    h.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    return h


def test_gemv_give_up_is_reported(dz, oracle, monkeypatch):
    """The one-launch product's bounded wait for its split-K partials, forced to give up from the
    host (DAIZA_GEMV_SPIN=0: every kernel still exits normally), is reported as DZ_ERR_DEVICE by the
    synchronous matvec and by dz_q1_0_matvec_dev_status for the asynchronous form -- never NaN with
    DZ_OK -- and the next calls are correct again."""
    import ctypes
    rows, cols = 1030, 5120
    aos, m = _mat(dz, oracle, rows, cols)
    x = oracle.synth_normal(SEED, K_X, 0, cols)
    ref = oracle.matvec(aos, rows, cols, x)
    L = dz.lib()
    monkeypatch.setenv("DAIZA_GEMV_SPIN", "0")
    with pytest.raises(dz.DaizaError) as e:
        m.matvec(x)
    assert e.value.code == dz.DZ_ERR_DEVICE
    h = _hip()
    dx, dy = ctypes.c_void_p(), ctypes.c_void_p()
    assert h.hipMalloc(ctypes.byref(dx), cols * 4) == 0 and h.hipMalloc(ctypes.byref(dy), rows * 4) == 0
    assert h.hipMemcpy(dx, x.ctypes.data, cols * 4, 1) == 0
    assert L.dz_q1_0_matvec_dev(m._h, dx, dy, 0, None) == 0
    assert L.dz_q1_0_matvec_dev_status(None) == dz.DZ_ERR_DEVICE
    assert L.dz_q1_0_matvec_dev_status(None) == 0  # reported once
    monkeypatch.delenv("DAIZA_GEMV_SPIN")
    assert normwise_rel(m.matvec(x), ref) < 1e-5
    assert L.dz_q1_0_matvec_dev(m._h, dx, dy, 0, None) == 0
    assert L.dz_q1_0_matvec_dev_status(None) == 0
    y = np.empty(rows, np.float32)
    assert h.hipMemcpy(y.ctypes.data, dy, rows * 4, 2) == 0
    assert normwise_rel(y, ref) < 1e-5
    h.hipFree(dx)
    h.hipFree(dy)


def test_gemv_calls_on_two_streams(dz, oracle):
    """Asynchronous products enqueued alternately on two streams (they share one buffer of tagged
    partials) run in call order and each matches the oracle."""
    import ctypes
    rows, cols = 2048, 5120
    L = dz.lib()
    h = _hip()
    mats = [_mat(dz, oracle, rows, cols, layer=i) for i in range(2)]
    x = oracle.synth_normal(SEED, K_X, 1, cols)
    refs = [oracle.matvec(a, rows, cols, x) for a, _ in mats]
    dx = ctypes.c_void_p()
    assert h.hipMalloc(ctypes.byref(dx), cols * 4) == 0
    assert h.hipMemcpy(dx, x.ctypes.data, cols * 4, 1) == 0
    ys, ss = [], []
    for i in range(8):
        p = ctypes.c_void_p()
        assert h.hipMalloc(ctypes.byref(p), rows * 4) == 0
        ys.append(p)
    for _ in range(2):
        s = ctypes.c_void_p()
        assert h.hipStreamCreate(ctypes.byref(s)) == 0
        ss.append(s)
    for i in range(8):
        assert L.dz_q1_0_matvec_dev(mats[i % 2][1]._h, dx, ys[i], 0, ss[i % 2]) == 0
    for s in ss:
        assert L.dz_q1_0_matvec_dev_status(s) == 0
    for i in range(8):
        y = np.empty(rows, np.float32)
        assert h.hipMemcpy(y.ctypes.data, ys[i], rows * 4, 2) == 0
        assert normwise_rel(y, refs[i % 2]) < 1e-5, i
        h.hipFree(ys[i])
    for s in ss:
        h.hipStreamDestroy(s)
    h.hipFree(dx)
