"""dz_q1_0_matvec_dev_noalloc: the same y = W x as dz_q1_0_matvec_dev, through a fixed per-device
workspace instead of a library allocation.  Bit-for-bit equal outputs on two calls in a row (the
second smaller), accumulate included; sizes past the workspace refused; device memory unchanged."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _mat(dz, rows, cols, seed):
    rng = np.random.default_rng(seed)
    blk = np.empty((rows, cols // 128, 18), np.uint8)
    blk[:, :, 2:] = rng.integers(0, 256, (rows, cols // 128, 16), dtype=np.uint8)
    blk[:, :, :2] = (np.abs(rng.standard_normal((rows, cols // 128))) * 0.02).astype(np.float16)[..., None].view(np.uint8)
    return dz.Q1_0Matrix(blk.reshape(-1), rows, cols), rng.standard_normal(cols).astype(np.float32)


class _Hip:
    def __init__(self):
        h = ctypes.CDLL("libamdhip64.so")
        h.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        h.hipFree.argtypes = [ctypes.c_void_p]
        h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        h.hipDeviceSynchronize.argtypes = []
        h.hipMemGetInfo.argtypes = [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]
        self.h = h

    def buf(self, n):
        p = ctypes.c_void_p()
        assert self.h.hipMalloc(ctypes.byref(p), max(4, n)) == 0
        return p

    def put(self, p, a):
        assert self.h.hipMemcpy(p, a.ctypes.data, a.nbytes, 1) == 0

    def get(self, p, n):
        a = np.empty(n, np.float32)
        assert self.h.hipMemcpy(a.ctypes.data, p, a.nbytes, 2) == 0
        return a

    def free_mem(self):
        f, t = ctypes.c_size_t(), ctypes.c_size_t()
        assert self.h.hipMemGetInfo(ctypes.byref(f), ctypes.byref(t)) == 0
        return f.value


def test_noalloc_matches_matvec_dev(dz):
    L = dz.lib()
    H = _Hip()
    # two calls in a row, the second on a smaller matrix (rows not a multiple of 64, three K tiles)
    for rows, cols, seed in ((17408, 5120, 1), (1000, 1536, 2)):
        m, x = _mat(dz, rows, cols, seed)
        dx, ya, yb = H.buf(cols * 4), H.buf(rows * 4), H.buf(rows * 4)
        H.put(dx, x)
        y0 = np.random.default_rng(seed + 10).standard_normal(rows).astype(np.float32)
        for acc in (0, 1):
            H.put(ya, y0)
            H.put(yb, y0)
            assert L.dz_q1_0_matvec_dev(m._h, dx, ya, acc, None) == 0
            assert L.dz_q1_0_matvec_dev_noalloc(m._h, dx, yb, acc, None) == 0, L.dz_last_error()
            assert H.h.hipDeviceSynchronize() == 0
            a, b = H.get(ya, rows), H.get(yb, rows)
            assert np.array_equal(a, b), (rows, cols, acc)
            assert np.abs(a).max() > 0
        for p in (dx, ya, yb):
            H.h.hipFree(p)
        m.close()


def test_noalloc_refuses_past_the_workspace_and_allocates_nothing(dz):
    L = dz.lib()
    H = _Hip()
    cap = L.dz_q1_0_noalloc_max_partials()
    assert cap == 4 << 20
    # 33 K tiles x 131072 rows = 4,325,376 partial sums > 4,194,304
    rows, cols = 131072, 33 * 512
    big = dz.Q1_0Matrix(np.zeros(rows * (cols // 128) * 18, np.uint8), rows, cols)
    dx, dy = H.buf(cols * 4), H.buf(rows * 4)
    assert L.dz_q1_0_matvec_dev_noalloc(big._h, dx, dy, 0, None) == dz.DZ_ERR_UNSUPPORTED
    assert b"workspace" in L.dz_last_error()
    big.close()
    H.h.hipFree(dx)
    H.h.hipFree(dy)
    # the largest product that fits (32 K tiles x 131072 rows = the whole workspace): a growing buffer
    # would have to allocate for it; free device memory stays where it was
    rows, cols = 131072, 32 * 512
    m, x = _mat(dz, rows, cols, 3)
    dx, dy = H.buf(cols * 4), H.buf(rows * 4)
    H.put(dx, x)
    assert H.h.hipDeviceSynchronize() == 0
    before = H.free_mem()
    assert L.dz_q1_0_matvec_dev_noalloc(m._h, dx, dy, 0, None) == 0, L.dz_last_error()
    assert H.h.hipDeviceSynchronize() == 0
    assert H.free_mem() == before
    y = H.get(dy, rows)
    import oracle
    # spot rows against the oracle (the full product on the CPU would take a while)
    blk_rows = np.concatenate([np.arange(0, 64), np.arange(rows - 64, rows)])
    rng = np.random.default_rng(3)
    aos = np.empty((rows, cols // 128, 18), np.uint8)
    aos[:, :, 2:] = rng.integers(0, 256, (rows, cols // 128, 16), dtype=np.uint8)
    aos[:, :, :2] = (np.abs(rng.standard_normal((rows, cols // 128))) * 0.02).astype(np.float16)[..., None].view(np.uint8)
    sub = np.ascontiguousarray(aos[blk_rows]).reshape(-1)
    yo = oracle.matvec(sub, len(blk_rows), cols, x)
    assert float(np.max(np.abs(y[blk_rows] - yo)) / np.max(np.abs(yo))) < 1e-5
    H.h.hipFree(dx)
    H.h.hipFree(dy)
    m.close()
