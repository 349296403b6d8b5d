"""ctypes loader for the CPU oracle (oracle/oracle.c).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker and the timed CPU restatement of the reference path.
The product package (daiza_amd) never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

f32p = ctypes.POINTER(ctypes.c_float)
u8p = ctypes.POINTER(ctypes.c_uint8)


def build():
    """Compile oracle/_build/liboracle.so with oracle/Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.or_f16_to_f32.restype = ctypes.c_float
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_f16_to_f32_bits.restype = ctypes.c_uint32
        L.or_f16_to_f32_bits.argtypes = [ctypes.c_uint16]
        L.or_f16_to_f32_fast.restype = ctypes.c_float
        L.or_f16_to_f32_fast.argtypes = [ctypes.c_uint16]
        L.or_dequant_row.argtypes = [u8p, ctypes.c_size_t, ctypes.c_size_t, f32p]
        L.or_dot_row_scalar.restype = ctypes.c_float
        L.or_dot_row_scalar.argtypes = [u8p, ctypes.c_size_t, ctypes.c_size_t, f32p, ctypes.c_int]
        L.or_matvec.argtypes = [u8p, ctypes.c_size_t, ctypes.c_size_t, f32p, f32p, ctypes.c_int, ctypes.c_int]
        L.or_matvec_scalar.argtypes = [u8p, ctypes.c_size_t, ctypes.c_size_t, f32p, f32p, ctypes.c_int]
        for n in ("or_exp_ps", "or_sigmoid_ps", "or_silu_ps"):
            getattr(L, n).argtypes = [f32p, f32p, ctypes.c_size_t]
        L.or_exp_fast.restype = ctypes.c_float
        L.or_exp_fast.argtypes = [ctypes.c_float]
        L.or_sigmoid_fast.restype = ctypes.c_float
        L.or_sigmoid_fast.argtypes = [ctypes.c_float]
        L.or_rmsnorm_into.argtypes = [f32p, f32p, f32p, ctypes.c_size_t, ctypes.c_float]
        L.or_l2norm_inplace.argtypes = [f32p, ctypes.c_size_t, ctypes.c_float]
        L.or_rope_freqs.argtypes = [ctypes.c_int, ctypes.c_float, f32p]
        L.or_rope_cos_sin.argtypes = [ctypes.c_int, f32p, ctypes.c_int, f32p, f32p]
        L.or_rope_partial.argtypes = [f32p, ctypes.c_int, f32p, f32p]
        L.or_swiglu.argtypes = [f32p, f32p, ctypes.c_size_t]
        L.or_argmax.restype = ctypes.c_int
        L.or_argmax.argtypes = [f32p, ctypes.c_size_t]
        L.or_ssm_scan_vhead.argtypes = [f32p, f32p, f32p, f32p, f32p, ctypes.c_float, ctypes.c_float,
                                        ctypes.c_float, ctypes.c_float, ctypes.c_int]
        L.or_lcg_next.restype = ctypes.c_float
        L.or_lcg_next.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        L.or_softmax_inplace.argtypes = [f32p, ctypes.c_size_t]
        L.or_softmax_pair_single.argtypes = [f32p, f32p, ctypes.c_size_t, ctypes.c_size_t,
                                             ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float)]
        L.or_sample_top_k_top_p.restype = ctypes.c_uint32
        L.or_sample_top_k_top_p.argtypes = [f32p, ctypes.c_size_t, ctypes.c_float, ctypes.c_int, ctypes.c_float,
                                            ctypes.POINTER(ctypes.c_uint64)]
        L.or_sample_bonus.restype = ctypes.c_uint32
        L.or_sample_bonus.argtypes = [f32p, f32p, ctypes.c_size_t, ctypes.c_float, ctypes.c_int, ctypes.c_float,
                                      ctypes.POINTER(ctypes.c_uint64)]
        L.or_leviathan_check.restype = ctypes.c_int
        L.or_leviathan_check.argtypes = [f32p, f32p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_float,
                                         ctypes.POINTER(ctypes.c_uint64)]
        L.or_model_synth.restype = ctypes.c_void_p
        L.or_model_synth.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int]
        L.or_model_free.argtypes = [ctypes.c_void_p]
        L.or_model_q1.restype = ctypes.c_void_p
        L.or_model_q1.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                  ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]
        L.or_model_f32.restype = ctypes.c_void_p
        L.or_model_f32.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_size_t)]
        L.or_ctx_new.restype = ctypes.c_void_p
        L.or_ctx_new.argtypes = [ctypes.c_void_p]
        L.or_ctx_free.argtypes = [ctypes.c_void_p]
        L.or_ctx_pos.restype = ctypes.c_int
        L.or_ctx_pos.argtypes = [ctypes.c_void_p]
        L.or_ctx_set_pos.argtypes = [ctypes.c_void_p, ctypes.c_int]
        L.or_kv_truncate.argtypes = [ctypes.c_void_p, ctypes.c_int]
        L.or_siphash.restype = ctypes.c_uint64
        L.or_siphash.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64, u8p, ctypes.c_size_t]
        L.or_model_embd_row.argtypes = [ctypes.c_void_p, ctypes.c_uint32, f32p]
        L.or_forward_token.restype = ctypes.c_int
        L.or_forward_token.argtypes = [ctypes.c_void_p, ctypes.c_uint32, f32p]
        L.or_mixer_step.argtypes = [ctypes.c_void_p, ctypes.c_int, f32p]
        L.or_set_ssm_state.argtypes = [ctypes.c_void_p, ctypes.c_int, f32p, f32p, ctypes.c_int]
        L.or_get_ssm_state.argtypes = [ctypes.c_void_p, ctypes.c_int, f32p, f32p, ctypes.POINTER(ctypes.c_int)]
        L.or_set_kv.argtypes = [ctypes.c_void_p, ctypes.c_int, f32p, f32p, ctypes.c_int]
        L.or_kv_len.restype = ctypes.c_int
        L.or_kv_len.argtypes = [ctypes.c_void_p, ctypes.c_int]
        L.or_get_kv.argtypes = [ctypes.c_void_p, ctypes.c_int, f32p, f32p, ctypes.c_int]
        L.or_synth_q1_0_rows.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_uint64,
                                         ctypes.c_uint64, ctypes.c_uint64, u8p]
        L.or_synth_normal_f32.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_uint64,
                                          ctypes.c_uint64, ctypes.c_double, ctypes.c_double, f32p]
        L.or_synth_embd_row_f16.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint64,
                                            ctypes.POINTER(ctypes.c_uint16)]
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f32_to_f16.argtypes = [ctypes.c_float]
        _lib = L
    return _lib


def synth_q1_0(seed, kind, layer, rows, cols, r0=0):
    out = np.empty(rows * (cols // 128) * 18, np.uint8)
    lib().or_synth_q1_0_rows(seed, kind, layer, cols, r0, r0 + rows, _u8(out))
    return out


def synth_normal(seed, kind, layer, n, mean=0.0, sigma=1.0, i0=0):
    out = np.empty(n, np.float32)
    lib().or_synth_normal_f32(seed, kind, layer, i0, n, mean, sigma, _f(out))
    return out


def synth_embd_row_f16(seed, token, hidden):
    out = np.empty(hidden, np.uint16)
    lib().or_synth_embd_row_f16(seed, int(token), hidden, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)))
    return out


def _f(a):
    return a.ctypes.data_as(f32p)


def _u8(a):
    return a.ctypes.data_as(u8p)


def siphash(c, d, k0, k1, msg):
    m = np.frombuffer(bytes(msg), np.uint8).copy() if len(msg) else np.zeros(1, np.uint8)
    return lib().or_siphash(c, d, k0, k1, _u8(m), len(msg))


def f16_to_f32(bits):
    return lib().or_f16_to_f32(int(bits))


def dequant_rows(aos, rows, cols):
    out = np.empty((rows, cols), np.float32)
    L = lib()
    for r in range(rows):
        L.or_dequant_row(_u8(aos), r, cols, _f(out[r]))
    return out


def matvec(aos, rows, cols, x, y=None, accumulate=False, nthreads=0):
    x = np.ascontiguousarray(x, np.float32)
    if y is None:
        y = np.zeros(rows, np.float32)
    lib().or_matvec(_u8(aos), rows, cols, _f(x), _f(y), int(accumulate), int(nthreads))
    return y


def matvec_scalar(aos, rows, cols, x, y=None, accumulate=False):
    x = np.ascontiguousarray(x, np.float32)
    if y is None:
        y = np.zeros(rows, np.float32)
    lib().or_matvec_scalar(_u8(aos), rows, cols, _f(x), _f(y), int(accumulate))
    return y


class Rng:
    """LcgRng state (sampling.rs:9-19) shared by the sampling helpers below."""

    def __init__(self, seed=0xC0FFEE):
        self.state = ctypes.c_uint64(seed)

    def next_f32(self):
        return lib().or_lcg_next(ctypes.byref(self.state))


def softmax(x):
    y = np.ascontiguousarray(x, np.float32).copy()
    lib().or_softmax_inplace(_f(y), y.size)
    return y


def softmax_pair_single(t, d, idx):
    t = np.ascontiguousarray(t, np.float32)
    d = np.ascontiguousarray(d, np.float32)
    p, q = ctypes.c_float(), ctypes.c_float()
    lib().or_softmax_pair_single(_f(t), _f(d), t.size, idx, ctypes.byref(p), ctypes.byref(q))
    return p.value, q.value


def sample_top_k_top_p(logits, temperature, top_k, top_p, rng):
    x = np.ascontiguousarray(logits, np.float32)
    return lib().or_sample_top_k_top_p(_f(x), x.size, temperature, top_k, top_p, ctypes.byref(rng.state))


def sample_bonus(target, draft, temperature, top_k, top_p, rng):
    t = np.ascontiguousarray(target, np.float32)
    d = np.ascontiguousarray(draft, np.float32)
    return lib().or_sample_bonus(_f(t), _f(d), t.size, temperature, top_k, top_p, ctypes.byref(rng.state))


def leviathan_check(target, draft, token, temperature, rng):
    t = np.ascontiguousarray(target, np.float32)
    d = np.ascontiguousarray(draft if draft is not None else target, np.float32)
    return bool(lib().or_leviathan_check(_f(t), _f(d), t.size, token, temperature, ctypes.byref(rng.state)))


def vec_op(name, x):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    getattr(lib(), name)(_f(x), _f(y), x.size)
    return y


class Model:
    """Synthetic model (daiza_synth.h bytes) plus one decode context."""

    def __init__(self, cfg_struct, seed, nthreads=0):
        self.cfg = cfg_struct
        self._m = lib().or_model_synth(ctypes.byref(cfg_struct), seed, nthreads)
        self._c = lib().or_ctx_new(self._m)

    def close(self):
        if self._c:
            lib().or_ctx_free(self._c)
            self._c = None
        if self._m:
            lib().or_model_free(self._m)
            self._m = None

    def __del__(self):
        self.close()

    def new_ctx(self):
        """Replace the context with a fresh one (pos 0, zero states)."""
        lib().or_ctx_free(self._c)
        self._c = lib().or_ctx_new(self._m)

    @property
    def pos(self):
        return lib().or_ctx_pos(self._c)

    def set_pos(self, p):
        lib().or_ctx_set_pos(self._c, p)

    def kv_truncate(self, n):
        """KvCache::truncate on every attention layer (kv_cache.rs:119-130), pos = n."""
        lib().or_kv_truncate(self._c, int(n))

    def forward(self, token, want_logits=True):
        logits = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        am = lib().or_forward_token(self._c, int(token), _f(logits) if want_logits else None)
        return am, logits

    def embd_row(self, token):
        out = np.empty(self.cfg.hidden, np.float32)
        lib().or_model_embd_row(self._m, int(token), _f(out))
        return out

    def mixer_step(self, layer, h):
        h = np.ascontiguousarray(h, np.float32).copy()
        lib().or_mixer_step(self._c, layer, _f(h))
        return h

    def q1(self, kind, layer):
        r, c = ctypes.c_size_t(), ctypes.c_size_t()
        p = lib().or_model_q1(self._m, kind, layer, ctypes.byref(r), ctypes.byref(c))
        if not p:
            return None
        n = r.value * (c.value // 128) * 18
        return np.ctypeslib.as_array((ctypes.c_uint8 * n).from_address(p)), r.value, c.value

    def f32(self, kind, layer):
        n = ctypes.c_size_t()
        p = lib().or_model_f32(self._m, kind, layer, ctypes.byref(n))
        if not p:
            return None
        return np.ctypeslib.as_array((ctypes.c_float * n.value).from_address(p)).copy()

    def set_ssm_state(self, layer, state, conv, head):
        lib().or_set_ssm_state(self._c, layer, _f(np.ascontiguousarray(state, np.float32)),
                               _f(np.ascontiguousarray(conv, np.float32)), int(head))

    def get_ssm_state(self, layer):
        c = self.cfg
        st = np.empty((c.ssm_v_heads, c.ssm_state, c.ssm_state), np.float32)
        qkvd = (2 * c.ssm_k_heads + c.ssm_v_heads) * c.ssm_state
        conv = np.empty((c.ssm_conv_kernel, qkvd), np.float32)
        head = ctypes.c_int()
        lib().or_get_ssm_state(self._c, layer, _f(st), _f(conv), ctypes.byref(head))
        return st, conv, head.value

    def set_kv(self, layer, k, v):
        n = k.shape[1]
        lib().or_set_kv(self._c, layer, _f(np.ascontiguousarray(k, np.float32)),
                        _f(np.ascontiguousarray(v, np.float32)), n)

    def get_kv(self, layer):
        c = self.cfg
        n = lib().or_kv_len(self._c, layer)
        k = np.empty((c.n_head_kv, n, c.head_dim), np.float32)
        v = np.empty_like(k)
        lib().or_get_kv(self._c, layer, _f(k), _f(v), n)
        return k, v
