"""daiza_amd — MI355X (gfx950) Q1_0 batch-1 decode behind a C ABI.

Python mirror of the reference interface for this path (guang384/Daiza, Daiza-engine):
  Q1_0Matrix      -> Daiza-engine/src/model/weights.rs:83-1208
  Config          -> Daiza-engine/src/model/config.rs:12-76
  Model / Context -> LoadedWeights + ForwardContext (weights.rs:1308, forward.rs:32-131)
Everything calls libdaiza_hip.so (include/daiza_hip.h) through ctypes; there is no CPU
fallback: if the library or a gfx950 device is missing, calls raise DaizaError.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_lib", "libdaiza_hip.so")

DZ_OK = 0
DZ_ERR_TENSOR = -1
DZ_ERR_MODEL = -2
DZ_ERR_UNSUPPORTED = -3
DZ_ERR_DEVICE = -4

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_vp = ctypes.c_void_p


class DaizaError(RuntimeError):
    """BonsaiError counterpart (Daiza-engine/src/lib.rs:42-78): code is the DZ_ERR_* status."""

    def __init__(self, code, msg):
        super().__init__("%s (%d): %s" % ({-1: "Tensor", -2: "Model", -3: "Unsupported", -4: "Device"}.get(code, "Error"),
                                          code, msg))
        self.code = code


class Config(ctypes.Structure):
    """dz_config; field meaning follows Config (config.rs:12-76)."""

    _fields_ = [
        ("n_layers", ctypes.c_int32), ("hidden", ctypes.c_int32), ("ffn", ctypes.c_int32),
        ("vocab", ctypes.c_int32), ("n_head", ctypes.c_int32), ("n_head_kv", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("rope_dim", ctypes.c_int32), ("rope_base", ctypes.c_float),
        ("rms_eps", ctypes.c_float), ("full_attn_interval", ctypes.c_int32), ("ssm_conv_kernel", ctypes.c_int32),
        ("ssm_state", ctypes.c_int32), ("ssm_k_heads", ctypes.c_int32), ("ssm_v_heads", ctypes.c_int32),
        ("embd_f16", ctypes.c_int32), ("max_ctx", ctypes.c_int32),
    ]

    @classmethod
    def bonsai27b(cls, max_ctx=4096):
        """Config::default (config.rs:47-76) with an f16 embedding."""
        return cls(n_layers=64, hidden=5120, ffn=17408, vocab=248320, n_head=24, n_head_kv=4, head_dim=256,
                   rope_dim=64, rope_base=1.0e7, rms_eps=1e-6, full_attn_interval=4, ssm_conv_kernel=4,
                   ssm_state=128, ssm_k_heads=16, ssm_v_heads=48, embd_f16=1, max_ctx=max_ctx)

    @classmethod
    def small(cls, n_layers=4, max_ctx=256, **kw):
        """A reduced hybrid stack with the same per-head shapes, for fast parity tests."""
        c = cls(n_layers=n_layers, hidden=512, ffn=1024, vocab=2048, n_head=4, n_head_kv=2, head_dim=256,
                rope_dim=64, rope_base=1.0e7, rms_eps=1e-6, full_attn_interval=4, ssm_conv_kernel=4,
                ssm_state=128, ssm_k_heads=2, ssm_v_heads=6, embd_f16=1, max_ctx=max_ctx)
        for k, v in kw.items():
            setattr(c, k, v)
        return c

    def is_full_attention(self, i):
        """Config::is_full_attention_block (config.rs:161-167)."""
        if self.full_attn_interval == 0:
            return True
        return i % self.full_attn_interval == self.full_attn_interval - 1

    @property
    def qkv_dim(self):
        return (2 * self.ssm_k_heads + self.ssm_v_heads) * self.ssm_state


_lib = None


def lib():
    """Load libdaiza_hip.so (built by daiza_amd.build); raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise DaizaError(DZ_ERR_DEVICE, "libdaiza_hip.so not built (run __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    L.dz_last_error.restype = ctypes.c_char_p
    L.dz_device_init.argtypes = [ctypes.c_int]
    L.dz_q1_0_upload.argtypes = [_u8p, ctypes.c_size_t, ctypes.c_size_t, ctypes.POINTER(_vp)]
    L.dz_q1_0_free.argtypes = [_vp]
    L.dz_q1_0_shape.argtypes = [_vp, ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]
    L.dz_q1_0_matvec.argtypes = [_vp, _f32p, _f32p, ctypes.c_int]
    L.dz_q1_0_matvec_multi.argtypes = [ctypes.POINTER(_vp), ctypes.c_int, _f32p, ctypes.POINTER(_f32p)]
    L.dz_q1_0_matvec_batch.argtypes = [_vp, _f32p, ctypes.c_int, _f32p, ctypes.c_int]
    L.dz_q1_0_matvec_dev.argtypes = [_vp, _vp, _vp, ctypes.c_int, _vp]
    L.dz_q1_0_matvec_dev_status.argtypes = [_vp]
    L.dz_q1_0_dequant_rows.argtypes = [_vp, ctypes.c_size_t, ctypes.c_size_t, _f32p]
    L.dz_q1_0_gemv_partials.argtypes = [_vp, _vp, _vp, _vp]
    L.dz_q1_0_partials_ld.argtypes = [_vp]
    L.dz_q1_0_partials_ld.restype = ctypes.c_size_t
    L.dz_q1_0_ntiles.argtypes = [_vp]
    L.dz_q1_0_matvec_dev_noalloc.argtypes = [_vp, _vp, _vp, ctypes.c_int, _vp]
    L.dz_q1_0_noalloc_max_partials.argtypes = []
    L.dz_q1_0_noalloc_max_partials.restype = ctypes.c_size_t
    for name, args in _MODEL_PROTOS.items():
        fn = getattr(L, name, None)
        if fn is not None:
            fn.argtypes = args[0]
            fn.restype = args[1]
    _lib = L
    return L


_MODEL_PROTOS = {
    "dz_config_bonsai27b": ([_vp, ctypes.c_int32], None),
    "dz_model_create": ([_vp, _vp, ctypes.c_int, ctypes.POINTER(_vp)], ctypes.c_int),
    "dz_model_create_synth": ([_vp, ctypes.c_uint64, ctypes.POINTER(_vp)], ctypes.c_int),
    "dz_gguf_open": ([ctypes.c_char_p, ctypes.POINTER(_vp)], ctypes.c_int),
    "dz_gguf_close": ([_vp], ctypes.c_int),
    "dz_gguf_n_tensors": ([_vp], ctypes.c_int),
    "dz_gguf_tensor_info": ([_vp, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_int32),
                             ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_uint64),
                             ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)], ctypes.c_int),
    "dz_gguf_tensor_data": ([_vp, ctypes.c_int], _vp),
    "dz_gguf_config": ([_vp, ctypes.c_int32, _vp, ctypes.POINTER(ctypes.c_int32)], ctypes.c_int),
    "dz_gguf_context_length": ([_vp, ctypes.POINTER(ctypes.c_uint64)], ctypes.c_int),
    "dz_model_create_gguf": ([_vp, _vp, ctypes.POINTER(_vp)], ctypes.c_int),
    "dz_model_free": ([_vp], ctypes.c_int),
    "dz_model_weight_bytes": ([_vp, ctypes.POINTER(ctypes.c_uint64)], ctypes.c_int),
    "dz_ctx_create": ([_vp, ctypes.POINTER(_vp)], ctypes.c_int),
    "dz_ctx_free": ([_vp], ctypes.c_int),
    "dz_ctx_reset": ([_vp], ctypes.c_int),
    "dz_ctx_pos": ([_vp], ctypes.c_int),
    "dz_forward_token": ([_vp, ctypes.c_uint32, _f32p, _u32p], ctypes.c_int),
    "dz_forward_batch": ([_vp, _u32p, ctypes.c_int, ctypes.c_int, _f32p, _f32p], ctypes.c_int),
    "dz_decode_greedy": ([_vp, ctypes.c_uint32, ctypes.c_int, _u32p], ctypes.c_int),
    "dz_decode_greedy_eos": ([_vp, ctypes.c_uint32, ctypes.c_int, ctypes.c_int32, _u32p, ctypes.POINTER(ctypes.c_int)],
                             ctypes.c_int),
    "dz_ctx_logits": ([_vp, _f32p], ctypes.c_int),
    "dz_ctx_set_ssm_state": ([_vp, ctypes.c_int, _f32p, _f32p, ctypes.c_int], ctypes.c_int),
    "dz_ctx_get_ssm_state": ([_vp, ctypes.c_int, _f32p, _f32p, ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
    "dz_ctx_set_kv": ([_vp, ctypes.c_int, _f32p, _f32p, ctypes.c_int], ctypes.c_int),
    "dz_ctx_get_kv": ([_vp, ctypes.c_int, _f32p, _f32p, ctypes.c_int], ctypes.c_int),
    "dz_ctx_kv_len": ([_vp, ctypes.c_int], ctypes.c_int),
    "dz_kv_truncate": ([_vp, ctypes.c_int], ctypes.c_int),
    "dz_ctx_set_pos": ([_vp, ctypes.c_int], ctypes.c_int),
    "dz_ctx_mixer_step": ([_vp, ctypes.c_int, _f32p], ctypes.c_int),
    "dz_ctx_mixer_step_dev": ([_vp, ctypes.c_int, _vp, _vp], ctypes.c_int),
    "dz_ctx_stream": ([_vp], _vp),
    "dz_ctx_copy_state": ([_vp, _vp], ctypes.c_int),
    "dz_session_cfg_hash": ([_vp, ctypes.c_uint64], ctypes.c_uint64),
    "dz_ctx_save": ([_vp, ctypes.c_char_p, ctypes.c_uint64, _u32p, ctypes.c_uint64, ctypes.c_int32, ctypes.c_char_p],
                    ctypes.c_int),
    "dz_ctx_load": ([_vp, ctypes.c_char_p, ctypes.c_uint64, _u32p, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64),
                     ctypes.POINTER(ctypes.c_int32), ctypes.c_char_p, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)],
                    ctypes.c_int),
    "dz_ctx_token_kernel": ([_vp], ctypes.c_int),
    "dz_ctx_vocab": ([_vp, ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
    "dz_verify_forward": ([_vp, _u32p, ctypes.c_int, _f32p], ctypes.c_int),
    "dz_verify_commit": ([_vp, ctypes.c_int], ctypes.c_int),
    "dz_lcg_next": ([ctypes.POINTER(ctypes.c_uint64)], ctypes.c_float),
    "dz_decode_sample": ([_vp, ctypes.c_uint32, ctypes.c_int, _vp, ctypes.POINTER(ctypes.c_uint64), _u32p], ctypes.c_int),
    "dz_sample": ([_f32p, ctypes.c_int, _vp, ctypes.POINTER(ctypes.c_uint64), _u32p], ctypes.c_int),
    "dz_leviathan_check": ([_f32p, _f32p, ctypes.c_int, ctypes.c_uint32, _vp, ctypes.POINTER(ctypes.c_uint64),
                            ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
    "dz_sample_bonus": ([_f32p, _f32p, ctypes.c_int, _vp, ctypes.POINTER(ctypes.c_uint64), _u32p], ctypes.c_int),
    "dz_spec_verify": ([_vp, _u32p, ctypes.c_int, _f32p, _vp, ctypes.c_int32, ctypes.POINTER(ctypes.c_uint64),
                        ctypes.POINTER(ctypes.c_int), _u32p], ctypes.c_int),
}

EXPORTED_SYMBOLS = [
    "dz_config_bonsai27b", "dz_last_error", "dz_device_init",
    "dz_q1_0_upload", "dz_q1_0_free", "dz_q1_0_shape", "dz_q1_0_matvec", "dz_q1_0_matvec_multi", "dz_q1_0_matvec_batch",
    "dz_q1_0_matvec_dev", "dz_q1_0_matvec_dev_status", "dz_q1_0_dequant_rows", "dz_q1_0_gemv_partials", "dz_q1_0_partials_ld", "dz_q1_0_ntiles",
    "dz_q1_0_matvec_dev_noalloc", "dz_q1_0_noalloc_max_partials",
] + list(k for k in _MODEL_PROTOS if k != "dz_config_bonsai27b")


def _check(rc):
    if rc != DZ_OK:
        raise DaizaError(rc, lib().dz_last_error().decode(errors="replace"))


def _f(a):
    return a.ctypes.data_as(_f32p)


class Q1_0Matrix:
    """Device-resident Q1_0 matrix (Q1_0Matrix, weights.rs:83-1208).

    `aos` is the reference byte layout: per row, cols/128 blocks of [f16 scale LE | 16 sign bytes].
    """

    def __init__(self, aos, rows, cols):
        aos = np.ascontiguousarray(aos, dtype=np.uint8)
        if aos.size != rows * (cols // 128) * 18:
            raise DaizaError(DZ_ERR_TENSOR, "byte count %d does not match %dx%d Q1_0" % (aos.size, rows, cols))
        self.rows, self.cols = int(rows), int(cols)
        h = _vp()
        _check(lib().dz_q1_0_upload(aos.ctypes.data_as(_u8p), rows, cols, ctypes.byref(h)))
        self._h = h

    def close(self):
        if getattr(self, "_h", None):
            lib().dz_q1_0_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def matvec_into_slice(self, x, y):
        """y = W x (weights.rs:123-325)."""
        x = np.ascontiguousarray(x, np.float32)
        assert x.size == self.cols and y.size == self.rows and y.dtype == np.float32 and y.flags.c_contiguous
        _check(lib().dz_q1_0_matvec(self._h, _f(x), _f(y), 0))

    def matvec_add_into_slice(self, x, y):
        """y += W x (weights.rs:334-465)."""
        x = np.ascontiguousarray(x, np.float32)
        assert x.size == self.cols and y.size == self.rows and y.dtype == np.float32 and y.flags.c_contiguous
        _check(lib().dz_q1_0_matvec(self._h, _f(x), _f(y), 1))

    def matvec(self, x):
        y = np.empty(self.rows, np.float32)
        self.matvec_into_slice(x, y)
        return y

    @staticmethod
    def matvec_multi_into_slice(x, matrices, outputs):
        """Several matrices sharing x in one pass (weights.rs:831-972)."""
        n = len(matrices)
        x = np.ascontiguousarray(x, np.float32)
        hs = (_vp * n)(*[m._h for m in matrices])
        ys = (_f32p * n)(*[_f(o) for o in outputs])
        _check(lib().dz_q1_0_matvec_multi(hs, n, _f(x), ys))

    def matvec_batch_into_slice(self, x, n_batch, y):
        """y[i] = W x[i] for i < n_batch; x [n][cols], y [n][rows] (weights.rs:475-682)."""
        x = np.ascontiguousarray(x, np.float32)
        assert x.size == n_batch * self.cols and y.size == n_batch * self.rows
        assert y.dtype == np.float32 and y.flags.c_contiguous
        _check(lib().dz_q1_0_matvec_batch(self._h, _f(x), n_batch, _f(y), 0))

    def matvec_add_batch_into_slice(self, x, n_batch, y):
        """y[i] += W x[i] for i < n_batch (weights.rs:976-980)."""
        x = np.ascontiguousarray(x, np.float32)
        assert x.size == n_batch * self.cols and y.size == n_batch * self.rows
        assert y.dtype == np.float32 and y.flags.c_contiguous
        _check(lib().dz_q1_0_matvec_batch(self._h, _f(x), n_batch, _f(y), 1))

    def matvec_batch(self, x):
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.cols)
        y = np.empty((x.shape[0], self.rows), np.float32)
        self.matvec_batch_into_slice(x, x.shape[0], y)
        return y

    def row_into_slice(self, row, y):
        """Dequantised row (weights.rs:106 -> quant.rs:161-194)."""
        _check(lib().dz_q1_0_dequant_rows(self._h, row, 1, _f(y)))

    def dequant_rows(self, r0, n):
        out = np.empty((n, self.cols), np.float32)
        _check(lib().dz_q1_0_dequant_rows(self._h, r0, n, _f(out)))
        return out


class Tensor(ctypes.Structure):
    """dz_tensor: one GGUF-named host tensor (type 0 = F32, 1 = F16, 41 = Q1_0)."""
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_int32), ("data", _vp), ("n_bytes", ctypes.c_size_t)]


GGUF_F32, GGUF_F16, GGUF_Q1_0 = 0, 1, 41


class Model:
    """Device-resident weights (LoadedWeights, weights.rs:1308-1379)."""

    def __init__(self, cfg, seed=None, tensors=None):
        self.cfg = cfg
        h = _vp()
        if tensors is None:
            _check(lib().dz_model_create_synth(ctypes.byref(cfg), int(seed), ctypes.byref(h)))
        else:
            # tensors: {GGUF name: (type, array)}; the arrays are borrowed for the call only
            keep = []
            arr = (Tensor * len(tensors))()
            for i, (name, (ty, a)) in enumerate(tensors.items()):
                a = np.ascontiguousarray(a)
                keep.append(a)
                arr[i] = Tensor(name.encode(), int(ty), a.ctypes.data, a.nbytes)
            _check(lib().dz_model_create(ctypes.byref(cfg), arr, len(tensors), ctypes.byref(h)))
            del keep
        self._h = h

    @classmethod
    def from_tensors(cls, cfg, tensors):
        """Weights from GGUF-named host tensors (LoadedWeights::load_all, weights.rs:1308-1379)."""
        return cls(cfg, tensors=tensors)

    @classmethod
    def synthetic(cls, cfg, seed):
        """Random Q1_0 model from the daiza_synth.h generator (BASELINE config 4 at Bonsai shape)."""
        return cls(cfg, seed=seed)

    def q1_bytes(self):
        v = ctypes.c_uint64()
        _check(lib().dz_model_weight_bytes(self._h, ctypes.byref(v)))
        return v.value

    def close(self):
        if getattr(self, "_h", None):
            lib().dz_model_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GgufFile:
    """A GGUF v3 file mapped read-only (GgufFile::open, gguf/parser.rs:40-119)."""

    def __init__(self, path):
        h = _vp()
        _check(lib().dz_gguf_open(os.fsencode(path), ctypes.byref(h)))
        self._h = h

    def close(self):
        if getattr(self, "_h", None):
            lib().dz_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensors(self):
        """[(name, type, dims in GGUF order, absolute offset, n_bytes)] in file order."""
        out = []
        for i in range(lib().dz_gguf_n_tensors(self._h)):
            name, ty, nd = ctypes.c_char_p(), ctypes.c_int32(), ctypes.c_int32()
            dims = (ctypes.c_uint64 * 4)()
            off, nb = ctypes.c_uint64(), ctypes.c_uint64()
            _check(lib().dz_gguf_tensor_info(self._h, i, ctypes.byref(name), ctypes.byref(ty), ctypes.byref(nd), dims,
                                             ctypes.byref(off), ctypes.byref(nb)))
            out.append((name.value.decode(), ty.value, tuple(dims[:nd.value]), off.value, nb.value))
        return out

    def tensor_bytes(self, i):
        p = lib().dz_gguf_tensor_data(self._h, i)
        if not p:
            return None
        n = self.tensors()[i][4]
        return np.ctypeslib.as_array((ctypes.c_uint8 * n).from_address(p)).copy()

    def config(self, max_ctx=4096):
        """Config::from_metadata (model/config.rs:76-160); returns (Config, eos_token_id)."""
        c = Config()
        eos = ctypes.c_int32()
        _check(lib().dz_gguf_config(self._h, int(max_ctx), ctypes.byref(c), ctypes.byref(eos)))
        return c, eos.value

    def context_length(self):
        """Config::context_length (model/config.rs:52, 92-93), hashed into DZSS session files."""
        v = ctypes.c_uint64()
        _check(lib().dz_gguf_context_length(self._h, ctypes.byref(v)))
        return v.value

    def model(self, cfg):
        """LoadedWeights::load_all (weights.rs:1308-1379) on the device."""
        m = Model.__new__(Model)
        m.cfg = cfg
        h = _vp()
        _check(lib().dz_model_create_gguf(self._h, ctypes.byref(cfg), ctypes.byref(h)))
        m._h = h
        return m


class SamplingParams(ctypes.Structure):
    """SamplingParams (sampling.rs:22-32) without the repetition penalties (dz_sampling)."""
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_int32), ("top_p", ctypes.c_float)]

    def __init__(self, temperature=0.7, top_k=20, top_p=0.95):
        super().__init__(temperature, top_k, top_p)


class LcgRng:
    """LcgRng (sampling.rs:9-19); the state advances through every sampling call it is passed to."""

    def __init__(self, seed=0xC0FFEE):
        self.state = ctypes.c_uint64(seed)

    def next_f32(self):
        return lib().dz_lcg_next(ctypes.byref(self.state))


def sample_top_k_top_p(logits, params, rng):
    """sample_top_k_top_p_into (sampling.rs:144-247)."""
    x = np.ascontiguousarray(logits, np.float32)
    out = ctypes.c_uint32()
    _check(lib().dz_sample(_f(x), x.size, ctypes.byref(params), ctypes.byref(rng.state), ctypes.byref(out)))
    return out.value


def leviathan_check(target, draft, token, params, rng):
    """leviathan_check (engine.rs:1791-1819)."""
    t = np.ascontiguousarray(target, np.float32)
    d = None if draft is None else np.ascontiguousarray(draft, np.float32)
    acc = ctypes.c_int()
    _check(lib().dz_leviathan_check(_f(t), _f(d) if d is not None else None, t.size, int(token), ctypes.byref(params),
                                    ctypes.byref(rng.state), ctypes.byref(acc)))
    return bool(acc.value)


def sample_bonus(target, draft, params, rng):
    """sample_bonus (engine.rs:1833-1866)."""
    t = np.ascontiguousarray(target, np.float32)
    d = np.ascontiguousarray(draft, np.float32)
    out = ctypes.c_uint32()
    _check(lib().dz_sample_bonus(_f(t), _f(d), t.size, ctypes.byref(params), ctypes.byref(rng.state),
                                 ctypes.byref(out)))
    return out.value


CONTEXT_LENGTH = 262144  # qwen35.context_length of Bonsai-27B (Config::context_length), hashed into DZSS files


def session_cfg_hash(cfg, context_length=CONTEXT_LENGTH):
    """cfg_hash of session_persist.rs:52-66 for this configuration."""
    return lib().dz_session_cfg_hash(ctypes.byref(cfg), int(context_length))


class Context:
    """ModelState + ForwardContext (forward.rs:32-131) on the device."""

    def __init__(self, model):
        self.model = model
        self.cfg = model.cfg
        h = _vp()
        _check(lib().dz_ctx_create(model._h, ctypes.byref(h)))
        self._h = h

    def close(self):
        if getattr(self, "_h", None):
            lib().dz_ctx_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def pos(self):
        return lib().dz_ctx_pos(self._h)

    @property
    def token_kernel(self):
        """True when forwards run in the persistent token kernel (see dz_ctx_token_kernel)."""
        return bool(lib().dz_ctx_token_kernel(self._h))

    def reset(self):
        _check(lib().dz_ctx_reset(self._h))

    def set_pos(self, pos):
        _check(lib().dz_ctx_set_pos(self._h, int(pos)))

    def verify_forward(self, draft, want_logits=True):
        """Forward of the drafts without moving the position; per-position logits [k][vocab]."""
        d = np.ascontiguousarray(draft, np.uint32)
        out = np.empty((d.size, self.cfg.vocab), np.float32) if want_logits else None
        _check(lib().dz_verify_forward(self._h, d.ctypes.data_as(_u32p), d.size, _f(out) if want_logits else None))
        return out

    def verify_commit(self, n_accept):
        _check(lib().dz_verify_commit(self._h, int(n_accept)))

    def spec_verify(self, draft, draft_logits, params, rng, eos_id=-1):
        """One speculative step (dz_spec_verify); returns (n_accepted, bonus or None at an accepted EOS)."""
        d = np.ascontiguousarray(draft, np.uint32)
        dl = None if draft_logits is None else np.ascontiguousarray(draft_logits, np.float32)
        na, b = ctypes.c_int(), ctypes.c_uint32()
        _check(lib().dz_spec_verify(self._h, d.ctypes.data_as(_u32p), d.size, _f(dl) if dl is not None else None,
                                    ctypes.byref(params), int(eos_id), ctypes.byref(rng.state), ctypes.byref(na),
                                    ctypes.byref(b)))
        return na.value, (None if b.value == 0xFFFFFFFF else b.value)

    def forward_single_token(self, token, want_logits=True):
        """forward.rs:204; returns (argmax, logits or None)."""
        am = ctypes.c_uint32()
        logits = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        _check(lib().dz_forward_token(self._h, int(token), _f(logits) if want_logits else None, ctypes.byref(am)))
        return am.value, logits

    def forward_batch(self, ids, per_pos_logits=False):
        """forward.rs:394; returns last logits, or all positions' logits [n][vocab]."""
        ids = np.ascontiguousarray(ids, np.uint32)
        n = ids.size
        last = np.empty(self.cfg.vocab, np.float32)
        per = np.empty((n, self.cfg.vocab), np.float32) if per_pos_logits else None
        _check(lib().dz_forward_batch(self._h, ids.ctypes.data_as(_u32p), n, self.pos, _f(last),
                                      _f(per) if per_pos_logits else None))
        return per if per_pos_logits else last

    def decode_greedy(self, first_token, n):
        """n greedy forwards on the device; the pick after each (engine.rs:850-871 without the EOS stop)."""
        out = np.empty(n, np.uint32)
        _check(lib().dz_decode_greedy(self._h, int(first_token), int(n), out.ctypes.data_as(_u32p)))
        return out

    def decode_sample(self, first_token, n, params, rng):
        """n sampled forwards (engine.rs:850-862 without the EOS stop): each next input is
        sample_top_k_top_p_into of the previous logits with params and rng (LcgRng, advanced once per
        token); on the token kernel the top-k and the draw run on the device."""
        out = np.empty(n, np.uint32)
        _check(lib().dz_decode_sample(self._h, int(first_token), int(n), ctypes.byref(params),
                                      ctypes.byref(rng.state), out.ctypes.data_as(_u32p)))
        return out

    def decode_greedy_eos(self, first_token, n, eos_id):
        """The greedy loop with its EOS stop (engine.rs:850-871): picks after each forward run; the last
        is eos_id when the loop stopped on it (that token is not forwarded)."""
        out = np.empty(max(n, 1), np.uint32)
        done = ctypes.c_int()
        _check(lib().dz_decode_greedy_eos(self._h, int(first_token), int(n), int(eos_id), out.ctypes.data_as(_u32p),
                                          ctypes.byref(done)))
        return out[:done.value].copy()

    def kv_truncate(self, n):
        """KvCache::truncate (kv_cache.rs:119-130): keeps n cached positions, pos = n; conv rings stay."""
        _check(lib().dz_kv_truncate(self._h, int(n)))

    def copy_state_from(self, src):
        """ModelState::clone onto this context (dz_ctx_copy_state): checkpoint into a spare context,
        restore by copying back."""
        _check(lib().dz_ctx_copy_state(self._h, src._h))

    def save(self, path, history=(), think_enabled=False, system_prompt=None, context_length=CONTEXT_LENGTH):
        """Session::save_to_disk (session_persist.rs:70-146): the DZSS v1 file of this context's state,
        with the session fields the caller holds (history tokens, think flag, system prompt)."""
        h = np.ascontiguousarray(history, np.uint32)
        sp = None if system_prompt is None else system_prompt.encode()
        _check(lib().dz_ctx_save(self._h, os.fsencode(path), int(context_length), h.ctypes.data_as(_u32p), h.size,
                                 int(bool(think_enabled)), sp))

    def load(self, path, context_length=CONTEXT_LENGTH, history_cap=1 << 20, prompt_cap=1 << 16):
        """Session::load_from_disk (session_persist.rs:188-312) into this context; returns
        (history tokens, think_enabled, system prompt or None)."""
        hist = np.empty(history_cap, np.uint32)
        nh, think, plen = ctypes.c_uint64(), ctypes.c_int32(), ctypes.c_uint64()
        buf = ctypes.create_string_buffer(prompt_cap)
        _check(lib().dz_ctx_load(self._h, os.fsencode(path), int(context_length), hist.ctypes.data_as(_u32p), history_cap,
                                 ctypes.byref(nh), ctypes.byref(think), buf, prompt_cap, ctypes.byref(plen)))
        has_sys = open(path, "rb").read(38)[37] != 0
        return hist[:nh.value].copy(), bool(think.value), (buf.raw[:plen.value].decode(errors="replace") if has_sys else None)

    def logits(self):
        out = np.empty(self.cfg.vocab, np.float32)
        _check(lib().dz_ctx_logits(self._h, _f(out)))
        return out

    def mixer_step(self, layer, h):
        h = np.ascontiguousarray(h, np.float32).copy()
        _check(lib().dz_ctx_mixer_step(self._h, int(layer), _f(h)))
        return h

    def set_ssm_state(self, layer, state, conv, head):
        _check(lib().dz_ctx_set_ssm_state(self._h, int(layer), _f(np.ascontiguousarray(state, np.float32)),
                                          _f(np.ascontiguousarray(conv, np.float32)), int(head)))

    def get_ssm_state(self, layer):
        c = self.cfg
        st = np.empty((c.ssm_v_heads, c.ssm_state, c.ssm_state), np.float32)
        conv = np.empty((c.ssm_conv_kernel, c.qkv_dim), np.float32)
        head = ctypes.c_int()
        _check(lib().dz_ctx_get_ssm_state(self._h, int(layer), _f(st), _f(conv), ctypes.byref(head)))
        return st, conv, head.value

    def set_kv(self, layer, k, v):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        _check(lib().dz_ctx_set_kv(self._h, int(layer), _f(k), _f(v), k.shape[1]))

    def get_kv(self, layer, n):
        c = self.cfg
        k = np.empty((c.n_head_kv, n, c.head_dim), np.float32)
        v = np.empty_like(k)
        _check(lib().dz_ctx_get_kv(self._h, int(layer), _f(k), _f(v), int(n)))
        return k, v

    def stream(self):
        return lib().dz_ctx_stream(self._h)
