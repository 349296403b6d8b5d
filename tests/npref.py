"""Float64 numpy restatement of one decode step, for checking the CPU oracle.

Written from the reference's semantics, independently of oracle/oracle.c (different precision,
vectorised form, and the conv weights regenerated in GGUF order rather than read back):
  embedding     forward.rs:212, F16 rows through f16_to_f32 (tensor/tensor.rs:68-80, quant.rs:39-74)
  RoPE          rope.rs:27-38 (freqs, f32), rope.rs:82-101 (theta = pos as f32 * freq, f32),
                rope.rs:187-231 (x1*c + x2*s, x2*c + x1*s)
  DeltaNet      ssm.rs:425-616 (conv ring 467-513, l2norm 76-135, scan 153-180, gate 246-286)
  attention     attention.rs:56-208 (q|gate interleave, q/k RMSNorm, 1/sqrt(hd), GQA qh // group)
  MLP           mlp.rs:28-47;  block order block.rs:53-124;  output norm + lm_head forward.rs:340-375
Matrix products use exact IEEE f16 scales, as the reference GEMV's _mm256_cvtph_ps does
(quant.rs:614-740).  Test infrastructure only.
"""
import numpy as np

# kinds of include/daiza_synth.h
K_EMBD, K_OUTPUT_NORM, K_OUTPUT = 1, 2, 3
K_ATTN_NORM, K_POST_NORM, K_FFN_GATE, K_FFN_UP, K_FFN_DOWN = 16, 17, 18, 19, 20
K_SSM_QKV, K_SSM_ALPHA, K_SSM_BETA, K_SSM_Z, K_SSM_OUT, K_SSM_CONV, K_SSM_A, K_SSM_DT, K_SSM_NORM = range(32, 41)
K_ATT_Q, K_ATT_K, K_ATT_V, K_ATT_O, K_ATT_QNORM, K_ATT_KNORM = range(48, 54)


def f16_ref_quirk(bits):
    """quant.rs:39-74 as a closed form: IEEE value, except that a subnormal half with leading
    mantissa bit p (0..9) comes out 2**(20 - 2p) times its IEEE value (the loop adds its shift
    count to the exponent instead of subtracting it)."""
    bits = np.asarray(bits, np.uint16)
    v = bits.view(np.float16).astype(np.float64)
    mant = (bits & 0x3FF).astype(np.int64)
    sub = ((bits & 0x7C00) == 0) & (mant != 0)
    p = np.where(sub, np.floor(np.log2(np.maximum(mant, 1))), 0).astype(np.int64)
    return np.where(sub, v * np.exp2(20 - 2 * p), v)


def dequant_ieee(aos, rows, cols):
    """Q1_0 AoS bytes -> float64 [rows][cols]; bit j of sign byte b is column 8b+j of the group."""
    blk = np.asarray(aos, np.uint8).reshape(rows, cols // 128, 18)
    scale = np.ascontiguousarray(blk[:, :, 0:2]).view(np.float16)[..., 0].astype(np.float64)
    bits = np.unpackbits(blk[:, :, 2:], axis=-1, bitorder="little")
    return (np.where(bits == 1, 1.0, -1.0) * scale[..., None]).reshape(rows, cols)


def rmsnorm(x, w, eps):
    return x / np.sqrt(np.mean(x * x) + eps) * w


def silu(x):
    return x / (1.0 + np.exp(-x))


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def softplus(x):
    return x if x > 20.0 else np.log1p(np.exp(x))


def rope_cos_sin(pos, rope_dim, base):
    half = rope_dim // 2
    i = np.arange(half)
    freqs = (np.float32(1.0) / np.power(np.float32(base), (2 * i).astype(np.float32) / np.float32(rope_dim),
                                        dtype=np.float32)).astype(np.float32)
    th = (np.float32(pos) * freqs).astype(np.float64)
    return np.cos(th), np.sin(th)


def rope_quirk(x, c, s):
    half = c.size
    x1, x2 = x[:half].copy(), x[half:2 * half].copy()
    y = x.copy()
    y[:half] = x1 * c + x2 * s
    y[half:2 * half] = x2 * c + x1 * s
    return y


class NpDecoder:
    """Float64 decoder over the weights of an oracle.Model (the shared synthetic generator)."""

    def __init__(self, om, cfg, seed):
        import oracle
        self.oracle = oracle
        self.om, self.c, self.seed = om, cfg, seed
        self._mats = {}
        c = cfg
        self.hd = c.ssm_state
        self.kdim = c.ssm_k_heads * self.hd
        self.inner = c.ssm_v_heads * self.hd
        self.qkvd = 2 * self.kdim + self.inner
        self.pos = 0
        self.S = {}
        self.ring = {}
        self.head = {}
        self.K = {}
        self.V = {}
        for l in range(c.n_layers):
            if c.is_full_attention(l):
                self.K[l] = np.zeros((c.n_head_kv, 0, c.head_dim))
                self.V[l] = np.zeros((c.n_head_kv, 0, c.head_dim))
            else:
                self.S[l] = np.zeros((c.ssm_v_heads, self.hd, self.hd))
                self.ring[l] = np.zeros((c.ssm_conv_kernel, self.qkvd))
                self.head[l] = 0

    def W(self, kind, layer):
        key = (kind, layer)
        if key not in self._mats:
            aos, r, cc = self.om.q1(kind, layer)
            self._mats[key] = dequant_ieee(aos, r, cc)
        return self._mats[key]

    def v(self, kind, layer):
        return self.om.f32(kind, layer).astype(np.float64)

    def conv_w(self, layer):
        """GGUF order [qkv_dim][conv_kernel], regenerated from the generator's stream."""
        ck = self.c.ssm_conv_kernel
        w = self.oracle.synth_normal(self.seed, K_SSM_CONV, layer, self.qkvd * ck, 0.0, 0.25)
        return w.astype(np.float64).reshape(self.qkvd, ck)

    def embed(self, token):
        return f16_ref_quirk(self.oracle.synth_embd_row_f16(self.seed, token, self.c.hidden))

    def deltanet(self, l, h):
        c, hd = self.c, self.hd
        n = rmsnorm(h, self.v(K_ATTN_NORM, l), c.rms_eps)
        qkv = self.W(K_SSM_QKV, l) @ n
        a = self.W(K_SSM_ALPHA, l) @ n
        b = self.W(K_SSM_BETA, l) @ n
        z = self.W(K_SSM_Z, l) @ n
        ring = self.ring[l]
        ring[self.head[l]] = qkv
        self.head[l] = (self.head[l] + 1) % c.ssm_conv_kernel
        w = self.conv_w(l)
        conv = np.zeros(self.qkvd)
        for t in range(c.ssm_conv_kernel):  # t = 0 oldest ... kernel-1 newest
            conv += ring[(self.head[l] + t) % c.ssm_conv_kernel] * w[:, t]
        conv = silu(conv)
        q = conv[:self.kdim].reshape(c.ssm_k_heads, hd)
        k = conv[self.kdim:2 * self.kdim].reshape(c.ssm_k_heads, hd)
        v = conv[2 * self.kdim:].reshape(c.ssm_v_heads, hd)
        q = q / np.sqrt(np.sum(q * q, axis=1, keepdims=True) + 1e-6) / np.sqrt(hd)
        k = k / np.sqrt(np.sum(k * k, axis=1, keepdims=True) + 1e-6)
        ssm_a, dt = self.v(K_SSM_A, l), self.v(K_SSM_DT, l)
        y = np.zeros((c.ssm_v_heads, hd))
        for vh in range(c.ssm_v_heads):
            kh = vh % c.ssm_k_heads
            decay = np.exp(ssm_a[vh] * softplus(a[vh] + dt[vh]))
            beta = sigmoid(b[vh])
            S = self.S[l][vh] * decay
            d = (v[vh] - S @ k[kh]) * beta
            S = S + np.outer(d, k[kh])
            self.S[l][vh] = S
            y[vh] = S @ q[kh]
        zz = silu(z).reshape(c.ssm_v_heads, hd)
        y = y / np.sqrt(np.mean(y * y, axis=1, keepdims=True) + c.rms_eps) * self.v(K_SSM_NORM, l) * zz
        return h + self.W(K_SSM_OUT, l) @ y.reshape(-1)

    def attention(self, l, h, cs):
        c = self.c
        hd, nq, nkv = c.head_dim, c.n_head, c.n_head_kv
        grp = nq // nkv
        n = rmsnorm(h, self.v(K_ATTN_NORM, l), c.rms_eps)
        qg = (self.W(K_ATT_Q, l) @ n).reshape(nq, 2, hd)
        k = (self.W(K_ATT_K, l) @ n).reshape(nkv, hd)
        v = (self.W(K_ATT_V, l) @ n).reshape(nkv, hd)
        qn, kn = self.v(K_ATT_QNORM, l), self.v(K_ATT_KNORM, l)
        q = np.stack([rope_quirk(rmsnorm(qg[i, 0], qn, c.rms_eps), *cs) for i in range(nq)]) / np.sqrt(hd)
        k = np.stack([rope_quirk(rmsnorm(k[i], kn, c.rms_eps), *cs) for i in range(nkv)])
        self.K[l] = np.concatenate([self.K[l], k[:, None, :]], axis=1)
        self.V[l] = np.concatenate([self.V[l], v[:, None, :]], axis=1)
        o = np.zeros((nq, hd))
        for qh in range(nq):
            kvh = qh // grp
            sc = self.K[l][kvh] @ q[qh]
            p = np.exp(sc - sc.max())
            o[qh] = (p / p.sum()) @ self.V[l][kvh]
        o = o * sigmoid(qg[:, 1])
        return h + self.W(K_ATT_O, l) @ o.reshape(-1)

    def mlp(self, l, h):
        n = rmsnorm(h, self.v(K_POST_NORM, l), self.c.rms_eps)
        g = self.W(K_FFN_GATE, l) @ n
        u = self.W(K_FFN_UP, l) @ n
        return h + self.W(K_FFN_DOWN, l) @ (silu(g) * u)

    def mixer_step(self, l, h):
        h = np.asarray(h, np.float64)
        cs = rope_cos_sin(self.pos, self.c.rope_dim, self.c.rope_base)
        out = self.attention(l, h, cs) if self.c.is_full_attention(l) else self.deltanet(l, h)
        self.pos += 1
        return out

    def forward(self, token):
        c = self.c
        h = self.embed(token)
        cs = rope_cos_sin(self.pos, c.rope_dim, c.rope_base)
        for l in range(c.n_layers):
            h = self.attention(l, h, cs) if c.is_full_attention(l) else self.deltanet(l, h)
            h = self.mlp(l, h)
        hn = rmsnorm(h, self.v(K_OUTPUT_NORM, -1), c.rms_eps)
        self.pos += 1
        return self.W(K_OUTPUT, -1) @ hn
