"""GGUF-named tensors of the oracle's synthetic model (the names LoadedWeights::load_all reads,
Daiza-engine/src/model/weights.rs:1308-1379), for dz_model_create and the GGUF writer.

Test infrastructure: the bytes come from the oracle's generator (include/daiza_synth.h), so a
model built from them must equal dz_model_create_synth with the same seed.
"""
import numpy as np

# stream kinds of include/daiza_synth.h
K_EMBD, K_OUTPUT_NORM, K_OUTPUT = 1, 2, 3
K_ATTN_NORM, K_POST_NORM, K_FFN_GATE, K_FFN_UP, K_FFN_DOWN = 16, 17, 18, 19, 20
K_SSM_QKV, K_SSM_ALPHA, K_SSM_BETA, K_SSM_Z, K_SSM_OUT, K_SSM_CONV, K_SSM_A, K_SSM_DT, K_SSM_NORM = range(32, 41)
K_ATT_Q, K_ATT_K, K_ATT_V, K_ATT_O, K_ATT_QNORM, K_ATT_KNORM = range(48, 54)

F32, F16, Q1_0 = 0, 1, 41


def named_tensors(oracle, om, cfg, seed):
    """{name: (gguf type, array)} for the oracle model `om` (built from cfg and seed)."""
    t = {}

    def q1(name, kind, layer):
        b, _, _ = om.q1(kind, layer)
        t[name] = (Q1_0, np.array(b, np.uint8))

    def f32(name, kind, layer):
        t[name] = (F32, om.f32(kind, layer).astype(np.float32))

    qkvd = cfg.qkv_dim
    for i in range(cfg.n_layers):
        b = "blk.%d." % i
        f32(b + "attn_norm.weight", K_ATTN_NORM, i)
        f32(b + "post_attention_norm.weight", K_POST_NORM, i)
        q1(b + "ffn_gate.weight", K_FFN_GATE, i)
        q1(b + "ffn_up.weight", K_FFN_UP, i)
        q1(b + "ffn_down.weight", K_FFN_DOWN, i)
        if cfg.is_full_attention(i):
            q1(b + "attn_q.weight", K_ATT_Q, i)
            q1(b + "attn_k.weight", K_ATT_K, i)
            q1(b + "attn_v.weight", K_ATT_V, i)
            q1(b + "attn_output.weight", K_ATT_O, i)
            f32(b + "attn_q_norm.weight", K_ATT_QNORM, i)
            f32(b + "attn_k_norm.weight", K_ATT_KNORM, i)
        else:
            q1(b + "attn_qkv.weight", K_SSM_QKV, i)
            q1(b + "attn_gate.weight", K_SSM_Z, i)
            q1(b + "ssm_alpha.weight", K_SSM_ALPHA, i)
            q1(b + "ssm_beta.weight", K_SSM_BETA, i)
            q1(b + "ssm_out.weight", K_SSM_OUT, i)
            # the oracle keeps the conv taps transposed [tap][channel] (weights.rs:1339-1356); GGUF
            # holds them [channel][tap]
            conv_t = om.f32(K_SSM_CONV, i).reshape(cfg.ssm_conv_kernel, qkvd)
            t[b + "ssm_conv1d.weight"] = (F32, np.ascontiguousarray(conv_t.T).astype(np.float32))
            f32(b + "ssm_a", K_SSM_A, i)
            f32(b + "ssm_dt.bias", K_SSM_DT, i)
            f32(b + "ssm_norm.weight", K_SSM_NORM, i)
    f32("output_norm.weight", K_OUTPUT_NORM, -1)
    q1("output.weight", K_OUTPUT, -1)
    if cfg.embd_f16:
        emb = np.stack([oracle.synth_embd_row_f16(seed, tok, cfg.hidden) for tok in range(cfg.vocab)])
        t["token_embd.weight"] = (F16, emb.astype(np.uint16))
    else:
        q1("token_embd.weight", K_EMBD, -1)
    return t
