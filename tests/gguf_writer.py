"""A GGUF v3 writer (test infrastructure): the container layout of the GGUF specification, as the
reference's parser reads it (Daiza-engine/src/gguf/parser.rs:40-119, metadata.rs,
tensor_info.rs:41-201): magic "GGUF", version 3, tensor count, metadata count, the metadata entries
{key, u32 type, value}, the tensor infos {name, n_dims, dims (innermost first), u32 type, u64
offset}, then the data section at the next multiple of the alignment, each tensor at its offset.
"""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _scalar(t, v):
    return _str(v) if t == STR else struct.pack(_FMT[t], v)


def write_gguf(path, metadata, tensors, alignment=32):
    """metadata: [(key, type, value)] with type ARR given as (ARR, (elem_type, [values]));
    tensors: [(name, ggml type, dims innermost first, bytes)].  Tensor data is placed in order at
    multiples of `alignment` (the data-section alignment the reader assumes).  Returns the file's
    bytes."""
    out = bytearray(b"GGUF")
    out += struct.pack("<IQQ", 3, len(tensors), len(metadata))
    for key, t, v in metadata:
        out += _str(key) + struct.pack("<I", t)
        if t == ARR:
            et, vals = v
            out += struct.pack("<IQ", et, len(vals)) + b"".join(_scalar(et, x) for x in vals)
        else:
            out += _scalar(t, v)
    offs, off = [], 0
    for name, ty, dims, data in tensors:
        offs.append(off)
        off = (off + len(data) + alignment - 1) // alignment * alignment
    for (name, ty, dims, data), o in zip(tensors, offs):
        out += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", ty, o)
    out += b"\0" * ((-len(out)) % alignment)
    base = len(out)
    for (name, ty, dims, data), o in zip(tensors, offs):
        out += b"\0" * (base + o - len(out))
        out += bytes(data)
    with open(path, "wb") as f:
        f.write(out)
    return bytes(out)


def model_metadata(cfg, eos=248046, int_tokens=True):
    """The qwen35.* keys Config::from_metadata reads (model/config.rs:76-160) for cfg; the vocabulary
    as an int32 tokenizer.ggml.tokens array (the reference counts an integer array's length)."""
    md = [
        ("general.architecture", STR, "qwen35"),
        ("qwen35.block_count", U32, cfg.n_layers),
        ("qwen35.context_length", U64, 262144),
        ("qwen35.embedding_length", U32, cfg.hidden),
        ("qwen35.feed_forward_length", U32, cfg.ffn),
        ("qwen35.attention.head_count", U32, cfg.n_head),
        ("qwen35.attention.head_count_kv", U32, cfg.n_head_kv),
        ("qwen35.attention.key_length", U32, cfg.head_dim),
        ("qwen35.attention.layer_norm_rms_epsilon", F32, cfg.rms_eps),
        ("qwen35.rope.dimension_count", U32, cfg.rope_dim),
        ("qwen35.rope.dimension_sections", ARR, (I32, [11, 11, 10, 0])),
        ("qwen35.rope.freq_base", F32, cfg.rope_base),
        ("qwen35.full_attention_interval", U32, cfg.full_attn_interval),
        ("qwen35.ssm.conv_kernel", U32, cfg.ssm_conv_kernel),
        ("qwen35.ssm.state_size", U32, cfg.ssm_state),
        ("qwen35.ssm.group_count", U32, cfg.ssm_k_heads),
        ("qwen35.ssm.time_step_rank", U32, cfg.ssm_v_heads),
        ("qwen35.ssm.inner_size", U32, cfg.ssm_v_heads * cfg.ssm_state),
        ("tokenizer.ggml.eos_token_id", U32, eos),
    ]
    if int_tokens:
        md.append(("tokenizer.ggml.tokens", ARR, (I32, list(range(cfg.vocab)))))
    return md


def model_tensors(named, cfg):
    """[(name, type, dims, bytes)] from named_tensors() output, with GGUF dims."""
    out = []
    H = cfg.hidden
    for name, (ty, a) in named.items():
        a = np.ascontiguousarray(a)
        if ty == 41:
            # K of each Q1_0 matrix from its name (the rows follow from the bytes)
            if name.endswith("ffn_down.weight"):
                K = cfg.ffn
            elif name.endswith("ssm_out.weight"):
                K = cfg.ssm_v_heads * cfg.ssm_state
            elif name.endswith("attn_output.weight"):
                K = cfg.n_head * cfg.head_dim
            else:
                K = H
            rows = a.size // (K // 128 * 18)
            dims = (K, rows)
        elif name.endswith("ssm_conv1d.weight"):
            dims = (cfg.ssm_conv_kernel, a.size // cfg.ssm_conv_kernel)
        elif name == "token_embd.weight":
            dims = (H, cfg.vocab)
        else:
            dims = (a.size,)
        out.append((name, ty, dims, a.tobytes()))
    return out
