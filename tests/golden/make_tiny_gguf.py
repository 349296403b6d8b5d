"""Writes tests/golden/tiny.gguf: a small GGUF v3 file with known content, for the parser test
(tests/test_gguf_cpu.py holds the expected values).

Metadata: general.architecture = "qwen35" (string), general.alignment = 64 (u64, the type the
reference's parser honours), qwen35.block_count = 2 (u32), qwen35.embedding_length = 256 (u32),
qwen35.attention.layer_norm_rms_epsilon = 1e-5 (f32), general.name = "tiny" (string),
qwen35.rope.dimension_sections = [11, 11, 10, 0] (i32 array), tokenizer.ggml.merges = ["a b", "c d"]
(string array), general.flag = true (bool), general.count = -3 (i64), general.ratio = 0.25 (f64).
Tensors (GGUF dims, innermost first):
  blk.0.ffn_up.weight  Q1_0 [256, 4]  bytes b[i] = (7*i + 3) & 0xFF, 144 bytes
  output_norm.weight   F32  [256]     values 0.5 + i/256
  token_embd.weight    F16  [256, 3]  values (i % 17) - 8 as f16
each at a multiple of 64 from the data section's start.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from gguf_writer import ARR, BOOL, F32, F64, I32, I64, STR, U32, U64, write_gguf  # noqa: E402


def tiny():
    q = ((7 * np.arange(144) + 3) & 0xFF).astype(np.uint8)
    norm = (0.5 + np.arange(256) / 256.0).astype(np.float32)
    emb = ((np.arange(768) % 17) - 8).astype(np.float16)
    md = [
        ("general.architecture", STR, "qwen35"),
        ("general.alignment", U64, 64),
        ("qwen35.block_count", U32, 2),
        ("qwen35.embedding_length", U32, 256),
        ("qwen35.attention.layer_norm_rms_epsilon", F32, 1e-5),
        ("general.name", STR, "tiny"),
        ("qwen35.rope.dimension_sections", ARR, (I32, [11, 11, 10, 0])),
        ("tokenizer.ggml.merges", ARR, (STR, ["a b", "c d"])),
        ("general.flag", BOOL, True),
        ("general.count", I64, -3),
        ("general.ratio", F64, 0.25),
    ]
    tensors = [
        ("blk.0.ffn_up.weight", 41, (256, 4), q.tobytes()),
        ("output_norm.weight", 0, (256,), norm.tobytes()),
        ("token_embd.weight", 1, (256, 3), emb.tobytes()),
    ]
    return md, tensors


if __name__ == "__main__":
    md, tensors = tiny()
    data = write_gguf(os.path.join(HERE, "tiny.gguf"), md, tensors, alignment=64)
    print("wrote tiny.gguf, %d bytes" % len(data))
