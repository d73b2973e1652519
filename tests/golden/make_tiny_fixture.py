"""Rebuilds tests/golden/tiny_model.gguf, the input of the reference's
whole-model golden vectors (tests/golden/oracle_output.json, copied from the
reference's tests/fixtures/oracle_output.json).

The reference produces its tiny test model with
training/export/generate_fixture.py:20-154 and quantizes it with
training/export/convert_to_gguf.py:135-156. This script restates those
published steps (it does not import the reference):

* weight matrices: a double-precision recurrence
  v <- (v * 1.337 + 0.123) mod 1 - 0.5, element = round(v * 0.2, 4)
  (generate_fixture.py:20-29), seeded per tensor;
* norm/conv vectors: v <- (v * 1.414 + 0.271) mod 1 - 0.5,
  element = round(v * 0.1 + scale, 4) (generate_fixture.py:32-38);
* matrices are stored Q8_0 with Python-double arithmetic: d = max|x| / 127
  (1e-6 if the block is zero), the scale stored as float16(d) (round to
  nearest even), q = round-half-even(x / d) clamped to [-128, 127]
  (convert_to_gguf.py:135-156); vectors are stored F32.

Run: python tests/golden/make_tiny_fixture.py  (writes tiny_model.gguf)
"""
from __future__ import annotations

import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "mivi-v4_amd"))
from mivi_hip.gguf import GGML_F32, GGML_Q8_0, GgufWriter  # noqa: E402

DIM, HIDDEN, N_LAYERS, N_HEADS, N_KV, HEAD_DIM, KV_DIM, VOCAB, MAX_SEQ = 64, 128, 2, 2, 1, 32, 32, 64, 512
ROPE_BASE = 1_000_000.0
TOKENS = [1, 5, 12, 3]


def det_matrix(rows: int, cols: int, seed: float) -> list:
    v = seed
    out = []
    for _ in range(rows):
        row = []
        for _ in range(cols):
            v = (v * 1.337 + 0.123) % 1.0 - 0.5
            row.append(round(v * 0.2, 4))
        out.append(row)
    return out


def det_vector(n: int, scale: float) -> list:
    v = 0.5
    out = []
    for _ in range(n):
        v = (v * 1.414 + 0.271) % 1.0 - 0.5
        out.append(round(v * 0.1 + scale, 4))
    return out


def q8_0_python(flat: list) -> bytes:
    assert len(flat) % 32 == 0
    out = bytearray()
    for i in range(0, len(flat), 32):
        chunk = flat[i: i + 32]
        amax = max(abs(x) for x in chunk) or 1e-6
        d = amax / 127.0
        out += np.float16(d).tobytes()
        inv = 1.0 / d
        for x in chunk:
            q = max(-128, min(127, int(round(x * inv))))
            out += struct.pack("b", q)
    return bytes(out)


def build() -> np.ndarray:
    w = {}
    w["token_embd.weight"] = det_matrix(VOCAB, DIM, 0.15)
    w["output.weight"] = det_matrix(VOCAB, DIM, 0.25)
    w["output_norm.weight"] = det_vector(DIM, 1.0)
    w["blk.0.ssm_norm.weight"] = det_vector(DIM, 1.0)
    w["blk.0.shortconv.in_proj.weight"] = det_matrix(3 * DIM, DIM, 0.3)
    w["blk.0.shortconv.conv.weight"] = det_vector(3 * DIM, 0.25)
    w["blk.0.shortconv.out_proj.weight"] = det_matrix(DIM, DIM, 0.4)
    w["blk.0.ffn_norm.weight"] = det_vector(DIM, 1.0)
    w["blk.0.ffn_gate.weight"] = det_matrix(HIDDEN, DIM, 0.5)
    w["blk.0.ffn_up.weight"] = det_matrix(HIDDEN, DIM, 0.6)
    w["blk.0.ffn_down.weight"] = det_matrix(DIM, HIDDEN, 0.7)
    w["blk.1.attn_norm.weight"] = det_vector(DIM, 1.0)
    w["blk.1.attn_q.weight"] = det_matrix(DIM, DIM, 0.8)
    w["blk.1.attn_k.weight"] = det_matrix(KV_DIM, DIM, 0.9)
    w["blk.1.attn_v.weight"] = det_matrix(KV_DIM, DIM, 1.1)
    w["blk.1.attn_output.weight"] = det_matrix(DIM, DIM, 1.2)
    w["blk.1.ffn_norm.weight"] = det_vector(DIM, 1.0)
    w["blk.1.ffn_gate.weight"] = det_matrix(HIDDEN, DIM, 1.3)
    w["blk.1.ffn_up.weight"] = det_matrix(HIDDEN, DIM, 1.4)
    w["blk.1.ffn_down.weight"] = det_matrix(DIM, HIDDEN, 1.5)

    g = GgufWriter()
    g.add_string("general.architecture", "lfm")
    g.add_string("general.name", "mivi-tiny-test")
    g.add_u32("lfm.context_length", MAX_SEQ)
    g.add_u32("lfm.embedding_length", DIM)
    g.add_u32("lfm.block_count", N_LAYERS)
    g.add_u32("lfm.feed_forward_length", HIDDEN)
    g.add_u32("lfm.attention.head_count", N_HEADS)
    g.add_u32("lfm.attention.head_count_kv", N_KV)
    g.add_f32("lfm.rope.freq_base", ROPE_BASE)
    toks = [f"<tok_{i}>" for i in range(VOCAB)]
    toks[0], toks[1] = "<|im_start|>", "<|im_end|>"
    g.add_string_array("tokenizer.ggml.tokens", toks)
    for name, data in w.items():
        if isinstance(data[0], list):
            rows, cols = len(data), len(data[0])
            flat = [v for r in data for v in r]
            g.add_tensor(name, [cols, rows], GGML_Q8_0, np.frombuffer(q8_0_python(flat), np.uint8))
        else:
            g.add_tensor(name, [len(data)], GGML_F32, np.asarray(data, np.float32))
    return g.tobytes()


if __name__ == "__main__":
    img = build()
    path = os.path.join(HERE, "tiny_model.gguf")
    img.tofile(path)
    print(f"wrote {path} ({img.nbytes} bytes)")
