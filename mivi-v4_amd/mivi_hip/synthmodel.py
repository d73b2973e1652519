"""Random-init LFM2-style hybrid models as GGUF images.

The benchmark/test model of the hybrid decode path: `n_layers` blocks, the
ones listed in `attn_layers` grouped-query attention, the rest gated
ShortConv, each followed by a SwiGLU FFN (crates/mivi-model/src/{ssm,
transformer,ffn}.rs). Projections are seeded N(0, std) quantized to
`weight_type`; the embedding is `embd_type` and is tied to the output head
when `tied` (model.rs:455-459). RMSNorm weights are 1.0 and ShortConv
weights are N(0, conv_std) stored F32: the reference leaves both open for a
random-init model, these are the values this build uses.

Tensor names and metadata keys are the ones the reference loader resolves
(loader.rs:33-177, 253-415).

mixed="q4_k_m" gives the mixed-format layout of a Q4_K_M file: ffn_down of
the first and last eighth of the layers and of every third layer in
between, and attn_v of the same selection over the attention layers, in
Q6_K, everything else `weight_type`. For the 1.2B shape that is 8 ffn_down
and 2 attn_v matrices, 11 Q6_K matrices with the embedding: the count the
reference reports for its 1.2B Q4_K_M file (CHANGELOG.md:584-586).
"""
from __future__ import annotations

import numpy as np

from . import GgmlType, synth_normal, synth_random_weights
from .gguf import GGML_F32, GgufWriter

LFM2_1B2 = dict(dim=2048, hidden=8192, n_layers=16, attn_layers=(2, 5, 8, 11, 13, 15), n_heads=32, n_kv=8,
                vocab=65536)


def more_bits(i: int, n: int) -> bool:
    """Whether the i-th of n like matrices of a Q4_K_M file is Q6_K: the
    first and last eighth, and every third one in between."""
    return i < n // 8 or i >= 7 * n // 8 or (i - n // 8) % 3 == 2


def q6k_matrices(n_layers: int, attn_layers, mixed) -> set:
    """Names of the projections a `mixed` layout stores as Q6_K."""
    if mixed is None:
        return set()
    if mixed != "q4_k_m":
        raise ValueError(f"unknown mixed layout {mixed!r}")
    attn = sorted(attn_layers)
    out = {f"blk.{i}.ffn_down.weight" for i in range(n_layers) if more_bits(i, n_layers)}
    out |= {f"blk.{l}.attn_v.weight" for j, l in enumerate(attn) if more_bits(j, len(attn))}
    return out


def build_hybrid(dim: int, hidden: int, n_layers: int, attn_layers, n_heads: int, n_kv: int, vocab: int,
                 ctx_len: int = 65536, weight_type=GgmlType.Q4_K, embd_type=GgmlType.Q6_K, seed: int = 1234,
                 std: float = 0.02, conv_std: float = 0.02, tied: bool = True, qk_norm: bool = False,
                 rope_base: float = 1_000_000.0, mixed=None) -> np.ndarray:
    head_dim = dim // n_heads
    kv_dim = n_kv * head_dim
    g = GgufWriter()
    g.add_string("general.architecture", "lfm2")
    g.add_string("general.name", f"mivi-hip-synthetic-{dim}x{n_layers}")
    g.add_u32("lfm2.context_length", ctx_len)
    g.add_u32("lfm2.embedding_length", dim)
    g.add_u32("lfm2.feed_forward_length", hidden)
    g.add_u32("lfm2.block_count", n_layers)
    g.add_u32("lfm2.attention.head_count", n_heads)
    g.add_u32_array("lfm2.attention.head_count_kv", [n_kv if i in attn_layers else 0 for i in range(n_layers)])
    g.add_f32("lfm2.rope.freq_base", rope_base)
    g.add_f32("lfm2.attention.layer_norm_rms_epsilon", 1e-5)
    g.add_u32("lfm2.ssm.conv_kernel", 3)
    # the loader takes vocab_size from the token list (loader.rs:146-148, model.rs:112-113)
    g.add_string_array("tokenizer.ggml.tokens", [f"<t{i}>" for i in range(vocab)])
    s = [seed * 1000]

    def nxt():
        s[0] += 1
        return s[0]

    q6 = q6k_matrices(n_layers, attn_layers, mixed)

    def mat(name, rows, cols, t=None):
        t = t if t is not None else GgmlType.Q6_K if name in q6 else weight_type
        g.add_matrix(name, rows, cols, int(t), synth_random_weights(t, nxt(), rows, cols, std))

    ones = np.ones(dim, np.float32)
    g.add_tensor("token_embd.weight", [dim, vocab], int(embd_type),
                 synth_random_weights(embd_type, nxt(), vocab, dim, std))
    g.add_f32_vector("output_norm.weight", ones)
    if not tied:
        mat("output.weight", vocab, dim, embd_type)
    for i in range(n_layers):
        p = f"blk.{i}."
        if i in attn_layers:
            g.add_f32_vector(p + "attn_norm.weight", ones)
            mat(p + "attn_q.weight", dim, dim)
            mat(p + "attn_k.weight", kv_dim, dim)
            mat(p + "attn_v.weight", kv_dim, dim)
            mat(p + "attn_output.weight", dim, dim)
            if qk_norm:
                # seeds of their own: every other tensor equals the qk_norm=False model's
                qs = seed * 1000 + 900_000 + 2 * i
                g.add_f32_vector(p + "attn_q_norm.weight", 1.0 + synth_normal(qs, head_dim, 0.0, 0.1))
                g.add_f32_vector(p + "attn_k_norm.weight", 1.0 + synth_normal(qs + 1, head_dim, 0.0, 0.1))
        else:
            g.add_f32_vector(p + "ssm_norm.weight", ones)
            mat(p + "shortconv.in_proj.weight", 3 * dim, dim)
            g.add_tensor(p + "shortconv.conv.weight", [3, dim], GGML_F32, synth_normal(nxt(), 3 * dim, 0.0, conv_std))
            mat(p + "shortconv.out_proj.weight", dim, dim)
        g.add_f32_vector(p + "ffn_norm.weight", ones)
        mat(p + "ffn_gate.weight", hidden, dim)
        mat(p + "ffn_up.weight", hidden, dim)
        mat(p + "ffn_down.weight", dim, hidden)
    return g.tobytes()


def weight_bytes_per_token(dim, hidden, n_layers, attn_layers, n_heads, n_kv, vocab, weight_type=GgmlType.Q4_K,
                           embd_type=GgmlType.Q6_K, mixed=None, **_) -> int:
    """Packed weight bytes a decode step streams (every projection + head)."""
    wt, et = GgmlType(weight_type), GgmlType(embd_type)
    q6 = q6k_matrices(n_layers, attn_layers, mixed)

    def rb(name, cols):
        t = GgmlType.Q6_K if name in q6 else wt
        return cols // t.block_size() * t.type_size()

    kv_dim = n_kv * (dim // n_heads)
    total = vocab * (dim // et.block_size() * et.type_size())
    for i in range(n_layers):
        p = f"blk.{i}."
        if i in attn_layers:
            total += 2 * dim * rb(p + "attn_q.weight", dim) + kv_dim * rb(p + "attn_k.weight", dim)
            total += kv_dim * rb(p + "attn_v.weight", dim)
        else:
            total += 4 * dim * rb(p + "shortconv.in_proj.weight", dim)
        total += 2 * hidden * rb(p + "ffn_gate.weight", dim) + dim * rb(p + "ffn_down.weight", hidden)
    return total
