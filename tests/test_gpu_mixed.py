"""GPU parity of mixed-format (Q4_K_M) models against the CPU oracle.

A Q4_K_M file is not all Q4_K: its 1.2B LFM2 file keeps 11 matrices in Q6_K
(CHANGELOG.md:584-586), the embedding and ffn_down / attn_v of selected
layers. `quantized_matvec` and `quantized_matmul_rows` serve every
projection through one type dispatch (crates/mivi-quant/src/lib.rs:89-131,
143-357), and so does this build: here the one-column decode GEMVs stream
the Q6_K projections packed (row quads at 2048 columns, unit planes at
8192), q|k and the Q6_K v run as two launches, and the chunked prefill runs
the Q6_K products on the matrix cores (gemm_q6k_kernel). The model below
has dim 2048 and hidden 8192, so every one of those paths is the one the
1.2B shape takes.

Bars (north star): logits within 1e-3 relative; identical greedy tokens.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# Q6_K: blk.2.ffn_down, blk.3.ffn_down, blk.3.attn_v (the Q4_K_M choice for 4 layers / 2 attention layers)
MIXED = dict(dim=2048, hidden=8192, n_layers=4, attn_layers=(1, 3), n_heads=32, n_kv=8, vocab=4096)


def rel_err(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b.astype(np.float64))) / np.max(np.abs(b)))


@pytest.fixture(scope="module")
def mixed_img():
    from mivi_hip.synthmodel import build_hybrid
    return build_hybrid(**MIXED, ctx_len=8192, seed=61, mixed="q4_k_m")


def oracle_run(oracle, img, prompt, n_greedy, max_ctx=1024):
    """The oracle's token path over prompt[:-1], the last token's logits, and
    n_greedy greedy tokens after it."""
    o = oracle.Model(img, max_ctx=max_ctx)
    for p, t in enumerate(prompt[:-1]):
        o.forward_step(int(t), p, False)
    n = len(prompt) - 1
    lo = o.forward(int(prompt[-1]), n)
    toks, t = [], oracle.argmax(lo)
    for i in range(n_greedy):
        toks.append(t)
        t = oracle.argmax(o.forward(t, n + 1 + i))
    o.close()
    return lo, toks


def test_mixed_model_types_and_weight_bytes(hip, mixed_img):
    from mivi_hip.gguf import read_tensor_index
    idx = read_tensor_index(mixed_img)
    q6 = sorted(n for n, (t, dims, off, ln) in idx.items() if t == 14 and len(dims) == 2)
    assert q6 == ["blk.2.ffn_down.weight", "blk.3.attn_v.weight", "blk.3.ffn_down.weight", "token_embd.weight"]
    data = len(mixed_img) - min(off for (t, dims, off, ln) in idx.values())
    packed = sum(ln for (t, dims, off, ln) in idx.values() if t in (12, 14) and len(dims) == 2)
    # the Q4_K projections' B operand for the prefill's row products: fp16
    # sc * q plus 640 bytes per 32 rows and super-block (dims: cols, rows)
    gemm = sum(d[1] * d[0] * 2 + d[1] // 32 * (d[0] // 256) * 640 for (t, d, off, ln) in idx.values()
               if t == 12 and len(d) == 2 and d[1] % 32 == 0 and d[0] % 2048 == 0)
    # every projection packed beside its GGUF rows, the (tied) head too
    assert hip.Model(mixed_img, max_ctx=256).info.weight_bytes == data + packed + gemm
    os.environ["MIVI_NO_GEMM_PACK"] = "1"
    try:
        assert hip.Model(mixed_img, max_ctx=256).info.weight_bytes == data + packed
    finally:
        del os.environ["MIVI_NO_GEMM_PACK"]
    os.environ["MIVI_NO_PACK"] = "1"
    try:
        assert hip.Model(mixed_img, max_ctx=256).info.weight_bytes == data
    finally:
        del os.environ["MIVI_NO_PACK"]


def test_mixed_token_path_matches_oracle(hip, oracle, mixed_img):
    # the one-column decode step: packed Q6_K v (row quads, RMSNorm prologue)
    # beside q|k on the Q4_K row quads, packed Q6_K ffn_down (unit planes, K
    # = 8192); every step's logits, then 16 greedy steps
    m = hip.Model(mixed_img, max_ctx=1024)
    o = oracle.Model(mixed_img, max_ctx=1024)
    toks = np.random.default_rng(62).integers(0, MIXED["vocab"], 40)
    worst = 0.0
    for p, t in enumerate(toks):
        worst = max(worst, rel_err(m.forward(int(t), p), o.forward(int(t), p)))
    assert worst <= 1e-3, worst
    n = len(toks)
    lo = o.forward(7, n)
    assert rel_err(m.forward(7, n), lo) <= 1e-3
    first = oracle.argmax(lo)
    want, t = [], first
    for i in range(16):
        t = oracle.argmax(o.forward(t, n + 1 + i))
        want.append(t)
    assert list(m.generate_greedy([first], [n + 1], 16)[:, 0]) == want


@pytest.mark.parametrize("tile", [64, 512])
def test_mixed_chunked_prefill_matches_oracle(hip, oracle, mixed_img, tile):
    # PrefillStrategy::Chunked on a 600-token prompt (tile 512: 512 + 87
    # rows, tile 64: nine tiles + 23 rows): the Q6_K ffn_down and v products
    # on the matrix cores with the Q4_K ones; the next token's logits and 8
    # greedy tokens against the oracle's token path
    prompt = np.random.default_rng(63).integers(0, MIXED["vocab"], 600)
    lo, want = oracle_run(oracle, mixed_img, prompt, 8)
    m = hip.Model(mixed_img, max_ctx=1024)
    m.set_prefill_strategy(tile)
    m.prefill(prompt[:-1])
    n = len(prompt) - 1
    lg = m.forward(int(prompt[-1]), n)
    assert rel_err(lg, lo) <= 1e-3, rel_err(lg, lo)
    assert int(np.argmax(lg)) == want[0]
    assert list(m.generate_greedy([want[0]], [n + 1], 7)[:, 0]) == want[1:]


@pytest.mark.parametrize("B", [3, 8])
def test_mixed_batched_decode_matches_oracle(hip, oracle, mixed_img, B):
    # one batched step over B sequences (Q6_K v and ffn_down as multi-column
    # GEMVs on the GGUF rows), each sequence's logits against its own oracle
    # run, then 6 batched greedy steps against each sequence's own
    # single-sequence run
    rng = np.random.default_rng(64 + B)
    prompts = [rng.integers(0, MIXED["vocab"], 5 + 4 * b) for b in range(B)]
    mb = hip.Model(mixed_img, max_ctx=256, max_batch=B)
    for b, pr in enumerate(prompts):
        mb.prefill(pr[:-1], seq=b)
    lg = mb.forward_batch([int(p[-1]) for p in prompts], [len(p) - 1 for p in prompts])
    for b, pr in enumerate(prompts):
        lo, _ = oracle_run(oracle, mixed_img, pr, 0, max_ctx=256)
        assert rel_err(lg[b], lo) <= 1e-3, (b, rel_err(lg[b], lo))
    nxt = [int(np.argmax(lg[b])) for b in range(B)]
    out = mb.generate_greedy(nxt, [len(p) for p in prompts], 6)
    for b, pr in enumerate(prompts):
        m1 = hip.Model(mixed_img, max_ctx=256)
        m1.prefill(pr[:-1])
        m1.forward(int(pr[-1]), len(pr) - 1)
        assert np.array_equal(out[:, b], m1.generate_greedy([nxt[b]], [len(pr)], 6)[:, 0]), b
