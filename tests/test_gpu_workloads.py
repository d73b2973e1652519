"""GPU parity at the decode benchmark's own workloads (BASELINE configs 4 and 5).

Config 4: the 1.2B hybrid with an fp16 cache filled by a 4096-token chunked
prefill (tiles of 512 rows, the matrix-core GEMM), working context 4352 (YaRN
scale 1.0625), then 256 greedy steps. The oracle continues from the state the
GPU built (exported, then imported into the oracle's fp16-rounded cache mode),
as the CPU leg of the benchmark does.

Config 4's prefill itself: the GPU's tile-512 prefill of a 1024-token prompt
at the config-4 working context (YaRN on) against the oracle's token path
over the same prompt: every fp16 K/V value within one fp16 step, the
ShortConv state within 1e-3, and the next token's logits.

Config 5: 8 sequences, each a seeded uniform-random prompt of 32768 tokens
prefilled in tiles of 512 rows into its own Q8_0 cache (working context
32896, YaRN scale 8.03), stepped together through the batched path (one GEMV
over the 8 columns per projection, one attention launch with the batch's
split count). The oracle continues each sequence from the state the GPU
built; its logits and its next 16 greedy tokens are compared.

Bars (north star): logits max |dl| <= 1e-3 * max |l_ref|; identical greedy
tokens.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import import_into_oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def img_1b2():
    from mivi_hip.synthmodel import LFM2_1B2, build_hybrid
    return build_hybrid(**LFM2_1B2, ctx_len=65536, seed=2024)


def rel_err(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b.astype(np.float64))) / np.max(np.abs(b)))


def oracle_greedy(oracle, o, tok, pos, n):
    """n greedy steps of the oracle from (tok, pos); returns (tokens, margins)
    where margin = top-1 minus top-2 logit of each step."""
    toks, margins = [], []
    for i in range(n):
        lg = o.forward(tok, pos + i)
        tok = oracle.argmax(lg)
        top2 = np.partition(lg, -2)[-2:]
        toks.append(tok)
        margins.append(float(top2[1] - top2[0]))
    return toks, margins


def first_divergence(got, want, margins):
    for i, (a, b) in enumerate(zip(got, want)):
        if a != b:
            return f"step {i}: device {a}, oracle {b}, oracle top-2 margin {margins[i]:.3g}"
    return None


def test_config4_workload_matches_oracle(hip, oracle, img_1b2):
    from mivi_hip.synthmodel import LFM2_1B2
    prefill, steps = 4096, 256
    ctx = prefill + steps
    m = hip.Model(img_1b2, max_ctx=ctx, kv_precision=hip.KvPrecision.F16)
    assert m.info.yarn == 1 and abs(m.info.yarn_scale - ctx / 4096) < 1e-6
    prompt = np.random.default_rng(11).integers(0, LFM2_1B2["vocab"], prefill + 1)
    m.set_prefill_strategy(512)
    m.prefill(prompt[:-1])
    k, v, conv = m.export_state(prefill)
    o = oracle.Model(img_1b2, max_ctx=ctx, kv_precision=oracle.KV_F16RT)
    import_into_oracle(o, k, v, conv, prefill, m.kv_row_bytes(), m.info.n_attn_layers, f16=True)
    tok = int(prompt[-1])
    lg = m.forward(tok, prefill)
    lo = o.forward(tok, prefill)
    assert rel_err(lg, lo) <= 1e-3, rel_err(lg, lo)
    first = oracle.argmax(lo)
    rest, margins = oracle_greedy(oracle, o, first, prefill + 1, steps - 1)
    want = [first] + rest
    # the same 256 steps from the same state through the captured greedy graph
    m.import_state(prefill, k, v, conv)
    got = [int(t) for t in m.generate_greedy([tok], [prefill], steps)[:, 0]]
    assert got == want, first_divergence(got, want, [0.0] + margins)


def test_config4_prefill_matches_oracle_token_path(hip, oracle, img_1b2):
    """The GPU's chunked prefill (tiles of 512 rows: the matrix-core GEMM,
    the rows' attention) against the oracle's token path (the reference's
    default strategy) over a 1024-token prompt at the config-4 working context
    (4352, YaRN on). Both caches hold fp16 roundings of nearly the same
    floats, but the two paths' projections differ in their float arithmetic
    (both far inside the 1e-4 |w| |x| bar), and the difference carries through
    the residual stream from layer to layer: measured, the K/V values beyond
    one fp16 step of each other differ by at most 3.4e-6 of their token row's
    largest value at the first attention layer and 1.3e-4 at the sixth, the
    GPU's own token path (the one-column GEMVs) drifting as far (9e-6 ...
    1.1e-4). Checked: within one fp16 step plus 2e-5 of the row's largest
    value at the first attention layer and 2e-4 at every layer, no layer
    drifting more than twice as far as the GPU token path's cache does, the
    ShortConv state within 1e-3 (measured 6.5e-6) and the next token's logits
    within 1e-3."""
    from mivi_hip.synthmodel import LFM2_1B2
    n, ctx = 1024, 4352
    prompt = np.random.default_rng(31).integers(0, LFM2_1B2["vocab"], n + 1)
    m = hip.Model(img_1b2, max_ctx=ctx, kv_precision=hip.KvPrecision.F16)
    assert m.info.yarn == 1
    m.set_prefill_strategy(512)
    m.prefill(prompt[:-1])
    k, v, conv = m.export_state(n)
    mt = hip.Model(img_1b2, max_ctx=ctx, kv_precision=hip.KvPrecision.F16)
    mt.prefill(prompt[:-1])
    kt, vt, _ = mt.export_state(n)
    o = oracle.Model(img_1b2, max_ctx=ctx, kv_precision=oracle.KV_F16RT)
    for p, t in enumerate(prompt[:-1]):
        o.forward_step(int(t), p, False)
    L, row = m.info.n_attn_layers, m.kv_row_bytes()
    ok, ov = o.kv_views()
    per = ok.size // L

    def drift(dev, ref, l):
        """max over values of (|a - b| - one fp16 step) / the token row's largest |b|"""
        a = dev[l * n * row:(l + 1) * n * row].view(np.float16).astype(np.float64).reshape(n, -1)
        b = ref[l * per:l * per + n * row * 2].view(np.float32).astype(np.float64).reshape(n, -1)
        step = np.spacing(np.maximum(np.abs(a), np.abs(b)).astype(np.float16)).astype(np.float64)
        scale = np.maximum(np.max(np.abs(b), axis=1, keepdims=True), 1e-30)
        return float(np.max((np.abs(a - b) - step) / scale))

    for name, dev, tok_dev, ref in (("K", k, kt, ok), ("V", v, vt, ov)):
        for l in range(L):
            dt, dtok = drift(dev, ref, l), drift(tok_dev, ref, l)
            assert dt <= (2e-5 if l == 0 else 2e-4), (name, l, dt)
            assert dt <= 2 * dtok + 1e-5, (name, l, dt, dtok)
    oc = o.conv_view()
    assert np.max(np.abs(conv.astype(np.float64) - oc)) <= 1e-3 * np.max(np.abs(oc))
    tok = int(prompt[-1])
    assert rel_err(m.forward(tok, n), o.forward(tok, n)) <= 1e-3


def test_config5_workload_matches_oracle(hip, oracle, img_1b2):
    from mivi_hip.synthmodel import LFM2_1B2
    batch, cached, greedy = 8, 32768, 16
    ctx = cached + 128
    m = hip.Model(img_1b2, max_ctx=ctx, kv_precision=hip.KvPrecision.Q8_0, max_batch=batch)
    info = m.info
    assert info.yarn == 1 and abs(info.yarn_scale - ctx / 4096) < 1e-6
    L, row = info.n_attn_layers, m.kv_row_bytes()
    prompts = np.random.default_rng(12).integers(0, LFM2_1B2["vocab"], (batch, cached + 1))
    m.set_prefill_strategy(512)
    for b in range(batch):
        m.prefill(prompts[b, :-1], 0, seq=b)
    states = [m.export_state(cached, seq=b) for b in range(batch)]
    toks = [int(prompts[b, -1]) for b in range(batch)]
    lg = m.forward_batch(toks, [cached] * batch)
    nxt = [int(np.argmax(lg[b])) for b in range(batch)]
    got = m.generate_greedy(nxt, [cached + 1] * batch, greedy - 1)
    o = oracle.Model(img_1b2, max_ctx=ctx, kv_precision=oracle.KV_Q8_0)
    for b in range(batch):
        o.reset()
        import_into_oracle(o, *states[b], cached, row, L)
        lo = o.forward(toks[b], cached)
        assert rel_err(lg[b], lo) <= 1e-3, (b, rel_err(lg[b], lo))
        first = oracle.argmax(lo)
        assert nxt[b] == first, b
        want, margins = oracle_greedy(oracle, o, first, cached + 1, greedy - 1)
        assert [int(t) for t in got[:, b]] == want, (b, first_divergence(list(got[:, b]), want, margins))
