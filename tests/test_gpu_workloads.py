"""GPU parity at the decode benchmark's own workloads (BASELINE configs 4 and 5).

Config 4: the 1.2B hybrid with an fp16 cache filled by a 4096-token chunked
prefill (tiles of 512 rows, the matrix-core GEMM), working context 4352 (YaRN
scale 1.0625), then 256 greedy steps. The oracle continues from the state the
GPU built (exported, then imported into the oracle's fp16-rounded cache mode),
as the CPU leg of the benchmark does.

Config 5: 8 sequences with Q8_0 caches of 32768 tokens each (working context
32896, YaRN scale 8.03), stepped together through the batched path (one GEMV
over the 8 columns per projection, one attention launch with the batch's
split count). Each sequence's logits and its next greedy tokens are compared
with its own oracle run from the same imported state.

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


def test_config5_workload_matches_oracle(hip, oracle, img_1b2):
    from mivi_hip.synthmodel import LFM2_1B2
    batch, cached, greedy = 8, 32768, 4
    ctx = cached + 128
    m = hip.Model(img_1b2, max_ctx=ctx, kv_precision=hip.KvPrecision.Q8_0, max_batch=batch)
    info = m.info
    assert info.yarn == 1 and abs(info.yarn_scale - ctx / 4096) < 1e-6
    L, kvd, row = info.n_attn_layers, info.kv_dim, m.kv_row_bytes()

    def state(b):  # the benchmark's synthetic caches and ShortConv states
        k = hip.synth_random_weights(hip.GgmlType.Q8_0, 500 + 2 * b, L * cached, kvd, 1.0)
        v = hip.synth_random_weights(hip.GgmlType.Q8_0, 501 + 2 * b, L * cached, kvd, 1.0)
        return k, v, hip.synth_normal(600 + b, m.conv_len(), std=0.1)

    for b in range(batch):
        m.import_state(cached, *state(b), seq=b)
    toks = [int(t) for t in np.random.default_rng(12).integers(0, LFM2_1B2["vocab"], batch)]
    lg = m.forward_batch(toks, [cached] * batch)
    nxt = [int(np.argmax(lg[b])) for b in range(batch)]
    got = m.generate_greedy(nxt, [cached + 1] * batch, greedy)
    o = oracle.Model(img_1b2, max_ctx=ctx, kv_precision=oracle.KV_Q8_0)
    for b in range(batch):
        o.reset()
        import_into_oracle(o, *state(b), cached, row, L)
        lo = o.forward(toks[b], cached)
        assert rel_err(lg[b], lo) <= 1e-3, (b, rel_err(lg[b], lo))
        first = oracle.argmax(lo)
        assert nxt[b] == first, b
        want, margins = oracle_greedy(oracle, o, first, cached + 1, greedy)
        assert [int(t) for t in got[:, b]] == want, (b, first_divergence(list(got[:, b]), want, margins))
