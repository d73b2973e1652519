"""Pins the oracle's mivi-core numerics and whole-model forward (CPU only)."""
from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest

from conftest import GOLDEN


def test_rms_norm_closed_forms(oracle):
    # crates/mivi-core/src/math.rs:188-197
    out = oracle.rms_norm(np.array([1, 2, 3, 4], np.float32), np.ones(4, np.float32))
    assert abs(math.sqrt(float(np.mean(out.astype(np.float64) ** 2))) - 1.0) < 1e-3
    # crates/mivi-model/src/prefill.rs:307-312: (3, 4, 0, 0) -> 1.2, 1.6
    out = oracle.rms_norm(np.array([3, 4, 0, 0], np.float32), np.ones(4, np.float32))
    assert abs(out[0] - 1.2) < 0.01 and abs(out[1] - 1.6) < 0.01
    # f64 closed form over a long vector with a tail (len % 8 != 0)
    x = np.random.default_rng(0).standard_normal(2051).astype(np.float32)
    w = np.random.default_rng(1).standard_normal(2051).astype(np.float32)
    ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5) * w
    assert np.allclose(oracle.rms_norm(x, w), ref, rtol=1e-5, atol=1e-6)


def test_softmax_silu_swiglu(oracle):
    # math.rs:199-241 and prefill.rs:316-320
    s = oracle.softmax([1.0, 2.0, 3.0])
    assert abs(s.sum() - 1) < 1e-5 and s[2] > s[1] > s[0]
    s = oracle.softmax([-np.inf] * 4)
    assert s[0] == 0.25 and abs(s.sum() - 1) < 1e-6
    s = oracle.softmax([np.inf, np.nan, 5.0, 10.0])
    assert np.all(np.isfinite(s)) and abs(s.sum() - 1) < 1e-5
    assert oracle.silu(0.0) == 0.0 and oracle.silu(2.0) > 0 and oracle.silu(-2.0) < 0
    assert oracle.silu(-50.0) == 0.0 and oracle.silu(-49.0) < 0
    g = oracle.swiglu([1.0, -1.0], [2.0, 3.0])
    assert 1.4 < g[0] < 1.5 and -1.0 < g[1] < -0.8
    for v in np.linspace(-40, 40, 81):
        assert abs(oracle.silu(float(v)) - v / (1 + math.exp(-v))) <= 1e-6 * max(1, abs(v))


def test_rope_table_matches_direct_formula(oracle):
    # crates/mivi-core/src/rope.rs:238-259
    hd, base, pos = 64, 10000.0, 5
    c, s = oracle.rope_table(hd, 16, base)
    q1, k1 = oracle.apply_rope_direct(np.ones(hd, np.float32), np.ones(hd, np.float32), hd, pos, base)
    q2 = oracle.rope_rotate(np.ones(hd, np.float32), 1, hd, c[pos], s[pos])
    assert np.all(np.abs(q1 - q2) < 1e-5) and np.all(np.abs(k1 - q2) < 1e-5)
    # closed form: angle pos * base^(-2i/hd), interleaved pairs (2i, 2i+1)
    i = np.arange(hd // 2)
    ang = pos * base ** (-2.0 * i / hd)
    assert np.allclose(c[pos], np.cos(ang), atol=2e-6) and np.allclose(s[pos], np.sin(ang), atol=2e-6)
    v = np.random.default_rng(3).standard_normal(hd).astype(np.float32)
    r = oracle.rope_rotate(v, 1, hd, c[pos], s[pos])
    want = np.empty(hd)
    want[0::2] = v[0::2] * np.cos(ang) - v[1::2] * np.sin(ang)
    want[1::2] = v[0::2] * np.sin(ang) + v[1::2] * np.cos(ang)
    assert np.allclose(r, want, atol=1e-5)


def test_rope_yarn_preserves_norm(oracle):
    # tests/long_context_retrieval.rs:45-91 (YaRN scale 16, base 1e6, 64K)
    hd = 64
    c, s = oracle.rope_table(hd, 65536, 1_000_000.0, scaling=2, scale=16.0)
    for pos in (0, 512, 4096, 8192, 16384, 32768, 65535):
        q = oracle.rope_rotate(np.ones(hd * 16, np.float32), 16, hd, c[pos], s[pos])
        assert np.all(np.isfinite(q))
        for h in range(16):
            assert abs(np.linalg.norm(q[h * hd:(h + 1) * hd].astype(np.float64)) - math.sqrt(hd)) < 1e-4


def test_yarn_ramp_limits(oracle):
    # rope.rs:71-105: high frequencies (wavelength < orig/beta_fast) keep the
    # base frequency, low ones (wavelength > orig/beta_slow) are divided by scale
    hd, base, scale = 64, 1_000_000.0, 8.0
    c0, s0 = oracle.rope_table(hd, 2, base)
    cy, sy = oracle.rope_table(hd, 2, base, scaling=2, scale=scale)
    inv0 = np.arctan2(s0[1], c0[1])
    invy = np.arctan2(sy[1], cy[1])
    wl = 2 * math.pi / inv0
    assert np.allclose(invy[wl < 4096 / 32], inv0[wl < 4096 / 32], rtol=1e-6)
    assert np.allclose(invy[wl > 4096], inv0[wl > 4096] / scale, rtol=1e-5)


def _yarn_ramp_violations(wl, ratio, scale, lo=4096 / 32, hi=4096 / 1):
    """Properties the YaRN ramp of rope.rs:71-105 fixes, checked on the
    per-frequency ratio r = inv_freq_yarn / inv_freq_base at wavelengths wl:
    r = 1 below orig/beta_fast, r = 1/scale above orig/beta_slow, and in
    between ramp = (1 - r) / (1 - 1/scale) is a straight line in the
    wavelength that meets 0 at the lower and 1 at the upper end. Returns the
    list of failed properties (empty when all hold)."""
    bad = []
    below, above = wl < lo, wl > hi
    inner = ~below & ~above
    if not np.allclose(ratio[below], 1.0, rtol=1e-6, atol=0):
        bad.append("below")
    if not np.allclose(ratio[above], 1.0 / scale, rtol=2e-5, atol=0):
        bad.append("above")
    ramp = (1.0 - ratio[inner]) / (1.0 - 1.0 / scale)
    if inner.sum() < 8:
        return bad + ["too few interior frequencies"]
    if np.any(ramp < -1e-4) or np.any(ramp > 1 + 1e-4):
        bad.append("ramp outside [0, 1]")
    # least-squares line through the interior points, in float64
    a, b = np.polyfit(wl[inner], ramp, 1)
    if np.max(np.abs(a * wl[inner] + b - ramp)) > 5e-4:
        bad.append("not linear in wavelength")
    if abs(a * lo + b) > 2e-3 or abs(a * hi + b - 1.0) > 2e-3:
        bad.append("does not meet the ends")
    return bad


@pytest.mark.parametrize("scale", [4352 / 4096, 32896 / 4096, 16.0])
def test_yarn_ramp_interior_linear_in_wavelength(oracle, scale):
    # rope.rs:71-105 with the model's parameters (model.rs:194-206: orig 4096,
    # beta_fast 32, beta_slow 1; scale = working ctx / 4096, configs 4 and 5).
    # head_dim 1024 gives 512 frequencies, about 130 of them inside the ramp
    # (wavelengths 128..4096). inv_freq is recovered from the pos-1 angles of
    # the table (angle = 1 * inv_freq, below pi).
    hd, base = 1024, 1_000_000.0
    c0, s0 = oracle.rope_table(hd, 2, base)
    cy, sy = oracle.rope_table(hd, 2, base, scaling=2, scale=scale)
    inv0 = np.arctan2(s0[1].astype(np.float64), c0[1].astype(np.float64))
    invy = np.arctan2(sy[1].astype(np.float64), cy[1].astype(np.float64))
    wl = 2 * math.pi / inv0
    assert _yarn_ramp_violations(wl, invy / inv0, scale) == []
    # the check tells plausible mistakes apart: a ramp in 1/wavelength (the
    # frequency-space form), a reversed ramp, swapped betas (a step at 4096)
    lo, hi = 128.0, 4096.0
    good = np.clip((wl - lo) / (hi - lo), 0, 1)
    mutants = {
        "ramp in 1/wavelength": np.clip((1 / wl - 1 / lo) / (1 / hi - 1 / lo), 0, 1),
        "reversed ramp": np.where((wl >= lo) & (wl <= hi), 1 - good, good),
        "swapped betas": (wl >= hi).astype(np.float64),
    }
    for name, ramp in mutants.items():
        ratio = (1 - ramp) + ramp / scale
        assert _yarn_ramp_violations(wl, ratio, scale), name
    # the model's head_dim (64): its 32 frequencies lie on the same curve
    c0, s0 = oracle.rope_table(64, 2, base)
    cy, sy = oracle.rope_table(64, 2, base, scaling=2, scale=scale)
    inv0_64 = np.arctan2(s0[1].astype(np.float64), c0[1].astype(np.float64))
    r64 = np.arctan2(sy[1].astype(np.float64), cy[1].astype(np.float64)) / inv0_64
    wl64 = 2 * math.pi / inv0_64
    curve = np.interp(wl64, wl, invy / inv0)
    inside = (wl64 > lo) & (wl64 < hi)
    assert inside.sum() == 9
    assert np.allclose(r64, curve, rtol=2e-4)


def test_model_yarn_decision(oracle):
    # model.rs:194-206: YaRN when the working context exceeds 4096, with
    # scale = working ctx / 4096 (configs 4 and 5 run it)
    from mivi_hip.synthmodel import build_hybrid
    img = build_hybrid(dim=256, hidden=512, n_layers=2, attn_layers=(1,), n_heads=4, n_kv=2, vocab=256,
                       ctx_len=65536, seed=3)
    for ctx, yarn in ((4096, 0), (4352, 1), (32896, 1)):
        m = oracle.Model(img, max_ctx=ctx)
        assert m.info.yarn == yarn
        assert m.info.yarn_scale == (np.float32(ctx) / np.float32(4096) if yarn else 1.0)


def test_argmax_first_strict_max(oracle):
    # sampler.rs:305-316
    assert oracle.argmax(np.array([1, 3, 3, 2], np.float32)) == 1
    assert oracle.argmax(np.array([-np.inf, -np.inf], np.float32)) == 0
    assert oracle.argmax(np.array([np.nan, 1.0, np.nan], np.float32)) == 1


def test_tiny_model_matches_reference_golden(oracle):
    # tests/oracle_comparison_test.rs:14-79 against tests/fixtures/oracle_output.json
    img = np.fromfile(os.path.join(GOLDEN, "tiny_model.gguf"), np.uint8)
    m = oracle.Model(img)
    assert (m.info.dim, m.info.n_layers, m.info.vocab_size) == (64, 2, 64)
    gold = json.load(open(os.path.join(GOLDEN, "oracle_output.json")))
    for tr in gold:
        logits = m.forward(tr["token"], tr["pos"])
        assert oracle.argmax(logits) == tr["top_token"]
        assert np.all(np.abs(logits[:8] - np.array(tr["logits_sample"])) < 0.05)


def test_tiny_fixture_is_reproducible():
    # the committed fixture equals what the restated generator produces
    import importlib.util
    spec = importlib.util.spec_from_file_location("mk", os.path.join(GOLDEN, "make_tiny_fixture.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    assert np.array_equal(mk.build(), np.fromfile(os.path.join(GOLDEN, "tiny_model.gguf"), np.uint8))


def _twopass_attention(q, K, V, scale):
    """Textbook two-pass softmax attention in float64 (reference_engine.py:146-166 form)."""
    s = (K.astype(np.float64) @ q.astype(np.float64)) * scale
    p = np.exp(s - s.max())
    p /= p.sum()
    return p @ V.astype(np.float64)


@pytest.mark.parametrize("seq", [1, 2, 37, 300])
def test_online_softmax_attention_matches_two_pass(oracle, seq):
    # The oracle's online-softmax GQA (transformer.rs:114-301) against the
    # textbook two-pass softmax in float64, for F32 and Q8_0 caches.
    nh, nkv, hd = 8, 2, 64
    rng = np.random.default_rng(seq)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    K = (rng.standard_normal((seq, nkv * hd)) * 2).astype(np.float32)
    V = rng.standard_normal((seq, nkv * hd)).astype(np.float32)
    out = oracle.attention(q, K, V, oracle.KV_F32, nh, nkv, hd, seq)
    for h in range(nh):
        kvh = h // (nh // nkv)
        ref = _twopass_attention(q[h * hd:(h + 1) * hd], K[:, kvh * hd:(kvh + 1) * hd], V[:, kvh * hd:(kvh + 1) * hd],
                                 1 / math.sqrt(hd))
        assert np.allclose(out[h * hd:(h + 1) * hd], ref, rtol=1e-5, atol=1e-5)
    # Q8_0 cache: the same two-pass form over the dequantized rows
    Kq = np.concatenate([oracle.quantize_q8_0_block(K.reshape(-1, 32)[i]) for i in range(seq * nkv * hd // 32)])
    Vq = np.concatenate([oracle.quantize_q8_0_block(V.reshape(-1, 32)[i]) for i in range(seq * nkv * hd // 32)])
    out = oracle.attention(q, Kq, Vq, oracle.KV_Q8_0, nh, nkv, hd, seq)
    Kd = oracle.dequantize_slice(8, Kq, seq * nkv * hd)[1].reshape(seq, -1)
    Vd = oracle.dequantize_slice(8, Vq, seq * nkv * hd)[1].reshape(seq, -1)
    for h in range(nh):
        kvh = h // (nh // nkv)
        ref = _twopass_attention(q[h * hd:(h + 1) * hd], Kd[:, kvh * hd:(kvh + 1) * hd],
                                 Vd[:, kvh * hd:(kvh + 1) * hd], 1 / math.sqrt(hd))
        assert np.allclose(out[h * hd:(h + 1) * hd], ref, rtol=1e-4, atol=1e-4)


def test_q8_kv_cache_sizes(oracle):
    # tests/quantized_kv_and_prefill.rs:4-39 arithmetic: 6 layers x 64K x 512
    row_q8 = (512 // 32) * 34
    assert 2 * 6 * 65536 * row_q8 == 427_819_008
    assert 2 * 6 * 65536 * 512 * 4 == 1_610_612_736


def test_serial_attention_is_the_parallel_result(oracle):
    # The reference loops over the query heads one after another
    # (transformer.rs:128); the oracle spreads long caches' heads over its
    # threads. Each head keeps its own running state in token order, so the
    # two schedules give the same bits (8 heads x 8200 tokens crosses the
    # oracle's threshold for the parallel form).
    nh, nkv, hd, seq = 8, 2, 64, 8200
    rng = np.random.default_rng(77)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    K = rng.standard_normal((seq, nkv * hd)).astype(np.float32)
    V = rng.standard_normal((seq, nkv * hd)).astype(np.float32)
    oracle.set_threads(4)
    par = oracle.attention(q, K, V, oracle.KV_F32, nh, nkv, hd, seq)
    oracle.set_serial_attention(True)
    try:
        ser = oracle.attention(q, K, V, oracle.KV_F32, nh, nkv, hd, seq)
    finally:
        oracle.set_serial_attention(False)
    assert np.array_equal(par.view(np.uint32), ser.view(np.uint32))
