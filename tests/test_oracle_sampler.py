"""Pins the CPU oracle's restatement of crates/mivi-model/src/sampler.rs.

The reference's own tests (sampler.rs:322-404) restated, plus closed forms:
xorshift64* computed by hand, categorical frequencies against the softmax
probabilities, and the support of top-k / top-p sampling.
"""
from __future__ import annotations

import numpy as np
import pytest

MASK = (1 << 64) - 1


def xorshift_ref(state: int, n: int):
    """sampler.rs:70-77 by hand: xorshift64* then (r >> 8) / 2^24."""
    out = []
    for _ in range(n):
        state ^= state >> 12
        state ^= (state << 25) & MASK
        state ^= state >> 27
        r = ((state * 0x2545F4914F6CDD1D) & MASK) >> 32
        out.append(np.float32((r >> 8) / 16777216.0))
    return out


def test_random_f32_matches_xorshift64_star(oracle):
    for seed in (1, 12345, 0xDEADBEEF, 0x853C49E6748FEA9B):
        rng = oracle.Rng(seed)
        got = [np.float32(rng.random_f32()) for _ in range(64)]
        assert got == xorshift_ref(seed, 64)
        assert all(0.0 <= g < 1.0 for g in got)


def test_zero_seed_not_absorbing(oracle):
    # sampler.rs:326-332 (seed 0 -> FALLBACK_RNG_SEED)
    rng = oracle.Rng(0)
    r1, r2 = rng.random_f32(), rng.random_f32()
    assert r1 != 0.0 and r1 != r2
    assert [r1, r2] == xorshift_ref(0x853C49E6748FEA9B, 2)


def test_deterministic_seed(oracle):
    # sampler.rs:391-403
    a, b = oracle.Rng(12345), oracle.Rng(12345)
    assert a.random_f32() == b.random_f32()
    assert a.random_f32() == b.random_f32()


def test_argmax(oracle):
    # sampler.rs:334-338
    assert oracle.argmax([1.0, 5.0, 3.0, 2.0]) == 1


def test_zero_temperature_still_applies_penalties(oracle):
    # sampler.rs:340-350 (other fields at GenerationConfig::default, config.rs:176-194)
    cfg = oracle.sampler_config(temperature=0.0, presence_penalty=2.0)
    tok, _ = oracle.sample([5.0, 4.0], [0], cfg, oracle.Rng(1))
    assert tok == 1


def test_penalties_repetition_presence_frequency(oracle):
    # sampler.rs:378-389
    out = oracle.apply_penalties([5.0, 5.0, 5.0, 5.0], [0, 1, 1, 1], 1.0, 1.0, 0.5)
    assert abs(out[0] - 3.5) < 1e-5 and abs(out[1] - 2.5) < 1e-5
    assert out[2] == 5.0 and out[3] == 5.0
    # the multiplicative branch: positive logits divided, the others multiplied
    out = oracle.apply_penalties([2.0, -2.0, 3.0], [0, 1, 7], 2.0, 0.0, 0.0)
    assert list(out) == [1.0, -4.0, 3.0]


def test_min_p(oracle):
    # sampler.rs:365-376
    out = oracle.apply_min_p([10.0, 8.0, 5.0, 1.0], 0.1)
    assert out[0] == 10.0 and out[1] == 8.0
    assert out[2] == -np.inf and out[3] == -np.inf


def test_top_k_keeps_ties_at_the_cutoff(oracle):
    out = oracle.apply_top_k([1.0, 4.0, 3.0, 4.0, 2.0], 2)
    assert list(out) == [-np.inf, 4.0, -np.inf, 4.0, -np.inf]
    out = oracle.apply_top_k([1.0, 4.0, 3.0, 4.0, 2.0], 3)
    assert list(out) == [-np.inf, 4.0, 3.0, 4.0, -np.inf]


def test_top_p_reaches_past_the_first_1024_tokens(oracle):
    # sampler.rs:352-363: a flat-ish distribution over 2048 tokens; logits
    # ln(p) give back p through the softmax (no penalties, temperature 1)
    count = 2048
    p = (count - np.arange(count)).astype(np.float64)
    p /= p.sum()
    cfg = oracle.sampler_config(temperature=1.0, top_p=0.9, top_k=0, repetition_penalty=1.0)
    rng = oracle.Rng(1)
    assert any(oracle.sample(np.log(p), [], cfg, rng)[0] >= 1024 for _ in range(256))


def test_categorical_frequencies_follow_the_softmax(oracle):
    logits = np.array([0.0, 1.0, 2.0, -1.0, 0.5], np.float32)
    p = np.exp(logits - logits.max())
    p /= p.sum()
    cfg = oracle.sampler_config(temperature=1.0, top_p=1.0, top_k=0, repetition_penalty=1.0)
    rng = oracle.Rng(7)
    n = 20000
    counts = np.bincount([oracle.sample(logits, [], cfg, rng)[0] for _ in range(n)], minlength=5)
    # 5 standard deviations of the binomial count
    assert np.all(np.abs(counts - n * p) <= 5 * np.sqrt(n * p * (1 - p)) + 1)


def test_top_k_and_top_p_support(oracle):
    rng_np = np.random.default_rng(3)
    logits = rng_np.standard_normal(500).astype(np.float32) * 3
    order = np.argsort(-logits, kind="stable")
    cfg = oracle.sampler_config(temperature=1.0, top_p=1.0, top_k=5, repetition_penalty=1.0)
    rng = oracle.Rng(11)
    picks = {oracle.sample(logits, [], cfg, rng)[0] for _ in range(400)}
    assert picks <= set(order[:5].tolist()) and len(picks) > 1
    # top-p: the smallest descending prefix reaching 0.5 of the mass
    p = np.exp(logits.astype(np.float64) - logits.max())
    p /= p.sum()
    m = int(np.searchsorted(np.cumsum(p[order]), 0.5) + 1)
    cfg = oracle.sampler_config(temperature=1.0, top_p=0.5, top_k=0, repetition_penalty=1.0)
    picks = {oracle.sample(logits, [], cfg, rng)[0] for _ in range(400)}
    assert picks <= set(order[:m + 1].tolist())


def test_softmax_special_cases(oracle):
    # math.rs:200-224
    x = oracle.softmax([1.0, 2.0, 3.0])
    assert abs(x.sum() - 1.0) < 1e-5 and x[2] > x[1] > x[0]
    x = oracle.softmax([-np.inf] * 4)
    assert x[0] == 0.25
    x = oracle.softmax([np.inf, np.nan, 5.0, 10.0])
    assert np.all(np.isfinite(x)) and abs(x.sum() - 1.0) < 1e-5
