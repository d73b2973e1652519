"""GPU parity of mivi_hip_sample and mivi_hip_sample_rows (Sampler::sample,
sampler.rs:91-135) against the CPU oracle's restatement on identical logits,
penalty windows and seeds. The rows entry point runs the split path (chunk
kernel + pick kernel over the chunks' top-k candidates) when top_k <= 128 and
the whole-row steps otherwise; the cases below reach both, and the fallback
from the split path when ties overflow a chunk's candidates.

Bars:
* the generator state equals the oracle's after every step (the draws are
  bit-exact);
* greedy path: the token and the penalised logits equal the oracle's bit for
  bit;
* sampling paths: the probabilities left in the logits equal the oracle's up
  to one common factor (the same exponentials, 1e-6; the normaliser within
  1e-3: the reference sums the exponentials sequentially in f32, whose
  rounding error over 65536 terms reaches ~1e-4, the device sums them in a
  tree), and the token equals the oracle's unless the draw falls within that
  rounding of a cumulative boundary, which is checked in float64 whenever the
  tokens differ (at most a quarter of the draws; the reference's own result
  there depends on its f32 summation order).
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MASK = (1 << 64) - 1
TOL = 2e-4  # cumulative-sum rounding budget (absolute, probabilities sum to 1)

CONFIGS = {
    "default": dict(),  # GenerationConfig::default (config.rs:176-194)
    "greedy_penalised": dict(temperature=0.0, presence_penalty=0.5, frequency_penalty=0.25),
    "categorical": dict(temperature=1.0, top_p=1.0, top_k=0, repetition_penalty=1.0),
    "nucleus_min_p": dict(temperature=0.8, top_p=0.95, top_k=0, min_p=0.05, presence_penalty=0.5,
                          frequency_penalty=0.3),
    "wide_top_k": dict(temperature=1.5, top_p=1.0, top_k=1000),
    "top_p_zero": dict(temperature=1.0, top_p=0.0, top_k=0),
    "min_p_top_k": dict(temperature=0.7, top_p=0.8, top_k=64, min_p=0.2, presence_penalty=0.3),
    "categorical_min_p": dict(temperature=0.9, top_p=1.0, top_k=0, min_p=0.1, presence_penalty=0.4,
                              frequency_penalty=0.2),
}


def draw(state: int):
    """sampler.rs:70-77: (next state, r)."""
    state ^= state >> 12
    state ^= (state << 25) & MASK
    state ^= state >> 27
    r = ((state * 0x2545F4914F6CDD1D) & MASK) >> 32
    return state, float(np.float32((r >> 8) / 16777216.0))


def near_boundary(tok, probs, r, top_p, tol=TOL):
    """Whether token tok's cumulative interval lies within tol of the draw, in
    the order the reference accumulates (index order; descending for top-p)."""
    TOL = tol
    p = probs.astype(np.float64)
    if top_p < 1.0:
        n = p.size
        cutoff = (1.0 - top_p) / (n - 1.0) if n > 1 else 0.0
        cand = np.nonzero((p >= cutoff) & (p > 0) & np.isfinite(p))[0]
        order = cand[np.lexsort((cand, -p[cand]))]
        cum = np.cumsum(p[order])
        m = int(np.searchsorted(cum, top_p - TOL)) + 1
        r = r * cum[min(m, cum.size) - 1]
    else:
        order = np.arange(p.size)
        cum = np.cumsum(p)
    k = int(np.nonzero(order == tok)[0][0])
    lo = cum[k - 1] if k else 0.0
    return lo - TOL <= r <= cum[k] + TOL


def device_sample(hip, torch, api, l_d, r_d, cfg_h, rng_d, tok_d):
    if api == "row":
        hip.sample(l_d, r_d, cfg_h, rng_d, tok_d)
    else:
        hip.sample_rows(l_d.view(1, -1), None if r_d is None else r_d.view(1, -1), cfg_h, rng_d, tok_d)


def run_pair(hip, oracle, torch, logits, recent, cfgkw, seed, steps, api="row"):
    """steps draws on the device and on the oracle with the same state."""
    cfg_h = hip.SamplerConfig.make(**cfgkw)
    cfg_o = oracle.sampler_config(**cfgkw)
    greedy = cfgkw.get("temperature", 0.2) <= 0.0
    top_p = cfgkw.get("top_p", 0.9)
    rng_o = oracle.Rng(seed)
    st = int(rng_o.state.value)
    rng_d = torch.tensor([st - (1 << 64) if st >= 1 << 63 else st], dtype=torch.int64, device="cuda")
    tok_d = torch.zeros(1, dtype=torch.int32, device="cuda")
    rec = list(recent)
    mismatches = 0
    for s in range(steps):
        l_d = torch.from_numpy(logits.copy()).cuda()
        r_d = torch.tensor(rec, dtype=torch.int32, device="cuda") if rec else None
        device_sample(hip, torch, api, l_d, r_d, cfg_h, rng_d, tok_d)
        torch.cuda.synchronize()
        state0 = int(rng_o.state.value)
        t_o, l_o = oracle.sample(logits, rec, cfg_o, rng_o)
        t_d = int(tok_d.item())
        assert (int(rng_d.item()) & MASK) == rng_o.state.value, (cfgkw, s)
        got = l_d.cpu().numpy()
        if greedy:
            assert t_d == t_o, (cfgkw, seed, s, t_d, t_o)
            assert np.array_equal(got, l_o)
        else:
            nz = l_o > 1e-30
            assert np.array_equal(got > 1e-30, nz)
            ratio = got[nz].astype(np.float64) / l_o[nz]
            assert abs(ratio.mean() - 1.0) < 1e-3 and np.ptp(ratio) < 2e-6 * max(1.0, ratio.mean())
            # the device's own rule: exact fixed-point sums over the
            # probabilities it returned, so without a nucleus (whose size is
            # a knife edge where tied probabilities sum to top_p exactly) the
            # draw lies in its token's interval of their float64 cumulative
            # sum to within 1e-6
            if top_p >= 1.0:
                assert near_boundary(t_d, got, draw(state0)[1], top_p, tol=1e-6), (cfgkw, s, t_d)
            if t_d != t_o:
                mismatches += 1
                r = draw(state0)[1]
                assert near_boundary(t_d, l_o, r, top_p) and near_boundary(t_o, l_o, r, top_p), (cfgkw, s, t_d, t_o)
        rec = (rec + [t_o])[-64:]  # RECENT_TOKENS_WINDOW (config.rs:11)
    # full-vocabulary categorical draws over 65536 tokens land within rounding
    # of a boundary most often (about one in seven here)
    assert mismatches <= steps // 4, (cfgkw, mismatches)


@pytest.mark.parametrize("api", ["row", "rows"])
@pytest.mark.parametrize("name", list(CONFIGS))
@pytest.mark.parametrize("n", [5, 1000, 65536])
def test_sample_matches_oracle(hip, oracle, torch_mod, name, n, api):
    rng = np.random.default_rng(n + len(name))
    logits = (rng.standard_normal(n) * 3).astype(np.float32)
    logits[rng.integers(0, n, max(1, n // 50))] = -np.inf
    recent = rng.integers(0, n, min(n, 40)).tolist()
    run_pair(hip, oracle, torch_mod, logits, recent, CONFIGS[name], 1234 + n, 64, api)


@pytest.mark.parametrize("name", ["default", "categorical", "min_p_top_k", "greedy_penalised"])
def test_rows_ragged_length(hip, oracle, torch_mod, name):
    # a row length that leaves the last chunk partial and needs 69 chunks
    n = 70001
    rng = np.random.default_rng(7 + len(name))
    logits = (rng.standard_normal(n) * 2).astype(np.float32)
    recent = rng.integers(0, n, 64).tolist()
    run_pair(hip, oracle, torch_mod, logits, recent, CONFIGS[name], 99, 24, "rows")


@pytest.mark.parametrize("api", ["row", "rows"])
@pytest.mark.parametrize("finite", [1, 3])
def test_categorical_masked_rows(hip, oracle, torch_mod, finite, api):
    # full-vocabulary categorical sampling over a ragged row with only a few
    # finite logits, in different chunks
    n = 70001
    logits = np.full(n, -np.inf, np.float32)
    logits[[3, 40000, 69999][:finite]] = [0.5, -1.0, 2.0][:finite]
    run_pair(hip, oracle, torch_mod, logits, [], CONFIGS["categorical"], 21 + finite, 16, api)


@pytest.mark.parametrize("api", ["row", "rows"])
def test_categorical_uniform_row(hip, oracle, torch_mod, api):
    """A row with no finite logit: the softmax's uniform branch (math.rs:43-48),
    1/n everywhere. The device takes the first index whose exact cumulative
    mass reaches r; the reference's float32 running sum (sampler.rs:137-148)
    drifts by up to ~5e-4 over 70001 equal terms, so its token can sit a few
    dozen indices away. Each is checked against its own rule."""
    torch = torch_mod
    n = 70001
    logits = np.full(n, -np.inf, np.float32)
    cfgkw = CONFIGS["categorical"]
    cfg_h = hip.SamplerConfig.make(**cfgkw)
    cfg_o = oracle.sampler_config(**cfgkw)
    rng_o = oracle.Rng(21)
    st = int(rng_o.state.value)
    rng_d = torch.tensor([st - (1 << 64) if st >= 1 << 63 else st], dtype=torch.int64, device="cuda")
    tok_d = torch.zeros(1, dtype=torch.int32, device="cuda")
    for s in range(16):
        l_d = torch.from_numpy(logits.copy()).cuda()
        device_sample(hip, torch, api, l_d, None, cfg_h, rng_d, tok_d)
        torch.cuda.synchronize()
        state0 = int(rng_o.state.value)
        t_o, l_o = oracle.sample(logits, [], cfg_o, rng_o)
        assert (int(rng_d.item()) & MASK) == rng_o.state.value
        got = l_d.cpu().numpy()
        assert np.all(got == np.float32(1.0 / n)) and np.all(l_o == np.float32(1.0 / n))
        r = draw(state0)[1]
        # device: exact masses, index floor-ish of r * n
        t_d = int(tok_d.item())
        assert near_boundary(t_d, l_o, r, 1.0), (s, t_d, r)
        # oracle: the float32 running sum
        cum32 = np.cumsum(l_o)
        lo = float(cum32[t_o - 1]) if t_o else 0.0
        assert lo - 1e-6 <= r <= float(cum32[t_o]) + 1e-6, (s, t_o, r)
        assert abs(t_d - t_o) <= 0.001 * n, (s, t_d, t_o)


@pytest.mark.parametrize("scale", [1.0, 0.3])
def test_rows_ties(hip, oracle, torch_mod, scale):
    # few distinct logits: at scale 1 about 70 ties per chunk at or above its
    # 40th value, handed on; at scale 0.3 about 500, more than a chunk may hand
    # on, and the row runs the whole-row steps
    n = 65536
    rng = np.random.default_rng(5)
    logits = np.floor(rng.standard_normal(n) * scale + 0.5).astype(np.float32)
    cfg = dict(temperature=1.0, top_p=0.9, top_k=40)
    run_pair(hip, oracle, torch_mod, logits, [], cfg, 17, 16, "rows")


@pytest.mark.parametrize("name", ["default", "categorical", "greedy_penalised", "min_p_top_k"])
def test_rows_batch_independent(hip, oracle, torch_mod, name):
    """Three rows at once, each with its own logits, window and state, against
    the oracle row by row."""
    torch = torch_mod
    n, rows, steps = 65536, 3, 12
    rng = np.random.default_rng(11 + len(name))
    logits = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
    recent = rng.integers(0, n, (rows, 40)).astype(np.int32)
    cfgkw = CONFIGS[name]
    cfg_h = hip.SamplerConfig.make(**cfgkw)
    cfg_o = oracle.sampler_config(**cfgkw)
    seeds = [5, 0, 1 << 63]
    rng_o = [oracle.Rng(s) for s in seeds]
    st = [int(r.state.value) for r in rng_o]
    rng_d = torch.tensor([s - (1 << 64) if s >= 1 << 63 else s for s in st], dtype=torch.int64, device="cuda")
    tok_d = torch.zeros(rows, dtype=torch.int32, device="cuda")
    greedy = cfgkw.get("temperature", 0.2) <= 0.0
    top_p = cfgkw.get("top_p", 0.9)
    mismatches = 0
    for s in range(steps):
        l_d = torch.from_numpy(logits.copy()).cuda()
        hip.sample_rows(l_d, torch.from_numpy(recent).cuda(), cfg_h, rng_d, tok_d)
        torch.cuda.synchronize()
        got_l = l_d.cpu().numpy()
        got_t = tok_d.cpu().numpy()
        got_s = rng_d.cpu().numpy()
        for b in range(rows):
            state0 = int(rng_o[b].state.value)
            t_o, l_o = oracle.sample(logits[b], recent[b].tolist(), cfg_o, rng_o[b])
            assert (int(got_s[b]) & MASK) == rng_o[b].state.value, (name, s, b)
            if greedy:
                assert int(got_t[b]) == t_o and np.array_equal(got_l[b], l_o), (name, s, b)
            else:
                nz = l_o > 1e-30
                assert np.array_equal(got_l[b] > 1e-30, nz)
                ratio = got_l[b][nz].astype(np.float64) / l_o[nz]
                assert abs(ratio.mean() - 1.0) < 1e-3 and np.ptp(ratio) < 2e-6 * max(1.0, ratio.mean())
                if top_p >= 1.0:
                    assert near_boundary(int(got_t[b]), got_l[b], draw(state0)[1], top_p, tol=1e-6), (name, s, b)
                if int(got_t[b]) != t_o:
                    mismatches += 1
                    r = draw(state0)[1]
                    assert near_boundary(int(got_t[b]), l_o, r, top_p) and near_boundary(t_o, l_o, r, top_p)
    assert mismatches <= rows * steps // 4, (name, mismatches)


def test_reference_cases_on_device(hip, oracle, torch_mod):
    torch = torch_mod
    # sampler.rs:340-350: zero temperature still applies penalties
    l = torch.tensor([5.0, 4.0], device="cuda")
    rng = torch.tensor([1], dtype=torch.int64, device="cuda")
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    hip.sample(l, torch.tensor([0], dtype=torch.int32, device="cuda"),
               hip.SamplerConfig.make(temperature=0.0, presence_penalty=2.0), rng, tok)
    assert int(tok.item()) == 1
    # sampler.rs:352-363: top-p reaches past the first 1024 tokens
    count = 2048
    p = (count - np.arange(count)).astype(np.float64)
    p /= p.sum()
    cfg = hip.SamplerConfig.make(temperature=1.0, top_p=0.9, top_k=0, repetition_penalty=1.0)
    rng = torch.tensor([1], dtype=torch.int64, device="cuda")
    seen = []
    for _ in range(256):
        l = torch.from_numpy(np.log(p).astype(np.float32)).cuda()
        hip.sample(l, None, cfg, rng, tok)
        seen.append(int(tok.item()))
    assert max(seen) >= 1024
    # an all -inf row: the softmax's uniform branch (math.rs:43-48), then top-p
    l = torch.full((8,), float("-inf"), device="cuda")
    hip.sample(l, None, hip.SamplerConfig.make(temperature=1.0, top_k=0), rng, tok)
    assert np.all(l.cpu().numpy() == np.float32(0.125))


def test_sample_rejects_null_arguments(hip, torch_mod):
    # validated on the host before any launch
    assert hip._lib.mivi_hip_sample(None, 4, None, 0, None, None, None, None) != 0
    assert hip.last_error().code == 101
    assert hip._lib.mivi_hip_sample_rows(None, 4, 1, 4, None, 0, 0, None, None, None, None, 0, None) != 0
    assert hip.last_error().code == 101
