"""GPU tests of the device-resident prefix cache (PrefixCache,
crates/mivi-kv/src/prefix.rs).

* Restoring a cached chunk chain and continuing gives the same logits, bit
  for bit, and the same greedy tokens as prefilling the whole prompt (the
  snapshots are exact copies of the model's caches and ShortConv state).
* The bookkeeping follows the reference's tests: a delta chunk needs its
  ancestor (prefix.rs:135-139), lookups stop at the first missing chunk
  (:160-211), eviction takes the least recently used of the deepest chunks
  (:214-257), and branches share their root under a byte budget (:42-81).
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SMALL = dict(dim=256, hidden=768, n_layers=6, attn_layers=(1, 4), n_heads=4, n_kv=2, vocab=1024)
CS = 64


@pytest.fixture(scope="module")
def img():
    from mivi_hip.synthmodel import build_hybrid
    return build_hybrid(**SMALL, ctx_len=4096, seed=7)


def model(hip, img, kvp):
    m = hip.Model(img, max_ctx=1024, kv_precision=kvp)
    m.set_prefill_strategy(32)
    return m


def prefill_chunks(m, pc, tokens, n_chunks, seq=0):
    """Prefill chunk by chunk, inserting each as a delta chunk."""
    prev = 0
    hashes = []
    for i in range(n_chunks):
        m.prefill(tokens[i * CS:(i + 1) * CS], i * CS, seq)
        prev = pc.insert_delta_chunk(m, prev, tokens[i * CS:(i + 1) * CS], i, (i + 1) * CS, seq)
        hashes.append(prev)
    return hashes


@pytest.mark.parametrize("kv", ["F16", "Q8_0"])
def test_restore_continues_bit_exact(hip, img, kv):
    kvp = getattr(hip.KvPrecision, kv)
    rng = np.random.default_rng(3)
    prompt = rng.integers(0, SMALL["vocab"], 3 * CS + 20).astype(np.uint32)
    # reference: the whole prompt prefilled, then greedy steps
    ref = model(hip, img, kvp)
    ref.prefill(prompt[:-1], 0)
    want_logits = ref.forward(int(prompt[-1]), len(prompt) - 1)
    ref.reset_context()
    ref.prefill(prompt[:-1], 0)
    want = ref.generate_greedy([int(prompt[-1])], [len(prompt) - 1], 12)
    # chunks cached, then restored into a fresh model
    pc = hip.PrefixCache()
    m = model(hip, img, kvp)
    hashes = prefill_chunks(m, pc, prompt, 3)
    assert len(pc) == 3 and all(pc.contains(h) for h in hashes)
    m2 = model(hip, img, kvp)
    matched, h = pc.restore_longest_prefix(m2, prompt)
    assert (matched, h) == (3 * CS, hashes[-1])
    m2.prefill(prompt[matched:-1], matched)
    got_logits = m2.forward(int(prompt[-1]), len(prompt) - 1)
    assert np.array_equal(got_logits, want_logits)
    m2.reset_context()
    matched, _ = pc.restore_longest_prefix(m2, prompt)
    m2.prefill(prompt[matched:-1], matched)
    got = m2.generate_greedy([int(prompt[-1])], [len(prompt) - 1], 12)
    assert np.array_equal(got, want)


def test_delta_rejects_missing_ancestor(hip, img):
    # prefix.rs:135-139
    m = model(hip, img, hip.KvPrecision.F16)
    pc = hip.PrefixCache()
    m.prefill(np.ones(2 * CS, np.uint32), 0)
    with pytest.raises(hip.ModelError):
        pc.insert_delta_chunk(m, 123, np.ones(CS, np.uint32), 1, 2 * CS)
    assert len(pc) == 0
    # the state must sit exactly at the chunk's end (DimMismatch otherwise)
    with pytest.raises(hip.ModelError):
        pc.insert_delta_chunk(m, 0, np.ones(CS, np.uint32), 0, 2 * CS)
    assert hip.last_error().code == 115
    assert len(pc) == 0


def test_lookup_stops_at_first_missing_chunk(hip, img):
    # prefix.rs:160-211
    m = model(hip, img, hip.KvPrecision.F16)
    pc = hip.PrefixCache()
    toks = np.arange(2 * CS, dtype=np.uint32)
    h0, h1 = prefill_chunks(m, pc, toks, 2)
    assert len(pc) == 2
    assert pc.find_longest_prefix(toks) == (2 * CS, h1)
    other = np.concatenate([toks[:CS], np.full(CS, 7, np.uint32)])
    assert pc.find_longest_prefix(other) == (CS, h0)
    assert pc.find_longest_prefix(toks[:CS - 1]) == (0, 0)
    assert pc.find_longest_prefix(np.full(2 * CS, 9, np.uint32)) == (0, 0)


def test_eviction_takes_oldest_of_deepest(hip, img):
    # prefix.rs:214-230: three root chunks, room for two: the oldest goes
    m = model(hip, img, hip.KvPrecision.F16)
    pc = hip.PrefixCache(max_chunks=2)
    hs = []
    for v in (1, 2, 3):
        m.reset_context()
        hs += prefill_chunks(m, pc, np.full(CS, v, np.uint32), 1)
    assert len(pc) == 2 and not pc.contains(hs[0]) and pc.contains(hs[1]) and pc.contains(hs[2])
    # prefix.rs:233-257: a chain of three, room for two: the new leaf goes and
    # the root chain stays reusable
    pc2 = hip.PrefixCache(max_chunks=2)
    m.reset_context()
    toks = np.arange(3 * CS, dtype=np.uint32)
    h0, h1, h2 = prefill_chunks(m, pc2, toks, 3)
    assert len(pc2) == 2 and not pc2.contains(h2)
    prompt = np.concatenate([toks[:2 * CS], [999, 1000, 1001]]).astype(np.uint32)
    assert pc2.find_longest_prefix(prompt) == (2 * CS, h1)


def test_branches_share_root_under_byte_budget(hip, img):
    # prefix.rs:42-81: root [1]*64 with children [2]*64 and [3]*64; pruning
    # to two nodes' bytes drops the older child; the other branch restores
    kvp = hip.KvPrecision.F16
    m = model(hip, img, kvp)
    pc = hip.PrefixCache(max_chunks=10)
    ones, twos, threes = (np.full(CS, v, np.uint32) for v in (1, 2, 3))
    m.prefill(ones, 0)
    root = pc.insert_delta_chunk(m, 0, ones, 0, CS)
    m.prefill(twos, CS)
    first = pc.insert_delta_chunk(m, root, twos, 1, 2 * CS)
    m.reset_context()
    assert pc.restore_longest_prefix(m, ones) == (CS, root)
    m.prefill(threes, CS)
    second = pc.insert_delta_chunk(m, root, threes, 1, 2 * CS)
    assert len(pc) == 3
    budget = pc.memory_usage_bytes() // 3 * 2
    assert pc.prune_to_bytes(budget) == 1
    assert pc.memory_usage_bytes() <= budget
    assert not pc.contains(first) and pc.contains(root) and pc.contains(second)
    prompt = np.concatenate([ones, threes, [5]]).astype(np.uint32)
    ref = model(hip, img, kvp)
    ref.prefill(prompt[:-1], 0)
    want = ref.forward(int(prompt[-1]), 2 * CS)
    m2 = model(hip, img, kvp)
    assert pc.restore_longest_prefix(m2, prompt) == (2 * CS, second)
    assert np.array_equal(m2.forward(int(prompt[-1]), 2 * CS), want)
    pc.clear()
    assert len(pc) == 0 and pc.memory_usage_bytes() == 0
