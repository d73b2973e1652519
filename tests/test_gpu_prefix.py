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


@pytest.mark.parametrize("kv", ["F32", "F16", "Q8_0"])
def test_state_interval_export_import(hip, img, kv):
    """export_state_range / import_state_at (cache.rs:688-746, :827-914):
    an interval export equals the same rows of a whole export; a prompt
    rebuilt from three interval imports at unaligned offsets (partial 16-token
    groups in the Q8_0 layout) continues bit for bit like the original; an
    interval import leaves the other positions as they were."""
    kvp = getattr(hip.KvPrecision, kv)
    rng = np.random.default_rng(31)
    prompt = rng.integers(0, SMALL["vocab"], 151).astype(np.uint32)
    n = len(prompt) - 1
    m = model(hip, img, kvp)
    m.prefill(prompt[:-1], 0)
    k, v, conv = m.export_state(n)
    row, L = m.kv_row_bytes(), m.info.n_attn_layers

    def rows(a, s0, t):  # rows [s0, s0 + t) of every layer of a whole export of n tokens
        return np.concatenate([a[(l * n + s0) * row:(l * n + s0 + t) * row] for l in range(L)])

    for s0, t in ((0, 37), (37, 50), (87, 63), (5, 3), (16, 32)):
        ki, vi = m.export_state_range(s0, t)
        assert np.array_equal(ki, rows(k, s0, t)) and np.array_equal(vi, rows(v, s0, t)), (s0, t)
    want = m.forward(int(prompt[-1]), n)
    m2 = model(hip, img, kvp)
    for s0, t in ((87, 63), (0, 37), (37, 50)):
        m2.import_state_at(s0, t, rows(k, s0, t), rows(v, s0, t), conv if s0 == 0 else None)
    assert np.array_equal(m2.forward(int(prompt[-1]), n), want)
    # an interval import touches nothing outside it
    m3 = model(hip, img, kvp)
    other = rng.integers(0, SMALL["vocab"], 150).astype(np.uint32)
    m3.prefill(other, 0)
    k3, v3, c3 = m3.export_state(n)
    m3.import_state_at(37, 50, rows(k, 37, 50), rows(v, 37, 50))
    k4, v4, c4 = m3.export_state(n)
    for a, b, src in ((k3, k4, k), (v3, v4, v)):
        assert np.array_equal(rows(b, 0, 37), rows(a, 0, 37)) and np.array_equal(rows(b, 87, 63), rows(a, 87, 63))
        assert np.array_equal(rows(b, 37, 50), rows(src, 37, 50))
    assert np.array_equal(c3, c4)


def test_state_interval_errors(hip, img):
    m = hip.Model(img, max_ctx=256, kv_precision=hip.KvPrecision.Q8_0)
    row, L = m.kv_row_bytes(), m.info.n_attn_layers
    with pytest.raises(hip.ModelError) as e:  # KvError::ContextOverflow (cache.rs:692-697)
        m.export_state_range(200, 57)
    assert e.value.code == 115
    with pytest.raises(hip.ModelError) as e:  # KvError::DimMismatch (cache.rs:851-856)
        m.import_state_at(0, 10, np.zeros(L * 10 * row - 1, np.uint8), np.zeros(L * 10 * row - 1, np.uint8))
    assert e.value.code == 115
    with pytest.raises(hip.ModelError) as e:
        m.import_state_at(250, 10, np.zeros(L * 10 * row, np.uint8), np.zeros(L * 10 * row, np.uint8))
    assert e.value.code == 115


@pytest.mark.parametrize("kv", ["F16", "Q8_0"])
def test_full_snapshots_restore_bit_exact(hip, img, kv):
    """insert_chunk (prefix.rs:239-249): chained full snapshots (each holds
    the whole prefix, no parent link); the lookup of prefix.rs:672-722
    (two chunks plus extra tokens match 128, a different second chunk 64),
    and restoring the deeper one into a fresh model continues bit for bit."""
    kvp = getattr(hip.KvPrecision, kv)
    rng = np.random.default_rng(41)
    prompt = rng.integers(0, SMALL["vocab"], 2 * CS + 3).astype(np.uint32)
    ref = model(hip, img, kvp)
    ref.prefill(prompt[:-1], 0)
    want = ref.forward(int(prompt[-1]), len(prompt) - 1)
    pc = hip.PrefixCache()
    m = model(hip, img, kvp)
    m.prefill(prompt[:CS], 0)
    h0 = pc.insert_chunk(m, 0, prompt[:CS], 0, CS)
    m.prefill(prompt[CS:2 * CS], CS)
    h1 = pc.insert_chunk(m, h0, prompt[CS:2 * CS], 1, 2 * CS)
    assert len(pc) == 2 and h1 == hip.chunk_hash(h0, prompt[CS:2 * CS])
    assert pc.find_longest_prefix(prompt) == (2 * CS, h1)
    assert pc.find_longest_prefix(np.concatenate([prompt[:CS], np.full(CS, 500, np.uint32)])) == (CS, h0)
    # restoring copies the deepest node alone: it holds the whole prefix
    fresh = model(hip, img, kvp)
    matched, h = pc.restore_longest_prefix(fresh, prompt)
    assert (matched, h) == (2 * CS, h1)
    fresh.prefill(prompt[2 * CS:-1], 2 * CS)
    assert np.array_equal(fresh.forward(int(prompt[-1]), len(prompt) - 1), want)


def test_suffix_match(hip, img):
    """find_longest_suffix_match, the reference's tests prefix.rs:771-862 on
    device snapshots: a cached chunk found as the suffix of a later prompt
    (skip 64, its position), no match on different content, the right one of
    two chunks, and a chunk cached under a chained hash found by its
    standalone hash."""
    m = model(hip, img, hip.KvPrecision.F16)
    pc = hip.PrefixCache(max_chunks=5)
    chunk = np.arange(64, dtype=np.uint32)
    m.prefill(chunk, 0)
    h = pc.insert_chunk(m, 0, chunk, 0, 64)
    history = np.arange(100, 164, dtype=np.uint32)
    assert pc.find_longest_suffix_match(64, np.concatenate([history, chunk])) == (64, 64, h)
    assert pc.find_longest_suffix_match(64, np.concatenate([history, np.arange(200, 264, dtype=np.uint32)])) is None
    assert pc.find_longest_suffix_match(64, chunk) is None  # nothing past start_pos
    # chunk1 cached at position 128 under the chain (h, chunk1)
    chunk1 = np.arange(900, 964, dtype=np.uint32)  # the small model has 1024 tokens
    m.prefill(chunk1, 64)
    h1 = pc.insert_chunk(m, h, chunk1, 1, 128)
    assert h1 != hip.chunk_hash(0, chunk1)
    got = pc.find_longest_suffix_match(64, np.concatenate([np.arange(500, 564, dtype=np.uint32), chunk1]))
    assert got == (64, 128, h1)
    # suffix positions must be chunk-aligned: a 64-token suffix at absolute 70 is skipped
    assert pc.find_longest_suffix_match(6, np.concatenate([history, chunk1])) is None


def test_q8_group_snapshots_near_unaligned_max_ctx(hip, img):
    """A Q8_0 model whose max_ctx (1000) is not a multiple of the 16-token
    group: a full snapshot inside the last, partial group holds whole groups
    (every kv head's codes and scales of those tokens), and a snapshot at the
    last chunk boundary restores and continues bit for bit."""
    kvp = hip.KvPrecision.Q8_0
    rng = np.random.default_rng(59)
    prompt = rng.integers(0, SMALL["vocab"], 999).astype(np.uint32)

    def mk():
        m = hip.Model(img, max_ctx=1000, kv_precision=kvp)
        m.set_prefill_strategy(32)
        return m

    ref = mk()
    ref.prefill(prompt[:-1], 0)
    want = ref.forward(int(prompt[-1]), len(prompt) - 1)
    # snapshot bytes: 992 tokens = 62 whole groups, 996 tokens = 63
    m = mk()
    m.prefill(prompt[:996], 0)
    pa, pb = hip.PrefixCache(chunk_size=496), hip.PrefixCache(chunk_size=496)
    pa.insert_chunk(m, 0, prompt[:992], 0, 992)
    pb.insert_chunk(m, 0, prompt[:996], 0, 996)
    row = (SMALL["dim"] // SMALL["n_heads"] * SMALL["n_kv"]) // 32 * 34
    n_attn = len(SMALL["attn_layers"])
    assert pb.memory_usage_bytes() - pa.memory_usage_bytes() == 2 * n_attn * 16 * row + 4 * 4
    # two delta chunks of 496 tokens up to 992, restored into a fresh model
    pc = hip.PrefixCache(chunk_size=496)
    m = mk()
    m.prefill(prompt[:496], 0)
    h0 = pc.insert_delta_chunk(m, 0, prompt[:496], 0, 496)
    m.prefill(prompt[496:992], 496)
    pc.insert_delta_chunk(m, h0, prompt[496:992], 1, 992)
    fresh = mk()
    matched, _ = pc.restore_longest_prefix(fresh, prompt)
    assert matched == 992
    fresh.prefill(prompt[992:-1], 992)
    assert np.array_equal(fresh.forward(int(prompt[-1]), len(prompt) - 1), want)
