"""The prefix cache's chunk hash and its host bookkeeping without a GPU.

compute_chunk_hash (crates/mivi-kv/src/prefix.rs:70-87) is 64-bit FNV-1a over
the tokens' little-endian bytes, chained through the previous hash xor a
domain separator. The FNV-1a restatement below follows the published
algorithm (offset basis 0xcbf29ce484222325, prime 0x100000001b3) and is
itself pinned by the published test vectors of FNV-1a 64.
"""
from __future__ import annotations

import numpy as np
import pytest

MASK = (1 << 64) - 1


@pytest.fixture(scope="module")
def mh():
    import mivi_hip  # host-side entry points only: no GPU call below
    return mivi_hip


def fnv1a64(data: bytes, h: int = 0xCBF29CE484222325) -> int:
    for b in data:
        h ^= b
        h = (h * 0x100000001B3) & MASK
    return h


def test_fnv1a_published_vectors():
    assert fnv1a64(b"") == 0xCBF29CE484222325
    assert fnv1a64(b"a") == 0xAF63DC4C8601EC8C
    assert fnv1a64(b"foobar") == 0x85944171F73967E8


def test_first_chunk_is_fnv1a_of_le_bytes(mh):
    rng = np.random.default_rng(0)
    for n in (0, 1, 64, 100):
        toks = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
        assert mh.chunk_hash(0, toks) == fnv1a64(toks.astype("<u4").tobytes())
    # "abcd" as one little-endian token
    assert mh.chunk_hash(0, [0x64636261]) == fnv1a64(b"abcd")


def test_chained_hash_determinism_and_chaining(mh):
    # prefix.rs:143-157
    a, b = np.full(64, 1, np.uint32), np.full(64, 2, np.uint32)
    h0 = mh.chunk_hash(0, a)
    assert h0 == mh.chunk_hash(0, a)
    h1 = mh.chunk_hash(h0, b)
    assert h1 != h0
    assert h1 != mh.chunk_hash(h0 ^ 1, b)
    # a chained chunk starts from prev ^ 0x9E3779B97F4A7C15 instead of the basis
    assert h1 == fnv1a64(b.astype("<u4").tobytes(), h0 ^ 0x9E3779B97F4A7C15)
    assert h1 != mh.chunk_hash(0, b)


def test_empty_cache_bookkeeping(mh):
    pc = mh.PrefixCache()
    assert len(pc) == 0 and pc.memory_usage_bytes() == 0
    assert pc.find_longest_prefix(np.arange(128, dtype=np.uint32)) == (0, 0)
    assert pc.find_longest_prefix(np.arange(10, dtype=np.uint32)) == (0, 0)
    assert pc.prune_to_bytes(0) == 0
    pc.clear()
    assert not pc.contains(123)
