"""`Model`: the hybrid decode step resident on the GPU.

Mirrors crates/mivi-model/src/model.rs: `forward(token, pos)` returns the
logits (model.rs:488-491), `forward_step(..., compute_logits)` (model.rs:336),
`reset_context()` (model.rs:494-497), plus the batched greedy loop and the
state export/import used for state injection (cache.rs:682-914,
arena.rs:110-123).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import KvPrecision, ModelError, MiviModelInfo, _check, _lib


class Model:
    def __init__(self, gguf: np.ndarray | bytes, max_ctx: int = 0, kv_precision=KvPrecision.F32,
                 max_batch: int = 1):
        img = np.frombuffer(gguf, np.uint8) if isinstance(gguf, (bytes, bytearray)) else \
            np.ascontiguousarray(gguf, np.uint8)
        h = C.c_void_p()
        _check(_lib.mivi_hip_model_create(img.ctypes.data_as(C.c_void_p), img.nbytes, max_ctx,
                                          int(kv_precision), max_batch, C.byref(h)), ModelError)
        self._h = h
        self.info = MiviModelInfo()
        _lib.mivi_hip_model_info(self._h, C.byref(self.info))

    def close(self):
        if getattr(self, "_h", None):
            _lib.mivi_hip_model_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    @property
    def vocab_size(self) -> int:
        return self.info.vocab_size

    def reset_context(self):
        _check(_lib.mivi_hip_model_reset(self._h), ModelError)

    def forward_step(self, token: int, pos: int, compute_logits: bool = True, seq: int = 0):
        out = np.empty(self.info.vocab_size, np.float32) if compute_logits else None
        ptr = out.ctypes.data_as(C.c_void_p) if out is not None else None
        _check(_lib.mivi_hip_model_forward_step(self._h, seq, token, pos, 1 if compute_logits else 0, ptr),
               ModelError)
        return out

    def forward(self, token: int, pos: int, seq: int = 0) -> np.ndarray:
        return self.forward_step(token, pos, True, seq)

    def forward_batch(self, tokens, pos) -> np.ndarray:
        """Model::forward of sequences 0..batch-1 in one batched step (the
        batched decode's kernels). Returns [batch, vocab] logits."""
        t = np.ascontiguousarray(np.atleast_1d(tokens), np.uint32)
        p = np.ascontiguousarray(np.atleast_1d(pos), np.uint64)
        out = np.empty((t.size, self.info.vocab_size), np.float32)
        _check(_lib.mivi_hip_model_forward_batch(self._h, t.size, t.ctypes.data_as(C.c_void_p),
                                                 p.ctypes.data_as(C.c_void_p), out.ctypes.data_as(C.c_void_p)),
               ModelError)
        return out

    def prefill(self, tokens, pos0: int = 0, seq: int = 0):
        t = np.ascontiguousarray(tokens, np.uint32)
        _check(_lib.mivi_hip_model_prefill(self._h, seq, t.ctypes.data_as(C.c_void_p), t.size, pos0), ModelError)

    def set_prefill_strategy(self, tile_tokens: int = 0):
        """Model::set_prefill_strategy (model.rs:260-266): 0/1 = Token,
        t > 1 = Chunked { tile_tokens: t }."""
        _check(_lib.mivi_hip_model_set_prefill_tile(self._h, tile_tokens), ModelError)

    def generate_greedy(self, tokens, pos, n_steps: int) -> np.ndarray:
        """tokens/pos: one entry per sequence. Returns [n_steps, batch] argmax tokens."""
        t = np.ascontiguousarray(np.atleast_1d(tokens), np.uint32)
        p = np.ascontiguousarray(np.atleast_1d(pos), np.uint64)
        out = np.empty((n_steps, t.size), np.uint32)
        _check(_lib.mivi_hip_model_generate_greedy(self._h, t.size, t.ctypes.data_as(C.c_void_p),
                                                   p.ctypes.data_as(C.c_void_p), n_steps,
                                                   out.ctypes.data_as(C.c_void_p)), ModelError)
        return out

    def generate(self, tokens, pos, n_steps: int, cfg, seeds, eos_ids=()) -> np.ndarray:
        """The generation loop with Sampler::sample on the device (cfg: a
        SamplerConfig; seeds: one per sequence). Returns [n_steps, batch] tokens."""
        t = np.ascontiguousarray(np.atleast_1d(tokens), np.uint32)
        p = np.ascontiguousarray(np.atleast_1d(pos), np.uint64)
        sd = np.ascontiguousarray(np.atleast_1d(seeds), np.uint64)
        eo = np.ascontiguousarray(np.atleast_1d(np.asarray(eos_ids, np.uint32)), np.uint32)
        out = np.empty((n_steps, t.size), np.uint32)
        _check(_lib.mivi_hip_model_generate(self._h, t.size, t.ctypes.data_as(C.c_void_p),
                                            p.ctypes.data_as(C.c_void_p), n_steps, C.byref(cfg),
                                            sd.ctypes.data_as(C.c_void_p),
                                            eo.ctypes.data_as(C.c_void_p) if eo.size else None, eo.size,
                                            out.ctypes.data_as(C.c_void_p)), ModelError)
        return out

    def kv_row_bytes(self) -> int:
        kvd = self.info.kv_dim
        return {0: 4 * kvd, 2: 2 * kvd, 1: kvd // 32 * 34}[self.info.kv_precision]

    def conv_len(self) -> int:
        return self.info.n_layers * self.info.dim * max(1, self.info.ssm_conv_kernel)

    def export_state(self, tokens: int, seq: int = 0):
        n = self.info.n_attn_layers * tokens * self.kv_row_bytes()
        k = np.empty(n, np.uint8)
        v = np.empty(n, np.uint8)
        conv = np.empty(self.conv_len(), np.float32)
        _check(_lib.mivi_hip_model_export_state(self._h, seq, tokens, k.ctypes.data_as(C.c_void_p),
                                                v.ctypes.data_as(C.c_void_p), n, conv.ctypes.data_as(C.c_void_p),
                                                conv.size), ModelError)
        return k, v, conv

    def import_state(self, tokens: int, k: np.ndarray, v: np.ndarray, conv: np.ndarray, seq: int = 0):
        k = np.ascontiguousarray(k, np.uint8)
        v = np.ascontiguousarray(v, np.uint8)
        conv = np.ascontiguousarray(conv, np.float32)
        _check(_lib.mivi_hip_model_import_state(self._h, seq, tokens, k.ctypes.data_as(C.c_void_p),
                                                v.ctypes.data_as(C.c_void_p), min(k.nbytes, v.nbytes),
                                                conv.ctypes.data_as(C.c_void_p), conv.size), ModelError)


    def export_state_range(self, start: int, tokens: int, seq: int = 0, conv: bool = False):
        """KvCache::export_state_range (cache.rs:688-746): K and V rows of
        positions [start, start + tokens) of every attention layer (and the
        ShortConv state when conv). Returns (k, v) or (k, v, conv)."""
        n = self.info.n_attn_layers * tokens * self.kv_row_bytes()
        k = np.empty(n, np.uint8)
        v = np.empty(n, np.uint8)
        cs = np.empty(self.conv_len(), np.float32) if conv else None
        _check(_lib.mivi_hip_model_export_state_range(self._h, seq, start, tokens, k.ctypes.data_as(C.c_void_p),
                                                      v.ctypes.data_as(C.c_void_p), n,
                                                      cs.ctypes.data_as(C.c_void_p) if conv else None,
                                                      cs.size if conv else 0), ModelError)
        return (k, v, cs) if conv else (k, v)

    def import_state_at(self, start: int, tokens: int, k: np.ndarray, v: np.ndarray, conv=None, seq: int = 0):
        """KvCache::import_state_at (cache.rs:827-914): rows of an interval
        export into positions [start, start + tokens); the ShortConv state too
        when conv is given."""
        k = np.ascontiguousarray(k, np.uint8)
        v = np.ascontiguousarray(v, np.uint8)
        cs = None if conv is None else np.ascontiguousarray(conv, np.float32)
        _check(_lib.mivi_hip_model_import_state_at(self._h, seq, start, tokens, k.ctypes.data_as(C.c_void_p),
                                                   v.ctypes.data_as(C.c_void_p), min(k.nbytes, v.nbytes),
                                                   None if cs is None else cs.ctypes.data_as(C.c_void_p),
                                                   0 if cs is None else cs.size), ModelError)


def chunk_hash(prev_hash: int, tokens) -> int:
    """compute_chunk_hash (prefix.rs:70-87)."""
    t = np.ascontiguousarray(tokens, np.uint32)
    return int(_lib.mivi_hip_prefix_chunk_hash(C.c_uint64(prev_hash), t.ctypes.data_as(C.c_void_p), t.size))


class PrefixCache:
    """PrefixCache (crates/mivi-kv/src/prefix.rs) with device-resident
    snapshots: chunks of a model sequence's KV intervals and ShortConv states,
    restored device to device."""

    def __init__(self, max_chunks: int = 0, chunk_size: int = 0, max_memory_bytes: int = 0):
        h = C.c_void_p()
        _check(_lib.mivi_hip_prefix_cache_create(max_chunks, chunk_size, max_memory_bytes, C.byref(h)), ModelError)
        self._h = h
        self.chunk_size = chunk_size or 64

    def close(self):
        if getattr(self, "_h", None):
            _lib.mivi_hip_prefix_cache_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __len__(self) -> int:
        return int(_lib.mivi_hip_prefix_cache_len(self._h))

    def memory_usage_bytes(self) -> int:
        return int(_lib.mivi_hip_prefix_cache_memory_bytes(self._h))

    def prune_to_bytes(self, target: int) -> int:
        return int(_lib.mivi_hip_prefix_cache_prune(self._h, target))

    def clear(self):
        _lib.mivi_hip_prefix_cache_clear(self._h)

    def contains(self, hash_: int) -> bool:
        return bool(_lib.mivi_hip_prefix_cache_contains(self._h, C.c_uint64(hash_)))

    def insert_delta_chunk(self, model: "Model", prev_hash: int, tokens, chunk_index: int, pos: int,
                           seq: int = 0) -> int:
        """insert_delta_chunk (prefix.rs:251-303) from sequence seq of model,
        which has processed exactly pos tokens."""
        t = np.ascontiguousarray(tokens, np.uint32)
        h = C.c_uint64()
        _check(_lib.mivi_hip_prefix_cache_insert_delta(self._h, model._h, seq, pos, C.c_uint64(prev_hash),
                                                       t.ctypes.data_as(C.c_void_p), t.size, chunk_index,
                                                       C.byref(h)), ModelError)
        return int(h.value)

    def insert_chunk(self, model: "Model", prev_hash: int, tokens, chunk_index: int, pos: int, seq: int = 0) -> int:
        """insert_chunk (prefix.rs:239-249): a full snapshot of positions
        [0, pos) of sequence seq of model and its ShortConv state."""
        t = np.ascontiguousarray(tokens, np.uint32)
        h = C.c_uint64()
        _check(_lib.mivi_hip_prefix_cache_insert(self._h, model._h, seq, pos, C.c_uint64(prev_hash),
                                                 t.ctypes.data_as(C.c_void_p), t.size, chunk_index, C.byref(h)),
               ModelError)
        return int(h.value)

    def find_longest_suffix_match(self, start_pos: int, tokens):
        """find_longest_suffix_match (prefix.rs:453-517): (suffix_len,
        match_pos, hash) of the matched chunk, or None."""
        t = np.ascontiguousarray(tokens, np.uint32)
        n, p, h = C.c_size_t(), C.c_size_t(), C.c_uint64()
        _check(_lib.mivi_hip_prefix_cache_find_suffix(self._h, start_pos, t.ctypes.data_as(C.c_void_p), t.size,
                                                      C.byref(n), C.byref(p), C.byref(h)), ModelError)
        return (int(n.value), int(p.value), int(h.value)) if n.value else None

    def find_longest_prefix(self, tokens):
        """(matched tokens, hash) of the deepest cached chunk, (0, 0) if none."""
        t = np.ascontiguousarray(tokens, np.uint32)
        n, h = C.c_size_t(), C.c_uint64()
        _check(_lib.mivi_hip_prefix_cache_find(self._h, t.ctypes.data_as(C.c_void_p), t.size, C.byref(n),
                                               C.byref(h)), ModelError)
        return int(n.value), int(h.value)

    def restore_longest_prefix(self, model: "Model", tokens, seq: int = 0):
        """restore_longest_prefix (prefix.rs:305-358) into sequence seq of
        model: (matched tokens, hash)."""
        t = np.ascontiguousarray(tokens, np.uint32)
        n, h = C.c_size_t(), C.c_uint64()
        _check(_lib.mivi_hip_prefix_cache_restore(self._h, model._h, seq, t.ctypes.data_as(C.c_void_p), t.size,
                                                  C.byref(n), C.byref(h)), ModelError)
        return int(n.value), int(h.value)
