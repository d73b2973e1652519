"""Python host binding of libmivi_hip.so (MI355X / gfx950).

Mirrors the reference's Rust surface so that callers and tests read like the
reference's own: `quantized_matvec`, `quantized_matmul_rows`,
`dequantize_slice`, `try_matvec_*` (crates/mivi-quant/src/lib.rs:35-251,
q4_k_m.rs:217, q6_k.rs:202, q8_0.rs:127, f16.rs:42-97) raise `QuantError`
where the reference returns `Err(QuantError::...)`; `Model` mirrors
crates/mivi-model/src/model.rs (`forward`, `forward_step`, `reset_context`).

Tensors are torch CUDA (HIP) tensors; torch only provides device memory and
streams. Every computation runs in the HIP kernels of libmivi_hip.so; the
module raises at import time if the library is missing, so nothing can fall
back to a CPU path.
"""
from __future__ import annotations

import ctypes as C
import enum
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmivi_hip.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"{LIB_PATH} is missing: build it with `python mivi-v4_amd/build.py` "
        "(or __graft_entry__.build()) before importing mivi_hip")


class GgmlType(enum.IntEnum):
    """crates/mivi-quant/src/types.rs:22-52 (the ids this library runs)."""
    F32 = 0
    F16 = 1
    Q8_0 = 8
    Q4_K = 12
    Q6_K = 14
    BF16 = 30

    def block_size(self) -> int:
        return {0: 1, 1: 1, 30: 1, 8: 32, 12: 256, 14: 256}[int(self)]

    def type_size(self) -> int:
        return {0: 4, 1: 2, 30: 2, 8: 34, 12: 144, 14: 210}[int(self)]


class KvPrecision(enum.IntEnum):
    """crates/mivi-kv/src/cache.rs:5-15 plus the half-precision layout."""
    F32 = 0
    Q8_0 = 1
    F16 = 2


class MiviError(C.Structure):
    _fields_ = [
        ("code", C.c_int32), ("type_id", C.c_uint32), ("expected", C.c_size_t), ("actual", C.c_size_t),
        ("dim", C.c_size_t), ("block_size", C.c_size_t), ("message", C.c_char * 256),
    ]


class QuantError(Exception):
    """crates/mivi-quant/src/types.rs:5-15; `kind` is the variant name."""
    KINDS = {1: "UnsupportedType", 2: "BufferTooSmall", 3: "DimensionMisaligned", 4: "ArithmeticOverflow"}

    def __init__(self, err: MiviError):
        self.code = err.code
        self.kind = self.KINDS.get(err.code, "Other")
        self.type_id = err.type_id
        self.expected = err.expected
        self.actual = err.actual
        self.dim = err.dim
        self.block_size = err.block_size
        super().__init__(err.message.decode(errors="replace"))


class ModelError(Exception):
    """crates/mivi-model/src/model.rs:25-49."""

    def __init__(self, err: MiviError):
        self.code = err.code
        super().__init__(err.message.decode(errors="replace"))


class MiviModelInfo(C.Structure):
    _fields_ = [(n, C.c_size_t) for n in (
        "dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "head_dim", "kv_dim", "vocab_size",
        "max_seq_len", "ssm_conv_kernel", "n_attn_layers", "max_batch")] + [
        ("rope_base", C.c_float), ("rms_norm_eps", C.c_float), ("kv_precision", C.c_int32),
        ("yarn", C.c_int32), ("yarn_scale", C.c_float), ("weight_bytes", C.c_size_t),
        ("kv_bytes", C.c_size_t)]


class SamplerConfig(C.Structure):
    """GenerationConfig's sampling fields (config.rs:163-194, defaults there)."""
    _fields_ = [(n, C.c_float) for n in ("temperature", "top_p", "min_p", "repetition_penalty",
                                         "presence_penalty", "frequency_penalty")] + [("top_k", C.c_uint32)]

    @classmethod
    def make(cls, temperature=0.2, top_p=0.9, top_k=40, min_p=0.0, repetition_penalty=1.05,
             presence_penalty=0.0, frequency_penalty=0.0):
        return cls(temperature, top_p, min_p, repetition_penalty, presence_penalty, frequency_penalty, top_k)


_lib = C.CDLL(LIB_PATH)
_P, _S, _I = C.c_void_p, C.c_size_t, C.c_int32
_sig = {
    "mivi_hip_last_error": ([C.POINTER(MiviError)], _I),
    "mivi_hip_version": ([], C.c_char_p),
    "mivi_hip_quantized_matvec": ([_P, _S, _I, _P, _S, _P, _S, _S, _S, _P], _I),
    "mivi_hip_try_matvec_q4_k_m": ([_P, _S, _P, _S, _P, _S, _S, _S, _P], _I),
    "mivi_hip_try_matvec_q6_k": ([_P, _S, _P, _S, _P, _S, _S, _S, _P], _I),
    "mivi_hip_try_matvec_q8_0": ([_P, _S, _P, _S, _P, _S, _S, _S, _P], _I),
    "mivi_hip_try_matvec_f16": ([_P, _S, _P, _S, _P, _S, _S, _S, _P], _I),
    "mivi_hip_try_matvec_bf16": ([_P, _S, _P, _S, _P, _S, _S, _S, _P], _I),
    "mivi_hip_quantized_matmul_rows": ([_P, _S, _I, _P, _S, _P, _S, _S, _S, _S, _P], _I),
    "mivi_hip_pack_weights": ([_I, _P, _S, _P, _S, _S, _S, _P], _I),
    "mivi_hip_quantized_matvec_packed": ([_P, _S, _I, _P, _S, _P, _S, _S, _S, _P], _I),
    "mivi_hip_quantized_matmul_rows_packed": ([_P, _S, _I, _P, _S, _P, _S, _S, _S, _S, _P], _I),
    "mivi_hip_gemm_packed_size": ([_I, _S, _S], _S),
    "mivi_hip_pack_weights_gemm": ([_I, _P, _S, _P, _S, _S, _S, _P], _I),
    "mivi_hip_quantized_matmul_rows_gemm_packed": ([_P, _S, _I, _P, _S, _P, _S, _P, _S, _S, _S, _S, _P], _I),
    "mivi_hip_dequantize_slice": ([_I, _P, _S, _P, _S, _P], _I),
    "mivi_hip_quantize_q8_0": ([_P, _S, _P, _S, _S, _P], _I),
    "mivi_hip_dot_q8_0_f32": ([_P, _S, _P, _S, _P, _S, _S, _P], _I),
    "mivi_hip_model_create": ([_P, _S, _S, _I, _S, C.POINTER(_P)], _I),
    "mivi_hip_model_destroy": ([_P], None),
    "mivi_hip_model_info": ([_P, C.POINTER(MiviModelInfo)], _I),
    "mivi_hip_model_reset": ([_P], _I),
    "mivi_hip_model_forward_step": ([_P, _S, C.c_uint32, _S, _I, _P], _I),
    "mivi_hip_model_forward": ([_P, _S, C.c_uint32, _S, _P], _I),
    "mivi_hip_model_forward_batch": ([_P, _S, _P, _P, _P], _I),
    "mivi_hip_model_generate_greedy": ([_P, _S, _P, _P, _S, _P], _I),
    "mivi_hip_model_prefill": ([_P, _S, _P, _S, _S], _I),
    "mivi_hip_model_set_prefill_tile": ([_P, _S], _I),
    "mivi_hip_model_export_state": ([_P, _S, _S, _P, _P, _S, _P, _S], _I),
    "mivi_hip_model_import_state": ([_P, _S, _S, _P, _P, _S, _P, _S], _I),
    "mivi_hip_model_export_state_range": ([_P, _S, _S, _S, _P, _P, _S, _P, _S], _I),
    "mivi_hip_model_import_state_at": ([_P, _S, _S, _S, _P, _P, _S, _P, _S], _I),
    "mivi_hip_read_floor": ([_P, _S, _P], _I),
    "mivi_hip_prefix_cache_create": ([_S, _S, _S, C.POINTER(_P)], _I),
    "mivi_hip_prefix_cache_destroy": ([_P], None),
    "mivi_hip_prefix_chunk_hash": ([C.c_uint64, _P, _S], C.c_uint64),
    "mivi_hip_prefix_cache_insert_delta": ([_P, _P, _S, _S, C.c_uint64, _P, _S, _S, C.POINTER(C.c_uint64)], _I),
    "mivi_hip_prefix_cache_insert": ([_P, _P, _S, _S, C.c_uint64, _P, _S, _S, C.POINTER(C.c_uint64)], _I),
    "mivi_hip_prefix_cache_find_suffix": ([_P, _S, _P, _S, C.POINTER(_S), C.POINTER(_S), C.POINTER(C.c_uint64)], _I),
    "mivi_hip_prefix_cache_find": ([_P, _P, _S, C.POINTER(_S), C.POINTER(C.c_uint64)], _I),
    "mivi_hip_prefix_cache_restore": ([_P, _P, _S, _P, _S, C.POINTER(_S), C.POINTER(C.c_uint64)], _I),
    "mivi_hip_prefix_cache_len": ([_P], _S),
    "mivi_hip_prefix_cache_memory_bytes": ([_P], _S),
    "mivi_hip_prefix_cache_prune": ([_P, _S], _S),
    "mivi_hip_prefix_cache_clear": ([_P], None),
    "mivi_hip_prefix_cache_contains": ([_P, C.c_uint64], _I),
    "mivi_hip_sample": ([_P, _S, _P, _S, C.POINTER(SamplerConfig), _P, _P, _P], _I),
    "mivi_hip_sample_noalloc": ([_P, _S, _P, _S, C.POINTER(SamplerConfig), _P, _P, _P], _I),
    "mivi_hip_sample_rows_workspace": ([_S, _S], _S),
    "mivi_hip_sample_rows": ([_P, _S, _S, _S, _P, _S, _S, C.POINTER(SamplerConfig), _P, _P, _P, _S, _P], _I),
    "mivi_hip_model_generate": ([_P, _S, _P, _P, _S, C.POINTER(SamplerConfig), _P, _P, _S, _P], _I),
    "mivi_synth_normal": ([C.c_uint64, C.c_float, C.c_float, _P, _S], None),
    "mivi_synth_quantize": ([_I, _P, _S, _S, _P, _S], _I),
    "mivi_synth_random_weights": ([_I, C.c_uint64, C.c_float, _S, _S, _P, _S], _I),
}
for _name, (_args, _res) in _sig.items():
    _f = getattr(_lib, _name)
    _f.argtypes = _args
    _f.restype = _res


def lib() -> C.CDLL:
    return _lib


def version() -> str:
    return _lib.mivi_hip_version().decode()


def last_error() -> MiviError:
    e = MiviError()
    _lib.mivi_hip_last_error(C.byref(e))
    return e


def _check(rc: int, exc=QuantError):
    if rc != 0:
        e = last_error()
        if 1 <= rc <= 4:
            raise QuantError(e)
        raise exc(e)


# ---------------------------------------------------------------- buffers

def _dev(t):
    """(pointer, numel) of a torch tensor, or (0, 0) for None."""
    if t is None:
        return None, 0
    return C.c_void_p(t.data_ptr()), t.numel()


def _nbytes(t):
    return 0 if t is None else t.numel() * t.element_size()


def _stream(stream):
    if stream is None:
        import torch
        return C.c_void_p(torch.cuda.current_stream().cuda_stream)
    if isinstance(stream, int):
        return C.c_void_p(stream)
    return C.c_void_p(stream.cuda_stream)


# ------------------------------------------------------------ mivi-quant

def quantized_matvec(out, ggml_type, weights, x, n: int, d: int, stream=None):
    """lib.rs:75-134. out (f32), weights (u8), x (f32) are GPU tensors."""
    po, lo = _dev(out)
    px, lx = _dev(x)
    _check(_lib.mivi_hip_quantized_matvec(po, lo, int(ggml_type), C.c_void_p(weights.data_ptr()),
                                          _nbytes(weights), px, lx, n, d, _stream(stream)))


def _typed(fn):
    def call(out, weights, x, n: int, d: int, stream=None):
        po, lo = _dev(out)
        px, lx = _dev(x)
        _check(fn(po, lo, C.c_void_p(weights.data_ptr()), _nbytes(weights), px, lx, n, d, _stream(stream)))
    return call


try_matvec_q4_k_m = _typed(_lib.mivi_hip_try_matvec_q4_k_m)   # q4_k_m.rs:217
try_matvec_q6_k = _typed(_lib.mivi_hip_try_matvec_q6_k)       # q6_k.rs:202
try_matvec_q8_0 = _typed(_lib.mivi_hip_try_matvec_q8_0)       # q8_0.rs:127
try_matvec_f16 = _typed(_lib.mivi_hip_try_matvec_f16)         # f16.rs:42
try_matvec_bf16 = _typed(_lib.mivi_hip_try_matvec_bf16)       # f16.rs:75


def pack_weights(ggml_type, src, dst, rows: int, cols: int, stream=None):
    """Q6_K rows into the packed layout (row quads at 2048 columns and rows % 4 == 0, unit planes
    otherwise; u8 GPU tensors of equal size)."""
    _check(_lib.mivi_hip_pack_weights(int(ggml_type), C.c_void_p(src.data_ptr()), _nbytes(src),
                                      C.c_void_p(dst.data_ptr()), _nbytes(dst), rows, cols, _stream(stream)))


def quantized_matvec_packed(out, ggml_type, packed, x, n: int, d: int, stream=None):
    """quantized_matvec over rows packed by pack_weights."""
    po, lo = _dev(out)
    px, lx = _dev(x)
    _check(_lib.mivi_hip_quantized_matvec_packed(po, lo, int(ggml_type), C.c_void_p(packed.data_ptr()),
                                                 _nbytes(packed), px, lx, n, d, _stream(stream)))


def quantized_matmul_rows_packed(out, ggml_type, packed, inputs, batch: int, rows: int, cols: int, stream=None):
    """quantized_matmul_rows over rows packed by pack_weights."""
    po, lo = _dev(out)
    pi, li = _dev(inputs)
    _check(_lib.mivi_hip_quantized_matmul_rows_packed(po, lo, int(ggml_type), C.c_void_p(packed.data_ptr()),
                                                      _nbytes(packed), pi, li, batch, rows, cols, _stream(stream)))


def gemm_packed_size(ggml_type, rows: int, cols: int) -> int:
    """Bytes of pack_weights_gemm's copy (0: the shape has none)."""
    return int(_lib.mivi_hip_gemm_packed_size(int(ggml_type), rows, cols))


def pack_weights_gemm(ggml_type, src, dst, rows: int, cols: int, stream=None):
    """Q4_K rows into the row products' operand layout (u8 GPU tensors; dst of gemm_packed_size bytes)."""
    _check(_lib.mivi_hip_pack_weights_gemm(int(ggml_type), C.c_void_p(src.data_ptr()), _nbytes(src),
                                           C.c_void_p(dst.data_ptr()), _nbytes(dst), rows, cols, _stream(stream)))


def quantized_matmul_rows_gemm_packed(out, ggml_type, weights, wg, inputs, batch: int, rows: int, cols: int,
                                      stream=None):
    """quantized_matmul_rows with the weights' pack_weights_gemm copy wg (the matrix-core path reads it)."""
    po, lo = _dev(out)
    pi, li = _dev(inputs)
    _check(_lib.mivi_hip_quantized_matmul_rows_gemm_packed(po, lo, int(ggml_type), C.c_void_p(weights.data_ptr()),
                                                           _nbytes(weights), C.c_void_p(wg.data_ptr()), _nbytes(wg),
                                                           pi, li, batch, rows, cols, _stream(stream)))


def quantized_matmul_rows(out, ggml_type, weights, inputs, batch: int, rows: int, cols: int, stream=None):
    """lib.rs:143-251: out[batch, rows] = inputs[batch, cols] W^T."""
    po, lo = _dev(out)
    pi, li = _dev(inputs)
    _check(_lib.mivi_hip_quantized_matmul_rows(po, lo, int(ggml_type), C.c_void_p(weights.data_ptr()),
                                               _nbytes(weights), pi, li, batch, rows, cols, _stream(stream)))


def dequantize_slice(ggml_type, raw, out, stream=None):
    """lib.rs:35-72 (bit-exact)."""
    po, lo = _dev(out)
    _check(_lib.mivi_hip_dequantize_slice(int(ggml_type), C.c_void_p(raw.data_ptr()), _nbytes(raw), po, lo,
                                          _stream(stream)))


def quantize_f32_to_q8_0(src, dst, n_blocks: int, stream=None):
    """q8_0.rs:31-58 over n_blocks consecutive blocks."""
    ps, ls = _dev(src)
    _check(_lib.mivi_hip_quantize_q8_0(ps, ls, C.c_void_p(dst.data_ptr()), _nbytes(dst), n_blocks,
                                       _stream(stream)))


def dot_q8_0_f32(q, k_blocks, out, n: int, stream=None):
    """q8_0.rs:60-124 over n (q, k_block) pairs."""
    pq, lq = _dev(q)
    po, lo = _dev(out)
    _check(_lib.mivi_hip_dot_q8_0_f32(pq, lq, C.c_void_p(k_blocks.data_ptr()), _nbytes(k_blocks), po, lo, n,
                                      _stream(stream)))


def sample(logits, recent, cfg: SamplerConfig, rng_state, token, stream=None):
    """Sampler::sample (sampler.rs:91-135) on the device: logits (f32 GPU
    tensor) modified in place, recent (u32/i32 GPU tensor of token ids),
    rng_state (1-element int64 GPU tensor holding the u64 state), token
    (1-element int32 GPU tensor) receives the id."""
    _check(_lib.mivi_hip_sample(C.c_void_p(logits.data_ptr()), logits.numel(),
                                C.c_void_p(recent.data_ptr()) if recent is not None and recent.numel() else None,
                                recent.numel() if recent is not None else 0, C.byref(cfg),
                                C.c_void_p(rng_state.data_ptr()), C.c_void_p(token.data_ptr()), _stream(stream)))


def sample_noalloc(logits, recent, cfg: SamplerConfig, rng_state, token, stream=None):
    """sample() with the library's fixed device scratch in place of an
    allocated workspace (at most 262144 logits; calls overlapping on one GPU
    race): it allocates nothing, for callers that cannot."""
    _check(_lib.mivi_hip_sample_noalloc(C.c_void_p(logits.data_ptr()), logits.numel(),
                                        C.c_void_p(recent.data_ptr()) if recent is not None and recent.numel() else None,
                                        recent.numel() if recent is not None else 0, C.byref(cfg),
                                        C.c_void_p(rng_state.data_ptr()), C.c_void_p(token.data_ptr()),
                                        _stream(stream)))


def sample_rows(logits, recent, cfg: SamplerConfig, rng_states, tokens, stream=None):
    """Sampler::sample on every row of logits (2-D f32 GPU tensor, rows
    contiguous), one sampler per row: recent (2-D u32/i32 GPU tensor, row b =
    row b's penalty window, or None), rng_states (int64 GPU tensor, one u64
    state per row), tokens (int32 GPU tensor) receives the ids. The same
    results as sample() on each row; the workspace comes from torch."""
    import torch

    rows, n = logits.shape
    if logits.stride(1) != 1 or (recent is not None and recent.numel() and recent.stride(1) != 1):
        raise ValueError("rows must be contiguous")
    ws_bytes = _lib.mivi_hip_sample_rows_workspace(n, rows)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=logits.device)
    has_recent = recent is not None and recent.numel() > 0
    _check(_lib.mivi_hip_sample_rows(C.c_void_p(logits.data_ptr()), n, rows, logits.stride(0),
                                     C.c_void_p(recent.data_ptr()) if has_recent else None,
                                     recent.shape[1] if has_recent else 0, recent.stride(0) if has_recent else 0,
                                     C.byref(cfg), C.c_void_p(rng_states.data_ptr()), C.c_void_p(tokens.data_ptr()),
                                     C.c_void_p(ws.data_ptr()), ws_bytes, _stream(stream)))
    return ws


def read_floor(buf, nbytes: int, stream=None):
    """One plain coalesced read of nbytes of the u8 GPU tensor buf (the floor
    for any kernel reading those bytes)."""
    _check(_lib.mivi_hip_read_floor(C.c_void_p(buf.data_ptr()), nbytes, _stream(stream)))


# ----------------------------------------------------------- synthetic data

def synth_normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    _lib.mivi_synth_normal(seed, mean, std, out.ctypes.data_as(C.c_void_p), n)
    return out


def synth_quantize(ggml_type, src: np.ndarray, rows: int, cols: int) -> np.ndarray:
    t = GgmlType(ggml_type)
    src = np.ascontiguousarray(src, np.float32)
    dst = np.empty(rows * (cols // t.block_size()) * t.type_size(), np.uint8)
    _check(_lib.mivi_synth_quantize(int(t), src.ctypes.data_as(C.c_void_p), rows, cols,
                                    dst.ctypes.data_as(C.c_void_p), dst.nbytes))
    return dst


def synth_random_weights(ggml_type, seed: int, rows: int, cols: int, std: float = 0.02) -> np.ndarray:
    t = GgmlType(ggml_type)
    dst = np.empty(rows * (cols // t.block_size()) * t.type_size(), np.uint8)
    _check(_lib.mivi_synth_random_weights(int(t), seed, std, rows, cols, dst.ctypes.data_as(C.c_void_p),
                                          dst.nbytes))
    return dst


from .model import Model, PrefixCache, chunk_hash  # noqa: E402,F401
