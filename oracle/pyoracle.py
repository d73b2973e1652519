"""ctypes bindings for the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: the oracle is a C restatement of the reference's
Rust CPU path and is used as the parity checker and the timed CPU baseline.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module. The product (mivi-v4_amd/) never does.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 8, 12, 14, 30
KV_F32, KV_Q8_0, KV_F16RT = 0, 1, 100

BLOCK = {F32: 1, F16: 1, BF16: 1, Q8_0: 32, Q4_K: 256, Q6_K: 256}
TYPE_SIZE = {F32: 4, F16: 2, BF16: 2, Q8_0: 34, Q4_K: 144, Q6_K: 210}


class QuantError(C.Structure):
    _fields_ = [
        ("kind", C.c_int32),
        ("type_id", C.c_uint32),
        ("expected", C.c_size_t),
        ("actual", C.c_size_t),
        ("dim", C.c_size_t),
        ("block_size", C.c_size_t),
    ]


class ModelInfo(C.Structure):
    _fields_ = [
        (n, C.c_size_t)
        for n in (
            "dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "head_dim", "kv_dim",
            "vocab_size", "max_seq_len", "ssm_conv_kernel",
        )
    ] + [
        ("rope_base", C.c_float),
        ("rms_norm_eps", C.c_float),
        ("n_attn_layers", C.c_int32),
        ("yarn", C.c_int32),
        ("yarn_scale", C.c_float),
    ]


class SamplerConfig(C.Structure):
    """GenerationConfig's sampling fields (config.rs:163-194; defaults there)."""
    _fields_ = [(n, C.c_float) for n in ("temperature", "top_p", "min_p", "repetition_penalty",
                                         "presence_penalty", "frequency_penalty")] + [("top_k", C.c_uint32)]


def sampler_config(temperature=0.2, top_p=0.9, top_k=40, min_p=0.0, repetition_penalty=1.05,
                   presence_penalty=0.0, frequency_penalty=0.0) -> SamplerConfig:
    return SamplerConfig(temperature, top_p, min_p, repetition_penalty, presence_penalty, frequency_penalty, top_k)


_lib = None


def build():
    subprocess.check_call(["make", "-s", "-C", HERE])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        P = C.c_void_p
        S = C.c_size_t
        L.or_set_threads.argtypes = [C.c_int]
        L.or_set_serial_attention.argtypes = [C.c_int]
        L.or_get_threads.restype = C.c_int
        L.or_set_avx2.argtypes = [C.c_int]
        L.or_f16_to_f32.argtypes = [C.c_uint16]
        L.or_f16_to_f32.restype = C.c_float
        L.or_f32_to_f16.argtypes = [C.c_float]
        L.or_f32_to_f16.restype = C.c_uint16
        L.or_get_scale_min_k4.argtypes = [C.c_int, P, P, P]
        for n in ("or_dequantize_q4_k", "or_dequantize_q6_k", "or_dequantize_q8_0",
                  "or_quantize_q8_0_block"):
            getattr(L, n).argtypes = [P, P]
        L.or_dot_q8_0_f32.argtypes = [P, P]
        L.or_dot_q8_0_f32.restype = C.c_float
        L.or_dequantize_slice.argtypes = [C.c_int32, P, S, P, S, P]
        L.or_quantized_matvec.argtypes = [P, S, C.c_int32, P, S, P, S, S, S, P]
        L.or_quantized_matmul_rows.argtypes = [P, S, C.c_int32, P, S, P, S, S, S, S, P]
        L.or_compute_rms_scale.argtypes = [P, S, C.c_float]
        L.or_compute_rms_scale.restype = C.c_float
        L.or_rms_norm.argtypes = [P, P, P, S, C.c_float]
        L.or_rms_norm_in_place.argtypes = [P, P, S, C.c_float]
        L.or_dot_product.argtypes = [P, P, S]
        L.or_dot_product.restype = C.c_float
        L.or_silu.argtypes = [C.c_float]
        L.or_silu.restype = C.c_float
        L.or_swiglu.argtypes = [P, P, S]
        L.or_softmax.argtypes = [P, S]
        L.or_rope_table.argtypes = [P, P, S, S, C.c_float, C.c_int, C.c_float, S, C.c_float, C.c_float]
        L.or_rope_rotate.argtypes = [P, S, S, P, P]
        L.or_apply_rope_direct.argtypes = [P, S, P, S, S, S, C.c_float]
        L.or_argmax.argtypes = [P, S]
        L.or_sampler_seed.argtypes = [C.c_uint64]
        L.or_sampler_seed.restype = C.c_uint64
        L.or_random_f32.argtypes = [C.POINTER(C.c_uint64)]
        L.or_random_f32.restype = C.c_float
        L.or_apply_penalties.argtypes = [P, S, P, S, C.c_float, C.c_float, C.c_float]
        L.or_apply_min_p.argtypes = [P, S, C.c_float]
        L.or_apply_top_k.argtypes = [P, S, S]
        L.or_sample.argtypes = [P, S, P, S, C.POINTER(SamplerConfig), C.POINTER(C.c_uint64)]
        L.or_sample.restype = C.c_uint32
        L.or_argmax.restype = C.c_uint32
        L.or_attention.argtypes = [P, P, P, C.c_int, S, S, S, S, P]
        L.or_model_create.argtypes = [P, S, S, C.c_int, C.POINTER(P), C.c_char_p, S]
        L.or_model_destroy.argtypes = [P]
        L.or_model_info_get.argtypes = [P, C.POINTER(ModelInfo)]
        L.or_model_reset.argtypes = [P]
        L.or_model_forward_step.argtypes = [P, C.c_uint32, S, C.c_int]
        L.or_model_logits.argtypes = [P]
        L.or_model_logits.restype = C.POINTER(C.c_float)
        L.or_model_hidden.argtypes = [P]
        L.or_model_hidden.restype = C.POINTER(C.c_float)
        L.or_model_kv_bytes.argtypes = [P]
        L.or_model_kv_bytes.restype = S
        for n in ("or_model_k_cache", "or_model_v_cache"):
            getattr(L, n).argtypes = [P]
            getattr(L, n).restype = P
        L.or_model_conv_states.argtypes = [P]
        L.or_model_conv_states.restype = C.POINTER(C.c_float)
        L.or_model_conv_len.argtypes = [P]
        L.or_model_conv_len.restype = S
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def set_threads(n: int):
    lib().or_set_threads(int(n))


def set_serial_attention(on: bool):
    """Attention heads one after another, as the reference's
    compute_gqa_attention loops over them (transformer.rs:128); off by
    default (long caches spread the heads over the threads)."""
    lib().or_set_serial_attention(1 if on else 0)


def set_avx2(on: bool):
    lib().or_set_avx2(1 if on else 0)


def f16_to_f32(h: int) -> float:
    return lib().or_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return lib().or_f32_to_f16(f)


def get_scale_min_k4(j: int, q: np.ndarray):
    d = np.zeros(1, np.uint8)
    m = np.zeros(1, np.uint8)
    lib().or_get_scale_min_k4(j, _p(np.ascontiguousarray(q, np.uint8)), _p(d), _p(m))
    return int(d[0]), int(m[0])


def dequantize_slice(t: int, raw: np.ndarray, n_out: int):
    raw = np.ascontiguousarray(raw, np.uint8)
    out = np.zeros(n_out, np.float32)
    e = QuantError()
    rc = lib().or_dequantize_slice(t, _p(raw), raw.nbytes, _p(out), n_out, C.byref(e))
    return rc, out, e


def quantized_matvec(t: int, w: np.ndarray, x: np.ndarray, n: int, d: int, out_len=None):
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(n if out_len is None else out_len, np.float32)
    e = QuantError()
    rc = lib().or_quantized_matvec(_p(out), out.size, t, _p(w), w.nbytes, _p(x), x.size, n, d, C.byref(e))
    return rc, out, e


def quantized_matmul_rows(t: int, w: np.ndarray, inp: np.ndarray, batch: int, rows: int, cols: int,
                          out_len=None):
    w = np.ascontiguousarray(w, np.uint8)
    inp = np.ascontiguousarray(inp, np.float32)
    out = np.zeros(batch * rows if out_len is None else out_len, np.float32)
    e = QuantError()
    rc = lib().or_quantized_matmul_rows(_p(out), out.size, t, _p(w), w.nbytes, _p(inp), inp.size,
                                        batch, rows, cols, C.byref(e))
    return rc, out, e


def quantize_q8_0_block(src: np.ndarray) -> np.ndarray:
    src = np.ascontiguousarray(src, np.float32)
    dst = np.zeros(34, np.uint8)
    lib().or_quantize_q8_0_block(_p(src), _p(dst))
    return dst


def dot_q8_0_f32(q: np.ndarray, k_block: np.ndarray) -> float:
    return lib().or_dot_q8_0_f32(_p(np.ascontiguousarray(q, np.float32)),
                                 _p(np.ascontiguousarray(k_block, np.uint8)))


def rms_norm(x, w, eps=1e-5):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.zeros_like(x)
    lib().or_rms_norm(_p(out), _p(x), _p(w), x.size, eps)
    return out


def silu(v: float) -> float:
    return lib().or_silu(v)


def swiglu(g, u):
    g = np.array(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    lib().or_swiglu(_p(g), _p(u), g.size)
    return g


def softmax(x):
    x = np.array(x, np.float32)
    lib().or_softmax(_p(x), x.size)
    return x


def rope_table(head_dim, max_seq_len, rope_base, scaling=0, scale=1.0, orig=4096, beta_fast=32.0,
               beta_slow=1.0):
    half = head_dim // 2
    c = np.zeros(max_seq_len * half, np.float32)
    s = np.zeros(max_seq_len * half, np.float32)
    rc = lib().or_rope_table(_p(c), _p(s), head_dim, max_seq_len, rope_base, scaling, scale, orig,
                             beta_fast, beta_slow)
    assert rc == 0
    return c.reshape(max_seq_len, half), s.reshape(max_seq_len, half)


def rope_rotate(v, n_heads, head_dim, cos_row, sin_row):
    v = np.array(v, np.float32)
    lib().or_rope_rotate(_p(v), n_heads, head_dim, _p(np.ascontiguousarray(cos_row, np.float32)),
                         _p(np.ascontiguousarray(sin_row, np.float32)))
    return v


def apply_rope_direct(q, k, head_dim, pos, base):
    q = np.array(q, np.float32)
    k = np.array(k, np.float32)
    lib().or_apply_rope_direct(_p(q), q.size, _p(k), k.size, head_dim, pos, base)
    return q, k


def argmax(v) -> int:
    v = np.ascontiguousarray(v, np.float32)
    return int(lib().or_argmax(_p(v), v.size))


class Rng:
    """The sampler's xorshift64* state (sampler.rs:28-77)."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(lib().or_sampler_seed(seed))

    def random_f32(self) -> float:
        return lib().or_random_f32(C.byref(self.state))


def apply_penalties(l, recent, rep, presence, frequency):
    l = np.array(l, np.float32)
    r = np.ascontiguousarray(recent, np.uint32)
    lib().or_apply_penalties(_p(l), l.size, _p(r), r.size, rep, presence, frequency)
    return l


def apply_min_p(l, min_p):
    l = np.array(l, np.float32)
    lib().or_apply_min_p(_p(l), l.size, min_p)
    return l


def apply_top_k(l, k):
    l = np.array(l, np.float32)
    lib().or_apply_top_k(_p(l), l.size, k)
    return l


def sample(logits, recent, cfg: SamplerConfig, rng: Rng):
    """Sampler::sample (sampler.rs:91-135); returns (token, logits as modified)."""
    l = np.array(logits, np.float32)
    r = np.ascontiguousarray(recent, np.uint32)
    t = lib().or_sample(_p(l), l.size, _p(r) if r.size else None, r.size, C.byref(cfg), C.byref(rng.state))
    return int(t), l


def attention(q, K, V, prec, n_heads, n_kv, hd, seq):
    q = np.ascontiguousarray(q, np.float32)
    out = np.zeros(n_heads * hd, np.float32)
    lib().or_attention(_p(q), _p(np.ascontiguousarray(K)), _p(np.ascontiguousarray(V)), prec, n_heads, n_kv,
                       hd, seq, _p(out))
    return out


class Model:
    """The oracle's Model (model.rs:76-497) over an in-memory GGUF image."""

    def __init__(self, gguf: np.ndarray | bytes, max_ctx: int = 0, kv_precision: int = KV_F32):
        if isinstance(gguf, (bytes, bytearray)):
            gguf = np.frombuffer(bytes(gguf), np.uint8)
        self._img = np.ascontiguousarray(gguf, np.uint8)  # must outlive the model
        h = C.c_void_p()
        eb = C.create_string_buffer(256)
        rc = lib().or_model_create(_p(self._img), self._img.nbytes, max_ctx, kv_precision,
                                   C.byref(h), eb, 256)
        if rc != 0:
            raise RuntimeError("oracle model load failed: " + eb.value.decode())
        self._h = h
        self.info = ModelInfo()
        lib().or_model_info_get(self._h, C.byref(self.info))

    def close(self):
        if self._h:
            lib().or_model_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except TypeError:  # interpreter shutdown: the module's globals are already gone
            pass

    def reset(self):
        lib().or_model_reset(self._h)

    def forward_step(self, token: int, pos: int, compute_logits: bool = True) -> int:
        return lib().or_model_forward_step(self._h, token, pos, 1 if compute_logits else 0)

    def forward(self, token: int, pos: int) -> np.ndarray:
        rc = self.forward_step(token, pos, True)
        if rc != 0:
            raise RuntimeError(f"oracle forward failed rc={rc}")
        return self.logits()

    def logits(self) -> np.ndarray:
        p = lib().or_model_logits(self._h)
        return np.ctypeslib.as_array(p, shape=(self.info.vocab_size,)).copy()

    def hidden(self) -> np.ndarray:
        p = lib().or_model_hidden(self._h)
        return np.ctypeslib.as_array(p, shape=(self.info.dim,)).copy()

    def kv_views(self):
        n = lib().or_model_kv_bytes(self._h)
        kp = lib().or_model_k_cache(self._h)
        vp = lib().or_model_v_cache(self._h)
        k = np.ctypeslib.as_array((C.c_uint8 * n).from_address(kp))
        v = np.ctypeslib.as_array((C.c_uint8 * n).from_address(vp))
        return k, v

    def conv_view(self):
        n = lib().or_model_conv_len(self._h)
        return np.ctypeslib.as_array(lib().or_model_conv_states(self._h), shape=(n,))
