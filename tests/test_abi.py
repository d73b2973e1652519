"""The C-ABI library loads and exports every entry point include/mivi_hip.h
declares; host-side synthetic input generators behave (CPU only, no GPU
compute calls)."""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

from conftest import ROOT

LIB = os.path.join(ROOT, "mivi-v4_amd", "mivi_hip", "libmivi_hip.so")
HEADER = os.path.join(ROOT, "include", "mivi_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:mivi_hip|mivi_synth)_\w+)\s*\(", text)))


def test_header_declares_the_quant_and_model_surface():
    syms = declared_symbols()
    for s in ("mivi_hip_quantized_matvec", "mivi_hip_quantized_matmul_rows", "mivi_hip_dequantize_slice",
              "mivi_hip_try_matvec_q4_k_m", "mivi_hip_try_matvec_q6_k", "mivi_hip_try_matvec_q8_0",
              "mivi_hip_model_create", "mivi_hip_model_forward", "mivi_hip_model_generate_greedy"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB), "build the library first (python mivi-v4_amd/build.py)"
    lib = C.CDLL(LIB)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_gemm_packed_size_and_validation_need_no_gpu():
    # the row products' operand layout: Q4_K, rows % 32 == 0, cols % 2048 == 0
    import mivi_hip
    lib = mivi_hip.lib()
    assert mivi_hip.gemm_packed_size(12, 8192, 2048) == 8192 * 2048 * 2 + 256 * 8 * 640
    assert mivi_hip.gemm_packed_size(12, 2048, 8192) == 2048 * 8192 * 2 + 64 * 32 * 640
    assert mivi_hip.gemm_packed_size(12, 8200, 2048) == 0   # rows % 32
    assert mivi_hip.gemm_packed_size(12, 8192, 1024) == 0   # cols % 2048
    assert mivi_hip.gemm_packed_size(14, 8192, 2048) == 0   # Q6_K
    # validated on the host before anything is launched
    rc = lib.mivi_hip_pack_weights_gemm(12, None, 32 * 8 * 144, None, 16, 32, 2048, None)
    assert rc == 2 and mivi_hip.last_error().expected == mivi_hip.gemm_packed_size(12, 32, 2048)
    rc = lib.mivi_hip_quantized_matmul_rows_gemm_packed(None, 16 * 32, 12, None, 32 * 8 * 144, None, 0, None,
                                                        16 * 2048, 16, 32, 2048, None)
    assert rc == 2


def test_python_binding_imports():
    import mivi_hip
    assert "gfx950" in mivi_hip.version()


def test_validation_errors_need_no_gpu():
    # validation runs on the host before anything is launched
    # (types.rs:146-181); null device pointers are never dereferenced
    import mivi_hip
    lib = mivi_hip.lib()
    rc = lib.mivi_hip_quantized_matvec(None, 10, 12, None, 0, None, 0, 2, 255, None)
    assert rc == 3
    e = mivi_hip.last_error()
    assert e.dim == 255 and e.block_size == 256
    rc = lib.mivi_hip_quantized_matvec(None, 1, 12, None, 288, None, 256, 2, 256, None)
    assert rc == 2 and mivi_hip.last_error().expected == 2
    rc = lib.mivi_hip_quantized_matvec(None, 2, 2, None, 288, None, 256, 2, 256, None)
    assert rc == 1 and mivi_hip.last_error().type_id == 2
    rc = lib.mivi_hip_quantized_matmul_rows(None, 3, 8, None, 64, None, 64, 2, 2, 32, None)
    assert rc == 2 and mivi_hip.last_error().expected == 4


def test_synth_normals_are_seeded_and_normal():
    import mivi_hip
    a = mivi_hip.synth_normal(7, 200_001)
    b = mivi_hip.synth_normal(7, 200_001)
    c = mivi_hip.synth_normal(8, 200_001)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1) < 0.01


def test_synth_quantizers_roundtrip(oracle):
    # the encoders only make inputs; their output must decode (oracle) close to the source
    import mivi_hip
    rows, cols = 64, 512
    src = mivi_hip.synth_normal(3, rows * cols, 0.0, 0.02).reshape(rows, cols)
    for t, tol in ((mivi_hip.GgmlType.Q4_K, 0.15), (mivi_hip.GgmlType.Q6_K, 0.03), (mivi_hip.GgmlType.Q8_0, 0.01)):
        packed = mivi_hip.synth_quantize(t, src, rows, cols)
        rc, deq, _ = oracle.dequantize_slice(int(t), packed, rows * cols)
        rel = np.linalg.norm(deq - src.reshape(-1)) / np.linalg.norm(src)
        assert rc == 0 and rel < tol, (t, rel)
    w = mivi_hip.synth_random_weights(mivi_hip.GgmlType.Q4_K, 11, rows, cols)
    assert w.nbytes == rows * 2 * 144


def test_synthetic_model_loads_in_the_oracle(oracle):
    from mivi_hip.synthmodel import build_hybrid, weight_bytes_per_token
    cfg = dict(dim=256, hidden=512, n_layers=4, attn_layers=(1, 3), n_heads=4, n_kv=2, vocab=512)
    img = build_hybrid(**cfg, ctx_len=256)
    m = oracle.Model(img, max_ctx=256)
    assert m.info.n_attn_layers == 2 and m.info.ssm_conv_kernel == 3 and m.info.vocab_size == 512
    assert m.info.n_kv_heads == 2 and m.info.head_dim == 64
    logits = m.forward(3, 0)
    assert np.all(np.isfinite(logits))
    assert weight_bytes_per_token(**cfg) > 0
    # the config-4 shape streams 692,846,592 weight bytes per token
    from mivi_hip.synthmodel import LFM2_1B2
    assert weight_bytes_per_token(**LFM2_1B2) == 692_846_592


def test_q4_k_m_layout_counts():
    # a Q4_K_M file of the 1.2B shape keeps 11 matrices in Q6_K, the
    # embedding among them (CHANGELOG.md:584-586); the mixed layout of the
    # synthetic builder gives the same count (8 ffn_down, 2 attn_v), checked
    # on the GGUF it writes for a smaller model of the same layer pattern
    from mivi_hip.gguf import read_tensor_index
    from mivi_hip.synthmodel import LFM2_1B2, build_hybrid, q6k_matrices, weight_bytes_per_token
    q6 = q6k_matrices(LFM2_1B2["n_layers"], LFM2_1B2["attn_layers"], "q4_k_m")
    assert len(q6) + 1 == 11
    assert sum(n.endswith("ffn_down.weight") for n in q6) == 8 and sum(n.endswith("attn_v.weight") for n in q6) == 2
    small = dict(LFM2_1B2, dim=256, hidden=512, n_heads=4, n_kv=2, vocab=256)
    idx = read_tensor_index(build_hybrid(**small, ctx_len=256, mixed="q4_k_m"))
    got = {n for n, (t, dims, off, ln) in idx.items() if t == 14 and len(dims) == 2}
    assert got == q6 | {"token_embd.weight"}
    # every other matrix is Q4_K (the F32 ShortConv weights aside)
    assert all(t == 12 for n, (t, dims, off, ln) in idx.items() if len(dims) == 2 and n not in got and t != 0)
    # 10 matrices of 1.46x the Q4_K bytes: 35.1 MB more per token
    assert weight_bytes_per_token(**LFM2_1B2, mixed="q4_k_m") - weight_bytes_per_token(**LFM2_1B2) == (
        8 * 2048 * 32 + 2 * 512 * 8) * (210 - 144)
