"""Pins the CPU oracle's mivi-quant restatement (CPU only).

Checks come from the reference's own tests (file:line cited per test), from
closed forms (the documented K-quant bit layouts, encoded independently here)
and from brute force in float64. The oracle is the checker of the GPU path.
"""
from __future__ import annotations

import struct

import numpy as np
import pytest

Q4_K, Q6_K, Q8_0, F16, BF16, F32 = 12, 14, 8, 1, 30, 0


def f16b(v: float) -> bytes:
    return np.float16(v).tobytes()


# ----------------------------------------------------------- known answers

def test_q6_k_known_answer(oracle):
    # crates/mivi-quant/src/q6_k.rs:236-252: d=1, scale[0]=2, ql[0]=5 -> -54.0
    blk = bytearray(210)
    blk[208:210] = f16b(1.0)
    blk[192] = 2
    blk[0] = 5
    rc, out, _ = oracle.dequantize_slice(Q6_K, np.frombuffer(bytes(blk), np.uint8), 256)
    assert rc == 0
    assert abs(out[0] - (-54.0)) < 1e-3


def test_q8_0_known_answer(oracle):
    # q8_0.rs:246-259: d = 0x4000 (2.0), q = 10, -5 -> 20, -10
    blk = bytearray(34)
    blk[0], blk[1] = 0x00, 0x40
    blk[2] = 10
    blk[3] = (-5) & 0xFF
    rc, out, _ = oracle.dequantize_slice(Q8_0, np.frombuffer(bytes(blk), np.uint8), 32)
    assert rc == 0 and out[0] == 20.0 and out[1] == -10.0


def test_q8_0_matvec_known_answer(oracle):
    # q8_0.rs:261-280: row 0 block 0 d=1.0, all ones; x = 2 -> 64.0
    dim, n = 64, 2
    w = bytearray(n * (dim // 32) * 34)
    w[0], w[1] = 0x00, 0x3C
    for j in range(32):
        w[2 + j] = 1
    x = np.full(dim, 2.0, np.float32)
    rc, out, _ = oracle.quantized_matvec(Q8_0, np.frombuffer(bytes(w), np.uint8), x, n, dim)
    assert rc == 0
    assert abs(out[0] - 64.0) < 1e-3
    assert out[1] == 0.0


def test_q8_0_quantize_and_dot(oracle):
    # q8_0.rs:282-307
    src = np.arange(32, dtype=np.float32) - 16.0
    blk = oracle.quantize_q8_0_block(src)
    rc, deq, _ = oracle.dequantize_slice(Q8_0, blk, 32)
    assert np.all(np.abs(src - deq) < 0.25)
    dot = oracle.dot_q8_0_f32(src, blk)
    expected = np.float32(0)
    for i in range(32):
        expected = np.float32(expected + src[i] * deq[i])
    assert abs(dot - expected) < 1e-3


def test_q8_0_fused_dot_accuracy(oracle):
    # tests/quantized_kv_and_prefill.rs:76-100
    i = np.arange(32, dtype=np.float32)
    q = np.clip(np.sin(i * np.float32(0.17)) * np.float32(2.5), -3, 3).astype(np.float32)
    k = np.clip(np.cos(i * np.float32(0.23)) * np.float32(1.8), -3, 3).astype(np.float32)
    blk = oracle.quantize_q8_0_block(k)
    approx = oracle.dot_q8_0_f32(q, blk)
    true = float(np.dot(q.astype(np.float64), k.astype(np.float64)))
    assert abs(approx - true) / max(abs(true), 1e-4) < 0.05


def test_q8_0_quantizer_closed_form(oracle):
    # q8_0.rs:31-58: d = amax/127 stored as f16 (RNE), q = round-half-away(x / d)
    rng = np.random.default_rng(5)
    for _ in range(200):
        x = (rng.standard_normal(32) * rng.uniform(0.01, 100)).astype(np.float32)
        blk = oracle.quantize_q8_0_block(x)
        amax = np.float32(np.max(np.abs(x)))
        d = np.float32(amax / np.float32(127.0))
        assert bytes(blk[:2]) == np.float16(d).tobytes()
        idv = np.float32(1.0) / d
        prod = (x * idv).astype(np.float32)
        q = np.where(prod >= 0, np.floor(prod + np.float32(0.5)), -np.floor(-prod + np.float32(0.5)))
        # halfway cases: f32 round() rounds away from zero
        exact_half = np.abs(prod - np.trunc(prod)) == 0.5
        q = np.where(exact_half, np.trunc(prod) + np.sign(prod), q)
        q = np.clip(q, -128, 127).astype(np.int8)
        assert np.array_equal(blk[2:].view(np.int8), q)
    # zero block: d = 0, all codes 0
    blk = oracle.quantize_q8_0_block(np.zeros(32, np.float32))
    assert np.all(blk == 0)


def test_f16_roundtrip_half_crate_semantics(oracle):
    # `half` 2.7.1: to_f32 exact, from_f32 RNE (q8_0.rs:246-273: 0x4000 = 2.0, 0x3C00 = 1.0)
    assert oracle.f16_to_f32(0x4000) == 2.0 and oracle.f16_to_f32(0x3C00) == 1.0
    for bits in range(0, 0x10000, 7):
        if (bits & 0x7C00) == 0x7C00:
            continue
        assert np.float32(oracle.f16_to_f32(bits)) == np.frombuffer(struct.pack("<H", bits), np.float16)[0]
    rng = np.random.default_rng(1)
    for v in rng.standard_normal(2000).astype(np.float32) * 100:
        assert oracle.f32_to_f16(float(v)) == int(np.float16(v).view(np.uint16))


# ----------------------------------------- closed-form K-quant bit layouts

def pack_q4k_scales(sc, mn):
    """The documented K-quant 6-bit scale packing (inverse of q4_k_m.rs:11-22)."""
    q = [0] * 12
    for j in range(4):
        q[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        q[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        q[j + 8] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
    return bytes(q)


def test_get_scale_min_k4_exhaustive(oracle):
    rng = np.random.default_rng(2)
    for j in range(8):
        for s in range(64):
            sc = [int(v) for v in rng.integers(0, 64, 8)]
            mn = [int(v) for v in rng.integers(0, 64, 8)]
            for m in range(64):
                sc[j], mn[j] = s, m
                q = np.frombuffer(pack_q4k_scales(sc, mn), np.uint8)
                assert oracle.get_scale_min_k4(j, q) == (s, m)


def make_q4k_block(d, dmin, sc, mn, codes):
    """codes[256] in 0..15; layout q4_k_m.rs:24-58: group g byte l holds
    value 64g+l (low nibble) and 64g+32+l (high nibble)."""
    qs = bytearray(128)
    for g in range(4):
        for l in range(32):
            qs[32 * g + l] = codes[64 * g + l] | (codes[64 * g + 32 + l] << 4)
    return f16b(d) + f16b(dmin) + pack_q4k_scales(sc, mn) + bytes(qs)


def test_q4k_dequant_closed_form(oracle):
    rng = np.random.default_rng(3)
    for _ in range(50):
        d, dmin = float(rng.uniform(0.001, 0.1)), float(rng.uniform(0.001, 0.1))
        sc = [int(v) for v in rng.integers(0, 64, 8)]
        mn = [int(v) for v in rng.integers(0, 64, 8)]
        codes = [int(v) for v in rng.integers(0, 16, 256)]
        blk = make_q4k_block(d, dmin, sc, mn, codes)
        rc, out, _ = oracle.dequantize_slice(Q4_K, np.frombuffer(blk, np.uint8), 256)
        df, mf = np.float32(np.float16(d)), np.float32(np.float16(dmin))
        for e in range(256):
            s = e // 32
            want = np.float32(np.float32(df * np.float32(sc[s])) * np.float32(codes[e])) - np.float32(mf * np.float32(mn[s]))
            assert out[e] == np.float32(want), (e, out[e], want)


def make_q6k_block(d, scales, codes):
    """codes[256] in 0..63 (value = code - 32); layout q6_k.rs:8-38."""
    ql, qh = bytearray(128), bytearray(64)
    for h in range(2):
        c = codes[128 * h:128 * h + 128]
        for l in range(32):
            ql[64 * h + l] = (c[l] & 0xF) | ((c[l + 64] & 0xF) << 4)
            ql[64 * h + 32 + l] = (c[l + 32] & 0xF) | ((c[l + 96] & 0xF) << 4)
            qh[32 * h + l] = (c[l] >> 4) | ((c[l + 32] >> 4) << 2) | ((c[l + 64] >> 4) << 4) | ((c[l + 96] >> 4) << 6)
    return bytes(ql) + bytes(qh) + np.asarray(scales, np.int8).tobytes() + f16b(d)


def test_q6k_dequant_closed_form(oracle):
    rng = np.random.default_rng(4)
    for _ in range(50):
        d = float(rng.uniform(0.0001, 0.01))
        scales = [int(v) for v in rng.integers(-128, 128, 16)]
        codes = [int(v) for v in rng.integers(0, 64, 256)]
        blk = make_q6k_block(d, scales, codes)
        rc, out, _ = oracle.dequantize_slice(Q6_K, np.frombuffer(blk, np.uint8), 256)
        df = np.float32(np.float16(d))
        for e in range(256):
            want = np.float32(np.float32(df * np.float32(scales[e // 16])) * np.float32(codes[e] - 32))
            assert out[e] == want


# ----------------------------------------------------- matvec / matmul

def random_blocks(t, rows, cols, seed):
    """Random packed bytes with finite f16 scales (|d| small, sane)."""
    rng = np.random.default_rng(seed)
    bs, ts = {Q4_K: (256, 144), Q6_K: (256, 210), Q8_0: (32, 34)}[t]
    nb = rows * cols // bs
    raw = rng.integers(0, 256, (nb, ts), dtype=np.uint8)
    scale_off = {Q4_K: [0, 2], Q6_K: [208], Q8_0: [0]}[t]
    for o in scale_off:
        raw[:, o:o + 2] = np.frombuffer(
            rng.uniform(-0.05, 0.05, nb).astype(np.float16).tobytes(), np.uint8).reshape(nb, 2)
    return raw.reshape(-1)


@pytest.mark.parametrize("t", [Q4_K, Q6_K, Q8_0])
@pytest.mark.parametrize("avx2", [True, False])
def test_matvec_f64_brute_force(oracle, t, avx2):
    rows, cols = 300, 512
    w = random_blocks(t, rows, cols, 10 + t)
    x = np.random.default_rng(7).standard_normal(cols).astype(np.float32)
    oracle.set_avx2(avx2)
    try:
        rc, y, _ = oracle.quantized_matvec(t, w, x, rows, cols)
    finally:
        oracle.set_avx2(True)
    assert rc == 0
    rc, deq, _ = oracle.dequantize_slice(t, w, rows * cols)
    W = deq.reshape(rows, cols).astype(np.float64)
    y64 = W @ x.astype(np.float64)
    bound = 1e-4 * np.linalg.norm(W, axis=1) * np.linalg.norm(x.astype(np.float64))
    assert np.all(np.abs(y - y64) <= bound)


def test_dense_matvec(oracle):
    rng = np.random.default_rng(8)
    rows, cols = 17, 100
    Wf = rng.standard_normal((rows, cols)).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    for t, raw in ((F32, Wf.tobytes()), (F16, Wf.astype(np.float16).tobytes()),
                   (BF16, (Wf.view(np.uint32) >> 16).astype(np.uint16).tobytes())):
        rc, y, _ = oracle.quantized_matvec(t, np.frombuffer(raw, np.uint8), x, rows, cols)
        rc2, deq, _ = oracle.dequantize_slice(t, np.frombuffer(raw, np.uint8), rows * cols)
        y64 = deq.reshape(rows, cols).astype(np.float64) @ x.astype(np.float64)
        assert rc == 0 and rc2 == 0
        assert np.allclose(y, y64, rtol=0, atol=1e-4 * np.abs(y64).max() + 1e-5)


@pytest.mark.parametrize("t,cols", [(F32, 8), (F16, 8), (BF16, 8), (Q8_0, 32), (Q4_K, 256), (Q6_K, 256)])
def test_batched_matches_matvec(oracle, t, cols):
    # crates/mivi-quant/src/lib.rs:367-412: zero weights, batch 1..3, exact equality
    rows = 3
    ts = {F32: 4, F16: 2, BF16: 2, Q8_0: 34, Q4_K: 144, Q6_K: 210}[t]
    bs = {F32: 1, F16: 1, BF16: 1, Q8_0: 32, Q4_K: 256, Q6_K: 256}[t]
    w = np.zeros(rows * cols // bs * ts, np.uint8)
    inputs = ((np.arange(3 * cols, dtype=np.float32) - 3.0) * np.float32(0.125)).astype(np.float32)
    for batch in (1, 2, 3):
        exp = np.zeros(batch * rows, np.float32)
        for b in range(batch):
            rc, y, _ = oracle.quantized_matvec(t, w, inputs[b * cols:(b + 1) * cols], rows, cols)
            exp[b * rows:(b + 1) * rows] = y
        rc, act, _ = oracle.quantized_matmul_rows(t, w, inputs[:batch * cols], batch, rows, cols)
        assert rc == 0 and np.array_equal(act, exp)


def pattern_weights(t, rows, cols):
    # lib.rs:419-429 / 491-510 byte patterns: ((i + 7 j) % 127), scale 0.125 (and dmin 0.0625)
    ts = {Q4_K: 144, Q6_K: 210, Q8_0: 34}[t]
    bs = {Q4_K: 256, Q6_K: 256, Q8_0: 32}[t]
    nb = rows * cols // bs
    i = np.arange(nb)[:, None]
    j = np.arange(ts)[None, :]
    w = ((i + 7 * j) % 127).astype(np.uint8)
    so = ts - 2 if t == Q6_K else 0
    w[:, so:so + 2] = np.frombuffer(f16b(0.125), np.uint8)
    if t == Q4_K:
        w[:, 2:4] = np.frombuffer(f16b(0.0625), np.uint8)
    return w.reshape(-1)


@pytest.mark.parametrize("t", [Q4_K, Q8_0])
def test_large_batches_match_matvec(oracle, t):
    # lib.rs:414-457
    cols, rows = 512, 257
    w = pattern_weights(t, rows, cols)
    for batch in (9, 32, 33, 64, 65):
        inputs = ((np.arange(batch * cols) % 23).astype(np.float32) * np.float32(0.0625) - np.float32(0.75))
        rc, act, _ = oracle.quantized_matmul_rows(t, w, inputs, batch, rows, cols)
        assert rc == 0
        for b in range(batch):
            rc, exp, _ = oracle.quantized_matvec(t, w, inputs[b * cols:(b + 1) * cols], rows, cols)
            assert np.all(np.abs(act[b * rows:(b + 1) * rows] - exp) < 1e-3)


def test_matmul_leaves_tail_untouched(oracle):
    # lib.rs:523-561: out longer than batch*rows keeps its sentinel
    t, cols, rows, batch = Q6_K, 256, 3, 33
    w = pattern_weights(t, rows, cols)
    inputs = ((np.arange(batch * cols) % 23).astype(np.float32) * np.float32(0.0625) - np.float32(0.75))
    import ctypes as C
    out = np.zeros(batch * rows + 1, np.float32)
    out[-1] = 123.0
    e = oracle.QuantError()
    lib = oracle.lib()
    rc = lib.or_quantized_matmul_rows(out.ctypes.data_as(C.c_void_p), out.size, t,
                                      w.ctypes.data_as(C.c_void_p), w.nbytes,
                                      inputs.ctypes.data_as(C.c_void_p), inputs.size, batch, rows, cols, C.byref(e))
    assert rc == 0 and out[-1] == 123.0


def test_matmul_errors(oracle):
    # lib.rs:567-607 and types.rs:330-337
    w = np.zeros(2 * 32, np.uint8)
    inp = np.zeros(2 * 32, np.float32)
    rc, _, e = oracle.quantized_matmul_rows(Q8_0, w, inp, 2, 2, 32, out_len=3)
    assert rc == 2 and e.expected == 4 and e.actual == 3
    rc, _, e = oracle.quantized_matmul_rows(Q8_0, w, inp[:31], 2, 2, 32)
    assert rc == 2
    rc, _, e = oracle.quantized_matmul_rows(Q8_0, w[:31], inp, 2, 2, 32)
    assert rc == 2
    rc, _, e = oracle.quantized_matmul_rows(Q8_0, w, inp, 2, 2, 31)
    assert rc == 3 and e.dim == 31 and e.block_size == 32
    rc, _, e = oracle.quantized_matmul_rows(4, w, inp, 2, 2, 32)
    assert rc == 1 and e.type_id == 4


def test_matvec_errors(oracle):
    w = np.zeros(144 * 2, np.uint8)
    x = np.zeros(256, np.float32)
    assert oracle.quantized_matvec(Q4_K, w, x, 2, 255)[0] == 3
    assert oracle.quantized_matvec(Q4_K, w, x, 2, 256, out_len=1)[0] == 2
    assert oracle.quantized_matvec(Q4_K, w, x[:255], 2, 256)[0] == 2
    assert oracle.quantized_matvec(Q4_K, w[:287], x, 2, 256)[0] == 2
    assert oracle.quantized_matvec(2, w, x, 2, 256)[0] == 1  # Q4_0 has no matvec arm


def test_q6k_all_offset_block_gives_zero(oracle):
    # every code 32 means w == 0 exactly; the result must be exactly 0
    blk = make_q6k_block(0.01, [100] * 16, [32] * 256)
    w = np.frombuffer(blk * 4, np.uint8)
    x = np.random.default_rng(1).standard_normal(256).astype(np.float32)
    rc, y, _ = oracle.quantized_matvec(Q6_K, w, x, 4, 256)
    assert rc == 0 and np.all(y == 0.0)
