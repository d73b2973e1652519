"""GPU parity of the mivi-quant surface through the C ABI (HIP kernels) against
the CPU oracle on identical packed bytes.

Bars: dequantization bit-exact; GEMV/GEMM max |y - y_ref| <=
1e-4 * ||w_row|| * ||x|| (fp32 accumulation), as the north star fixes.
"""
from __future__ import annotations

import numpy as np
import pytest

from test_oracle_quant import make_q6k_block, pattern_weights, random_blocks

pytestmark = pytest.mark.gpu

Q4_K, Q6_K, Q8_0, F16, BF16, F32 = 12, 14, 8, 1, 30, 0
BS = {Q4_K: 256, Q6_K: 256, Q8_0: 32, F16: 1, BF16: 1, F32: 1}
TS = {Q4_K: 144, Q6_K: 210, Q8_0: 34, F16: 2, BF16: 2, F32: 4}


def dev(torch, a):
    return torch.from_numpy(np.array(a, order="C", copy=True)).cuda()


def dense_bytes(t, W):
    if t == F32:
        return W.astype(np.float32).view(np.uint8).reshape(-1)
    if t == F16:
        return W.astype(np.float16).view(np.uint8).reshape(-1)
    return (W.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(-1)


def weights(t, rows, cols, seed):
    if t in (Q4_K, Q6_K, Q8_0):
        return random_blocks(t, rows, cols, seed)
    return dense_bytes(t, np.random.default_rng(seed).standard_normal((rows, cols)))


def check_bound(oracle, t, w, x, y, rows, cols):
    rc, deq, _ = oracle.dequantize_slice(t, w, rows * cols)
    W = deq.reshape(rows, cols).astype(np.float64)
    rc2, yref, _ = oracle.quantized_matvec(t, w, x, rows, cols)
    assert rc == 0 and rc2 == 0
    bound = 1e-4 * np.linalg.norm(W, axis=1) * np.linalg.norm(x.astype(np.float64))
    err = np.abs(y.astype(np.float64) - yref.astype(np.float64))
    assert np.all(err <= bound), (float(err.max()), float(bound.min()))


@pytest.mark.parametrize("t", [Q4_K, Q6_K, Q8_0, F16, BF16, F32])
def test_dequantize_bit_exact(hip, oracle, torch_mod, t):
    torch = torch_mod
    rows, cols = 37, 512
    w = weights(t, rows, cols, 100 + t)
    n = rows * cols
    out = torch.full((n + 3,), 7.5, dtype=torch.float32, device="cuda")
    hip.dequantize_slice(t, dev(torch, w), out[:n])
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    rc, ref, _ = oracle.dequantize_slice(t, w, n)
    assert rc == 0
    assert np.array_equal(got[:n].view(np.uint32), ref.view(np.uint32))
    assert np.all(got[n:] == 7.5)


def test_dequantize_exhaustive_q4k_scales(hip, oracle, torch_mod):
    # every 12-byte scale pattern position with all 256 byte values
    torch = torch_mod
    rng = np.random.default_rng(9)
    blocks = np.tile(random_blocks(Q4_K, 1, 256, 1), 12 * 256).reshape(12 * 256, 144)
    for p in range(12):
        blocks[p * 256:(p + 1) * 256, 4 + p] = np.arange(256)
    blocks[:, 16:] = rng.integers(0, 256, (12 * 256, 128))
    w = blocks.reshape(-1)
    n = 12 * 256 * 256
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    hip.dequantize_slice(Q4_K, dev(torch, w), out)
    torch.cuda.synchronize()
    rc, ref, _ = oracle.dequantize_slice(Q4_K, w, n)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))


SHAPES = [(1, 256), (7, 512), (255, 2048), (257, 2048), (100, 768), (33, 4096), (64, 8192)]


@pytest.mark.parametrize("t", [Q4_K, Q6_K, Q8_0])
@pytest.mark.parametrize("shape", SHAPES)
def test_gemv_matches_oracle(hip, oracle, torch_mod, t, shape):
    torch = torch_mod
    rows, cols = shape
    w = weights(t, rows, cols, rows * 7 + cols + t)
    x = np.random.default_rng(rows + cols).standard_normal(cols).astype(np.float32)
    out = torch.full((rows + 5,), -3.0, dtype=torch.float32, device="cuda")
    hip.quantized_matvec(out, t, dev(torch, w), dev(torch, x), rows, cols)
    torch.cuda.synchronize()
    y = out.cpu().numpy()
    assert np.all(y[rows:] == -3.0)      # tail untouched (types.rs:312-328)
    check_bound(oracle, t, w, x, y[:rows], rows, cols)


@pytest.mark.parametrize("t", [F16, BF16, F32])
def test_gemv_dense(hip, oracle, torch_mod, t):
    torch = torch_mod
    rows, cols = 129, 1000
    w = weights(t, rows, cols, 5)
    x = np.random.default_rng(6).standard_normal(cols).astype(np.float32)
    out = torch.empty(rows, dtype=torch.float32, device="cuda")
    hip.quantized_matvec(out, t, dev(torch, w), dev(torch, x), rows, cols)
    torch.cuda.synchronize()
    check_bound(oracle, t, w, x, out.cpu().numpy(), rows, cols)


def test_gemv_unaligned_f32_rows(hip, oracle, torch_mod):
    # lib.rs:95-129: F32 weights need not be 4-byte aligned
    torch = torch_mod
    rows, cols = 9, 50
    W = np.random.default_rng(1).standard_normal((rows, cols)).astype(np.float32)
    buf = np.zeros(rows * cols * 4 + 2, np.uint8)
    buf[2:] = W.view(np.uint8).reshape(-1)
    d = dev(torch, buf)
    x = np.random.default_rng(2).standard_normal(cols).astype(np.float32)
    out = torch.empty(rows, dtype=torch.float32, device="cuda")
    hip.quantized_matvec(out, F32, d[2:], dev(torch, x), rows, cols)
    torch.cuda.synchronize()
    check_bound(oracle, F32, W.view(np.uint8).reshape(-1), x, out.cpu().numpy(), rows, cols)


@pytest.mark.parametrize("fn,t", [("try_matvec_q4_k_m", Q4_K), ("try_matvec_q6_k", Q6_K), ("try_matvec_q8_0", Q8_0),
                                  ("try_matvec_f16", F16), ("try_matvec_bf16", BF16)])
def test_typed_entry_points(hip, oracle, torch_mod, fn, t):
    torch = torch_mod
    rows, cols = 40, 512
    w = weights(t, rows, cols, 77)
    x = np.random.default_rng(3).standard_normal(cols).astype(np.float32)
    out = torch.empty(rows, dtype=torch.float32, device="cuda")
    getattr(hip, fn)(out, dev(torch, w), dev(torch, x), rows, cols)
    torch.cuda.synchronize()
    check_bound(oracle, t, w, x, out.cpu().numpy(), rows, cols)


def test_q6k_all_offset_rows_are_exactly_zero(hip, torch_mod):
    torch = torch_mod
    blk = make_q6k_block(0.01, [100] * 16, [32] * 256)
    w = np.frombuffer(blk * 8 * 16, np.uint8)   # 16 rows of 2048
    x = np.random.default_rng(1).standard_normal(2048).astype(np.float32)
    out = torch.full((16,), 5.0, dtype=torch.float32, device="cuda")
    hip.quantized_matvec(out, Q6_K, dev(torch, w), dev(torch, x), 16, 2048)
    torch.cuda.synchronize()
    assert np.all(out.cpu().numpy() == 0.0)


def test_errors_leave_output_untouched(hip, torch_mod):
    # validation before any write (types.rs:146-235, lib.rs:152-169)
    torch = torch_mod
    w = torch.zeros(144 * 4, dtype=torch.uint8, device="cuda")
    x = torch.zeros(256, dtype=torch.float32, device="cuda")
    out = torch.full((4,), 9.0, dtype=torch.float32, device="cuda")
    for n, d, ww, xx, kind in ((4, 255, w, x, "DimensionMisaligned"), (5, 256, w, x, "BufferTooSmall"),
                               (4, 256, w[:500], x, "BufferTooSmall"), (4, 256, w, x[:200], "BufferTooSmall")):
        with pytest.raises(hip.QuantError) as ei:
            hip.quantized_matvec(out, Q4_K, ww, xx, n, d)
        assert ei.value.kind == kind
    with pytest.raises(hip.QuantError) as ei:
        hip.quantized_matvec(out, 2, w, x, 4, 256)
    assert ei.value.kind == "UnsupportedType" and ei.value.type_id == 2
    with pytest.raises(hip.QuantError):
        hip.quantized_matmul_rows(out, Q4_K, w, x, 2, 2, 256)   # out too small for 2x2? (4 ok) -> inputs short
    torch.cuda.synchronize()
    assert np.all(out.cpu().numpy() == 9.0)


@pytest.mark.parametrize("t", [Q4_K, Q6_K, Q8_0, F32])
@pytest.mark.parametrize("batch", [1, 2, 8, 9, 33])
def test_matmul_rows_matches_oracle(hip, oracle, torch_mod, t, batch):
    torch = torch_mod
    rows, cols = 257, 512
    w = pattern_weights(t, rows, cols) if t != F32 else weights(F32, rows, cols, 3)
    inputs = ((np.arange(batch * cols) % 23).astype(np.float32) * np.float32(0.0625) - np.float32(0.75))
    out = torch.full((batch * rows + 1,), 123.0, dtype=torch.float32, device="cuda")
    hip.quantized_matmul_rows(out[:batch * rows], t, dev(torch, w), dev(torch, inputs), batch, rows, cols)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert got[-1] == 123.0
    rc, ref, _ = oracle.quantized_matmul_rows(t, w, inputs, batch, rows, cols)
    rc2, deq, _ = oracle.dequantize_slice(t, w, rows * cols)
    W = deq.reshape(rows, cols).astype(np.float64)
    X = inputs.reshape(batch, cols).astype(np.float64)
    bound = 1e-4 * np.linalg.norm(X, axis=1)[:, None] * np.linalg.norm(W, axis=1)[None, :]
    assert np.all(np.abs(got[:-1].reshape(batch, rows) - ref.reshape(batch, rows)) <= bound)


def test_quantize_q8_0_bit_exact_and_dot(hip, oracle, torch_mod):
    torch = torch_mod
    nb = 4096
    src = (np.random.default_rng(4).standard_normal(nb * 32) * np.repeat(
        np.random.default_rng(5).uniform(0.001, 50, nb), 32)).astype(np.float32)
    src[:32] = 0.0                      # zero block
    src[32:64] = np.arange(32) - 16.0   # reference test values
    dst = torch.zeros(nb * 34, dtype=torch.uint8, device="cuda")
    hip.quantize_f32_to_q8_0(dev(torch, src), dst, nb)
    torch.cuda.synchronize()
    got = dst.cpu().numpy()
    ref = np.concatenate([oracle.quantize_q8_0_block(src[i * 32:(i + 1) * 32]) for i in range(nb)])
    assert np.array_equal(got, ref)
    q = np.random.default_rng(6).standard_normal(nb * 32).astype(np.float32)
    out = torch.empty(nb, dtype=torch.float32, device="cuda")
    hip.dot_q8_0_f32(dev(torch, q), dst, out, nb)
    torch.cuda.synchronize()
    d = out.cpu().numpy()
    for i in range(0, nb, 97):
        blk = ref[i * 34:(i + 1) * 34]
        qi = q[i * 32:(i + 1) * 32]
        r = oracle.dot_q8_0_f32(qi, blk)
        kd = oracle.dequantize_slice(Q8_0, blk, 32)[1].astype(np.float64)
        assert abs(d[i] - r) <= 1e-5 * np.abs(qi.astype(np.float64) * kd).sum() + 1e-30


@pytest.mark.parametrize("t,rows", [(Q4_K, 8192), (Q6_K, 65536)])
def test_config_shapes_match_oracle(hip, oracle, torch_mod, t, rows):
    # BASELINE configs 1 and 2 at full size, synthetic N(0, 0.02) weights
    torch = torch_mod
    cols = 2048
    w = hip.synth_random_weights(t, 42 + t, rows, cols, 0.02)
    x = hip.synth_normal(43, cols)
    out = torch.empty(rows, dtype=torch.float32, device="cuda")
    dw, dx = dev(torch, w), dev(torch, x)
    hip.quantized_matvec(out, t, dw, dx, rows, cols)
    torch.cuda.synchronize()
    y = out.cpu().numpy()
    check_bound(oracle, t, w, x, y, rows, cols)
    # size-independent property: linearity in x
    x2 = hip.synth_normal(44, cols)
    out2 = torch.empty(rows, dtype=torch.float32, device="cuda")
    out3 = torch.empty(rows, dtype=torch.float32, device="cuda")
    hip.quantized_matvec(out2, t, dw, dev(torch, x2), rows, cols)
    hip.quantized_matvec(out3, t, dw, dev(torch, (2.0 * x + x2).astype(np.float32)), rows, cols)
    torch.cuda.synchronize()
    lin = 2.0 * y + out2.cpu().numpy()
    assert np.max(np.abs(out3.cpu().numpy() - lin)) <= 1e-4 * np.abs(lin).max() + 1e-4


def _matmul_check(hip, oracle, torch, t, w, X, rows, cols):
    batch = X.shape[0]
    out = torch.full((batch * rows + 1,), 123.0, dtype=torch.float32, device="cuda")
    hip.quantized_matmul_rows(out[:batch * rows], t, dev(torch, w), dev(torch, X.reshape(-1)), batch, rows, cols)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert got[-1] == 123.0
    rc, ref, _ = oracle.quantized_matmul_rows(t, w, X.reshape(-1), batch, rows, cols)
    assert rc == 0
    rc2, deq, _ = oracle.dequantize_slice(t, w, rows * cols)
    wn = np.linalg.norm(deq.reshape(rows, cols).astype(np.float64), axis=1)
    xn = np.linalg.norm(X.astype(np.float64), axis=1)
    bound = 1e-4 * xn[:, None] * wn[None, :]
    err = np.abs(got[:-1].reshape(batch, rows).astype(np.float64) - ref.reshape(batch, rows))
    assert np.all(err <= bound), (float(err.max()), float((err / np.maximum(bound, 1e-30)).max()))


def test_matmul_rows_config3_shape(hip, oracle, torch_mod):
    # BASELINE config 3 at full size: X [512 x 2048] ~ N(0, 1), W [8192 x 2048] Q4_K (MFMA path)
    torch = torch_mod
    rows, cols, batch = 8192, 2048, 512
    w = hip.synth_random_weights(Q4_K, 77, rows, cols, 0.02)
    X = hip.synth_normal(78, batch * cols).reshape(batch, cols)
    _matmul_check(hip, oracle, torch, Q4_K, w, X, rows, cols)


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
@pytest.mark.parametrize("batch,rows,cols", [(16, 128, 2048), (127, 200, 2048), (129, 384, 4096), (70, 300, 8192)])
def test_matmul_rows_mfma_ragged_and_scaled_rows(hip, oracle, torch_mod, t, batch, rows, cols):
    # the matrix-core GEMM (at least 16 rows, cols % 2048 == 0): row
    # magnitudes from 0 to 1e3 (the per-row power-of-two scaling), ragged M
    # and N, Q4_K and Q6_K
    torch = torch_mod
    w = hip.synth_random_weights(t, 80 + batch, rows, cols, 0.02)
    X = hip.synth_normal(81 + batch, batch * cols).reshape(batch, cols).astype(np.float32)
    X[0] = 0.0
    X[1] *= np.float32(1e-3)
    X[2] *= np.float32(1e3)
    X[3] = 0.0
    X[3, 5] = np.float32(7.5e3)      # one dominant value
    _matmul_check(hip, oracle, torch, t, w, X, rows, cols)


def test_matmul_rows_q6k_ffn_down_prefill_shape(hip, oracle, torch_mod):
    # a Q4_K_M file's Q6_K ffn_down [2048 x 8192] on a prefill tile of 512
    # rows (the matrix-core GEMM with the per-sub-block scale)
    torch = torch_mod
    rows, cols, batch = 2048, 8192, 512
    w = hip.synth_random_weights(Q6_K, 83, rows, cols, 0.02)
    X = hip.synth_normal(84, batch * cols).reshape(batch, cols)
    _matmul_check(hip, oracle, torch, Q6_K, w, X, rows, cols)


@pytest.mark.parametrize("batch,rows,cols", [(16, 256, 2048), (512, 8192, 2048), (70, 2080, 2048), (33, 512, 8192),
                                             (129, 6144, 2048), (8, 64, 2048)])
def test_matmul_rows_gemm_packed_bit_exact(hip, torch_mod, batch, rows, cols):
    # the row products on the weights' operand-layout copy (sc * q converted
    # once, B loaded straight into the MFMA registers) against the same
    # products on the GGUF rows: the same MFMA chains in the same order, so
    # equal bit for bit (below 16 inputs both run the GEMVs on the GGUF rows)
    torch = torch_mod
    w = hip.synth_random_weights(Q4_K, 90 + batch, rows, cols, 0.02)
    X = hip.synth_normal(91 + batch, batch * cols)
    dw, dX = dev(torch, w), dev(torch, X)
    wg = torch.full((hip.gemm_packed_size(Q4_K, rows, cols),), 0xAB, dtype=torch.uint8, device="cuda")
    hip.pack_weights_gemm(Q4_K, dw, wg, rows, cols)
    a = torch.full((batch * rows + 1,), 7.0, dtype=torch.float32, device="cuda")
    b = torch.full((batch * rows + 1,), 7.0, dtype=torch.float32, device="cuda")
    hip.quantized_matmul_rows(a[:-1], Q4_K, dw, dX, batch, rows, cols)
    hip.quantized_matmul_rows_gemm_packed(b[:-1], Q4_K, dw, wg, dX, batch, rows, cols)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert b[-1].item() == 7.0


def test_gemm_pack_rejects_unsupported_shapes(hip, torch_mod):
    torch = torch_mod
    w = dev(torch, hip.synth_random_weights(Q4_K, 5, 40, 2048, 0.02))
    wg = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    with pytest.raises(hip.QuantError):
        hip.pack_weights_gemm(Q4_K, w, wg, 40, 2048)   # rows % 32
    w6 = dev(torch, hip.synth_random_weights(Q6_K, 5, 32, 2048, 0.02))
    with pytest.raises(hip.QuantError):
        hip.pack_weights_gemm(Q6_K, w6, wg, 32, 2048)  # Q4_K only


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
@pytest.mark.parametrize("batch,rows,cols", [(2, 64, 2048), (3, 1001, 2048), (5, 6144, 2048), (4, 65536, 2048),
                                             (7, 1001, 2048), (8, 8192, 2048), (15, 260, 2048),
                                             (3, 300, 8192), (6, 2048, 8192), (8, 2048, 8192), (5, 300, 8192),
                                             (2, 130, 4096)])
def test_batched_gemv_columns_match_matvec(hip, oracle, torch_mod, t, batch, rows, cols):
    # matmul_rows below the MFMA threshold runs batched GEMVs (inputs as
    # columns: up to 8 per launch at d = 2048 and 4 at d = 8192, Q4_K on the
    # int8 matrix cores; one launch per input at other depths): every input's
    # row of outputs equals its own matvec (lib.rs:404-457) bit for bit, except
    # on the Q4_K matrix-core kernel (3+ columns at d = 2048, any batch at
    # d = 8192), which takes the matvecs' activation digits but sums each
    # superblock in int32 before its float steps (the matvecs take a float
    # step per 64-value unit): it agrees to 1e-5 ||w_row|| ||x||, a tenth of
    # the bar; all meet the oracle bound
    torch = torch_mod
    w = hip.synth_random_weights(t, 70 + batch, rows, cols, 0.02)
    X = np.stack([hip.synth_normal(80 + b, cols) for b in range(batch)])
    dw, dX = dev(torch, w), dev(torch, X.reshape(-1))
    out = torch.full((batch * rows + 1,), 5.0, dtype=torch.float32, device="cuda")
    hip.quantized_matmul_rows(out[:batch * rows], t, dw, dX, batch, rows, cols)
    ones = []
    for b in range(batch):
        y = torch.empty(rows, dtype=torch.float32, device="cuda")
        hip.quantized_matvec(y, t, dw, dX[b * cols:(b + 1) * cols], rows, cols)
        ones.append(y)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert got[-1] == 5.0
    mfma_cols = t == Q4_K and ((cols == 2048 and batch > 2) or cols == 8192)
    if mfma_cols:
        rc, deq, _ = oracle.dequantize_slice(t, w, rows * cols)
        wn = np.linalg.norm(deq.reshape(rows, cols).astype(np.float64), axis=1)
    for b in range(batch):
        g, one = got[b * rows:(b + 1) * rows], ones[b].cpu().numpy()
        if mfma_cols:
            tol = 1e-5 * wn * np.linalg.norm(X[b].astype(np.float64))
            assert np.all(np.abs(g.astype(np.float64) - one) <= tol), b
        else:
            assert np.array_equal(g.view(np.uint32), one.view(np.uint32))
    if rows <= 1001:
        for b in range(batch):
            check_bound(oracle, t, w, X[b], got[b * rows:(b + 1) * rows], rows, cols)


def q6k_codes(w, rows, cols):
    """6-bit codes [rows, cols] of GGUF Q6_K rows (q6_k.rs:8-43, before the -32)."""
    B = w.reshape(rows, cols // 256, 210).astype(np.uint32)
    ql, qh = B[:, :, :128], B[:, :, 128:192]
    out = np.zeros((rows, cols // 256, 256), np.uint32)
    for h in range(2):
        for q in range(4):
            lo = ql[:, :, 64 * h + 32 * (q & 1):64 * h + 32 * (q & 1) + 32]
            lo = (lo >> 4) if q & 2 else (lo & 0xF)
            hi = (qh[:, :, 32 * h:32 * h + 32] >> (2 * q)) & 3
            out[:, :, 128 * h + 32 * q:128 * h + 32 * q + 32] = lo | (hi << 4)
    return out.reshape(rows, cols)


def quad_pack_ref(w, rows):
    """The row-quad packed layout of a Q6_K matrix with 2048 columns, restated
    from its definition: quad Q holds rows 4Q..4Q+3 in 6720 bytes; lane
    l = 4b + j owns units b and b + 16 of row j; slot g = 4i + q (quarter q of
    unit i) is dwords 3g..3g+2 of the lane's codes, byte e of dword 3g+m being
    c[4m+e] | (bits 2m..2m+1 of c[12+e]) << 6; then the slot scales; the d
    pairs (superblock s, s + 4) per (row, s < 4) follow (even quads) or lead
    (odd quads, whose codes and scales then start 64 bytes in)."""
    nq = rows // 4
    codes = q6k_codes(w, rows, 2048).reshape(nq, 4, 8, 256)
    B = w.reshape(nq, 4, 8, 210)
    out = np.zeros((nq, 6720), np.uint8)
    for l in range(64):
        b, j = l >> 2, l & 3
        for g in range(8):
            u, q = b + 16 * (g >> 2), g & 3
            sb, h, jj = u >> 2, (u >> 1) & 1, u & 1
            c = codes[:, j, sb, 128 * h + 32 * q + 16 * jj:128 * h + 32 * q + 16 * jj + 16]
            for m in range(3):
                byte = c[:, 4 * m:4 * m + 4] | (((c[:, 12:16] >> (2 * m)) & 3) << 6)
                D = 3 * g + m
                o = 1024 * (D >> 2) + 16 * l + 4 * (D & 3)
                out[:, o:o + 4] = byte.astype(np.uint8)
            out[:, 6144 + 8 * l + g] = B[:, j, sb, 192 + 8 * h + jj + 2 * q]
    for j in range(4):
        for s4 in range(4):
            o = 6656 + 4 * (4 * j + s4)
            out[:, o:o + 2] = B[:, j, s4, 208:210]
            out[:, o + 2:o + 4] = B[:, j, s4 + 4, 208:210]
    out[1::2] = np.roll(out[1::2], 64, axis=1)  # odd quads: d first
    return out.reshape(-1)


@pytest.mark.parametrize("rows,cols", [(64, 2048), (66, 2048), (1000, 4096), (130, 8192), (65536, 2048)])
def test_packed_q6k_matvec_bit_exact_with_raw(hip, oracle, torch_mod, rows, cols):
    # the packed GEMV must give the raw GEMV's result bit for bit, and both
    # meet the oracle bound; 2048 columns with rows % 4 == 0 use the row-quad
    # layout (matrix cores), other shapes the unit-plane byte permutation
    torch = torch_mod
    w = hip.synth_random_weights(Q6_K, 90 + cols, rows, cols, 0.02)
    x = hip.synth_normal(91, cols)
    dw, dx = dev(torch, w), dev(torch, x)
    packed = torch.empty_like(dw)
    hip.pack_weights(Q6_K, dw, packed, rows, cols)
    y_raw = torch.empty(rows, dtype=torch.float32, device="cuda")
    y_pk = torch.full((rows + 1,), 7.0, dtype=torch.float32, device="cuda")
    hip.quantized_matvec(y_raw, Q6_K, dw, dx, rows, cols)
    hip.quantized_matvec_packed(y_pk[:rows], Q6_K, packed, dx, rows, cols)
    torch.cuda.synchronize()
    a, b = y_raw.cpu().numpy(), y_pk.cpu().numpy()
    assert b[-1] == 7.0
    assert np.array_equal(a.view(np.uint32), b[:-1].view(np.uint32))
    pw = packed.cpu().numpy()
    if cols == 2048 and rows % 4 == 0:
        n = min(rows, 256)  # the layout restated on the first quads
        assert np.array_equal(pw[:n * 1680], quad_pack_ref(w[:n * 1680], n))
    else:
        # the unit-plane bytes are a permutation of each row
        pw = pw.reshape(rows, -1)
        assert np.array_equal(np.sort(pw[:3], axis=1), np.sort(w.reshape(rows, -1)[:3], axis=1))
    if rows <= 1000:
        check_bound(oracle, Q6_K, w, x, a, rows, cols)


def q4k_quad_pack_ref(oracle, w, nq, cols):
    """The row-quad packed layout of the first nq quads of a Q4_K matrix with
    cols = 2048 S columns, restated from its definition: sub-quad s of quad Q
    (4608 bytes) holds values [2048 s, 2048 s + 2048) of rows 4Q..4Q+3; lane
    l = 4b + j owns units t = 32 s + b and t + 16 of row j (unit t: sub-blocks
    2g, 2g + 1 of superblock t / 4, g = t & 3); the units' 32 code bytes at
    1024 k + 16 l (k = 0, 1 unit t, k = 2, 3 unit t + 16), the four sub-blocks'
    6-bit scales (bits 0-23) and mins (bits 24-47) in 6 bytes at 4096 + 6 l,
    the superblocks' d | dmin at 4480 + 8 (4 j + b / 4)."""
    S = cols // 2048
    B = w.reshape(-1, 4, cols // 256, 144)[:nq]
    out = np.zeros((nq, S, 4608), np.uint8)
    for q in range(nq):
        for l in range(64):
            b, j = l >> 2, l & 3
            for sq in range(S):
                bits = 0
                for ii in range(2):
                    t = 32 * sq + b + 16 * ii
                    g, blk = t & 3, B[q, j, t >> 2]
                    out[q, sq, 1024 * 2 * ii + 16 * l:1024 * 2 * ii + 16 * l + 16] = blk[16 + 32 * g:32 + 32 * g]
                    out[q, sq, 1024 * (2 * ii + 1) + 16 * l:1024 * (2 * ii + 1) + 16 * l + 16] = blk[32 + 32 * g:48 + 32 * g]
                    (s0, m0), (s1, m1) = (oracle.get_scale_min_k4(2 * g + h, blk[4:16]) for h in range(2))
                    bits |= (s0 | s1 << 6) << (12 * ii) | (m0 | m1 << 6) << (24 + 12 * ii)
                    o = 4480 + 8 * (4 * j + (b >> 2)) + 4 * ii
                    out[q, sq, o:o + 4] = blk[0:4]
                out[q, sq, 4096 + 6 * l:4096 + 6 * l + 6] = np.frombuffer(bits.to_bytes(6, "little"), np.uint8)
    return out.reshape(-1)


@pytest.mark.parametrize("rows,cols", [(4, 2048), (3072, 2048), (8192, 2048), (20000, 2048), (12, 8192), (2048, 8192)])
def test_packed_q4k_matvec_bit_exact_with_raw(hip, oracle, torch_mod, rows, cols):
    # Q4_K row quads (matrix cores): the packed GEMV gives the GGUF-row
    # streaming GEMV's result bit for bit, and meets the oracle bound
    torch = torch_mod
    w = hip.synth_random_weights(Q4_K, 70 + cols + rows, rows, cols, 0.02)
    x = hip.synth_normal(71 + rows, cols)
    dw, dx = dev(torch, w), dev(torch, x)
    packed = torch.empty_like(dw)
    hip.pack_weights(Q4_K, dw, packed, rows, cols)
    y_raw = torch.empty(rows, dtype=torch.float32, device="cuda")
    y_pk = torch.full((rows + 1,), 7.0, dtype=torch.float32, device="cuda")
    hip.quantized_matvec(y_raw, Q4_K, dw, dx, rows, cols)
    hip.quantized_matvec_packed(y_pk[:rows], Q4_K, packed, dx, rows, cols)
    torch.cuda.synchronize()
    a, b = y_raw.cpu().numpy(), y_pk.cpu().numpy()
    assert b[-1] == 7.0
    assert np.array_equal(a.view(np.uint32), b[:-1].view(np.uint32))
    nq = min(rows // 4, 3)
    assert np.array_equal(packed.cpu().numpy()[:nq * 4 * cols // 256 * 144], q4k_quad_pack_ref(oracle, w, nq, cols))
    if rows <= 3072:
        check_bound(oracle, Q4_K, w, x, a, rows, cols)


@pytest.mark.parametrize("t,batch,rows", [(Q6_K, 2, 64), (Q6_K, 3, 1000), (Q6_K, 4, 4096), (Q6_K, 5, 260),
                                           (Q6_K, 8, 65536), (Q6_K, 11, 4096), (Q4_K, 3, 64),
                                           (Q6_K, 3, 1001), (Q6_K, 6, 1002), (Q6_K, 8, 1003), (Q6_K, 5, 65535)])
def test_packed_matmul_rows_bit_exact_with_packed_matvec(hip, torch_mod, t, batch, rows):
    # the inputs as columns of batched packed launches (Q6_K row quads: up to
    # eight per launch, 3-4 and 5-8 columns in the two eight-wave variants, 2
    # in the two-column one; unit planes, rows not a multiple of four: two
    # columns per launch): every input's outputs equal its own packed
    # matvec bit for bit; a tiny, a huge, an all-zero and an infinite input
    # ride along (the infinite one: NaN outputs, as the matvec's)
    torch = torch_mod
    cols = 2048
    w = hip.synth_random_weights(t, 120 + batch, rows, cols, 0.02)
    X = np.stack([hip.synth_normal(130 + b, cols) for b in range(batch)])
    if batch > 2:
        X[1] *= np.float32(1e-3)
        X[2] *= np.float32(1e3)
    if batch > 4:
        X[3] = 0.0
        X[4, 17] = np.inf
    dw, dX = dev(torch, w), dev(torch, X.reshape(-1))
    packed = torch.empty_like(dw)
    hip.pack_weights(t, dw, packed, rows, cols)
    out = torch.full((batch * rows + 1,), 5.0, dtype=torch.float32, device="cuda")
    hip.quantized_matmul_rows_packed(out[:batch * rows], t, packed, dX, batch, rows, cols)
    ones = []
    for b in range(batch):
        y = torch.empty(rows, dtype=torch.float32, device="cuda")
        hip.quantized_matvec_packed(y, t, packed, dX[b * cols:(b + 1) * cols], rows, cols)
        ones.append(y)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert got[-1] == 5.0
    for b in range(batch):
        g, one = got[b * rows:(b + 1) * rows], ones[b].cpu().numpy()
        if np.isinf(X[b]).any():
            assert np.isnan(g).all() and np.isnan(one).all(), b
        else:
            assert np.array_equal(g.view(np.uint32), one.view(np.uint32)), b


def test_packed_rejects_other_types_and_shapes(hip, torch_mod):
    torch = torch_mod
    w = torch.zeros(144 * 8 * 6, dtype=torch.uint8, device="cuda")
    dst = torch.zeros_like(w)
    with pytest.raises(hip.QuantError):
        hip.pack_weights(Q4_K, w, dst, 6, 2048)    # Q4_K row quads need rows % 4 == 0
    with pytest.raises(hip.QuantError):
        hip.pack_weights(Q4_K, w, dst, 3, 4096)    # and 2048 or 8192 columns
    w8 = torch.zeros(34 * 64 * 4, dtype=torch.uint8, device="cuda")
    with pytest.raises(hip.QuantError):
        hip.pack_weights(Q8_0, w8, torch.zeros_like(w8), 4, 2048)
    w6 = torch.zeros(210 * 4 * 4, dtype=torch.uint8, device="cuda")
    with pytest.raises(hip.QuantError):
        hip.pack_weights(Q6_K, w6, torch.zeros_like(w6), 4, 1024)   # no packed layout for d = 1024
    out = torch.zeros(4, dtype=torch.float32, device="cuda")
    x = torch.zeros(1024, dtype=torch.float32, device="cuda")
    with pytest.raises(hip.QuantError):
        hip.quantized_matvec_packed(out, Q6_K, w6, x, 4, 1024)
    assert hip.last_error().code == 116
    with pytest.raises(hip.QuantError):
        hip.quantized_matmul_rows_packed(out, Q6_K, w6, x, 1, 4, 1024)
    assert hip.last_error().code == 116
