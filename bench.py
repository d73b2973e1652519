"""Benchmark of the mivi-v4 quantized-inference hot path on one MI355X.

Default line (BASELINE.json metric, configs[1]): the Q6_K output-head GEMV,
W [65536 x 2048] from seeded N(0, 0.02), x [2048] ~ N(0, 1), reported as HBM
GB/s of algorithmic bytes (W + x + y = 110,370,816 B per call). Weights are
rotated over enough distinct copies (> 1 GB) that the 256 MB Infinity Cache
cannot serve repeats; inputs are resident in HBM before timing.

`extra` carries the other configs measured in the same run: the Q4_K GEMV
(config 1), the Q4_K prefill GEMM (config 3) and, unless --no-decode, the
1.2B-shape hybrid decode (config 4: fp16 KV prefilled with 4096 tokens, 256
greedy steps) and the batched long-context decode (config 5: 8 sequences,
Q8_0 KV of 32768 tokens, 128 greedy steps) in tok/s. Each carries the CPU
oracle's figure on this host (the process's CPUs, at most 16, and the
reference binary's default of 2 threads), and the decodes a parity record:
the device's greedy tokens against the oracle's from the same state.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-decode] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mivi-v4_amd"))

HBM_PEAK_GBS = 8000.0
WARM_S = 0.5  # seconds of untimed launches before each GEMV timing
METRIC = "Q4_K/Q6_K GEMV HBM GB/s (% of peak); 1.2B hybrid decode tok/s at batch 1"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def graph_ms(torch, launch, n, reps=3):
    """ms per launch of `n` dependent launches (launch(i, stream)) captured in
    one HIP graph on a side stream, as the decode step runs its kernels:
    WARM_S of untimed replays, then the median of `reps` replays timed with
    HIP events on that stream. Without the graph a Python loop issues a
    launch every 4-5 us, about a short GEMV's own duration, so the loop's
    figure (host_loop_ms_per_call) partly times the host."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(n):
            launch(i, s)
    times = []
    with torch.cuda.stream(s):
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < WARM_S:
            g.replay()
            torch.cuda.synchronize()
        for _ in range(reps):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(s)
            g.replay()
            e1.record(s)
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1) / n)
    del g
    return sorted(times)[len(times) // 2]


def gemv_bench(torch, hip, t, rows, cols, steps, warmup, seed, packed=False):
    """Times `steps` launches over rotating weight copies; returns dict.
    packed: the weights are first rewritten once by mivi_hip_pack_weights
    (the same bytes rearranged; not timed) and the packed GEMV is timed.
    Then the same copies are read once each by mivi_hip_read_floor, a plain
    coalesced read, timed the same way: the floor for these bytes.
    ms_per_call: the launches in one graph (graph_ms); host_loop_ms_per_call:
    the same launches issued one by one from Python."""
    stream = torch.cuda.current_stream()
    w_host = hip.synth_random_weights(t, seed, rows, cols, 0.02)
    x_host = hip.synth_normal(seed + 1, cols)
    wbytes = w_host.nbytes
    copies = max(4, -(-1_100_000_000 // wbytes))
    base = torch.from_numpy(w_host).cuda()
    if packed:
        pk = torch.empty_like(base)
        hip.pack_weights(t, base, pk, rows, cols, stream=stream)
        base = pk
    ws = [base] + [base.clone() for _ in range(copies - 1)]
    x = torch.from_numpy(x_host).cuda()
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    mv = hip.quantized_matvec_packed if packed else hip.quantized_matvec
    for i in range(warmup):
        mv(y, t, ws[i % copies], x, rows, cols, stream=stream)
    torch.cuda.synchronize()
    # then at least WARM_S of back-to-back launches: the first few hundred
    # milliseconds of GPU work on a fresh box run about 20 % slower
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < WARM_S:
        for i in range(100):
            mv(y, t, ws[i % copies], x, rows, cols, stream=stream)
        torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(steps):
        mv(y, t, ws[i % copies], x, rows, cols, stream=stream)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    loop_ms = e0.elapsed_time(e1) / steps
    ev_ms = graph_ms(torch, lambda i, s: mv(y, t, ws[i % copies], x, rows, cols, stream=s), steps)
    for i in range(2 * copies):
        hip.read_floor(ws[i % copies], wbytes, stream=stream)
    torch.cuda.synchronize()
    floor_ms = graph_ms(torch, lambda i, s: hip.read_floor(ws[i % copies], wbytes, stream=s), steps)
    algo = wbytes + cols * 4 + rows * 4
    return dict(rows=rows, cols=cols, weight_bytes=wbytes, algo_bytes=algo, copies=copies,
                ms_per_call=ev_ms, host_loop_ms_per_call=loop_ms, wall_ms_per_call=1e3 * wall / steps,
                gbs=algo / (ev_ms * 1e-3) / 1e9,
                read_floor_us=floor_ms * 1e3, frac_of_read_floor=floor_ms / ev_ms,
                w_host=w_host, x_host=x_host)


REF_THREADS = 2  # the reference binary's default rayon pool: at most 2 threads (src/main.rs:12-24)


def cpu_threads():
    """(threads of the CPU legs, CPUs visible to this process): every CPU the
    process may run on, at most 16 (the host cores one GPU's box grants)."""
    try:
        vis = len(os.sched_getaffinity(0))
    except AttributeError:
        vis = os.cpu_count() or 1
    return max(1, min(vis, 16)), vis


def _oracle():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle
    return pyoracle


def cpu_time(fn, budget_s, min_calls=1):
    """Seconds per call of fn after one untimed call, over about budget_s."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        if n >= min_calls and time.perf_counter() - t0 > budget_s:
            break
    return (time.perf_counter() - t0) / n, n


def cpu_gemv_baseline(t, w, x, rows, cols, budget_s):
    """The oracle's AVX2 restatement of try_matvec on the same bytes at the
    process's threads (the primary figure) and at the reference binary's 2."""
    pyoracle = _oracle()
    threads, vis = cpu_threads()
    algo = w.nbytes + cols * 4 + rows * 4
    res = None
    for th, budget in ((threads, budget_s), (REF_THREADS, budget_s / 2)):
        pyoracle.set_threads(th)
        sec, n = cpu_time(lambda: pyoracle.quantized_matvec(int(t), w, x, rows, cols), budget)
        leg = dict(value=algo / sec / 1e9, unit="GB/s", cores=th, kind="port",
                   sample=f"{n} calls of the oracle's AVX2 restatement of try_matvec (same {rows}x{cols} bytes), "
                          f"{sec * 1e3:.2f} ms/call")
        if res is None:
            res = dict(leg, host_cpus_visible=vis)
        else:
            res["at_reference_default_threads"] = leg
    return res


def cpu_gemm_baseline(w, x, batch, rows, cols, budget_s):
    """Config 3 on the CPU: the oracle's restatement of quantized_matmul_rows
    (lib.rs:143-357, batch > 8: transposed inputs, per-lane accumulation)."""
    pyoracle = _oracle()
    threads, vis = cpu_threads()
    flop = 2.0 * batch * rows * cols
    out = {"host_cpus_visible": vis}
    for th, budget in ((threads, budget_s), (REF_THREADS, budget_s)):
        pyoracle.set_threads(th)
        sec, n = cpu_time(lambda: pyoracle.quantized_matmul_rows(12, w, x, batch, rows, cols), budget)
        out[f"threads_{th}"] = dict(value=flop / sec / 1e12, unit="TFLOP/s", cores=th, kind="port",
                                    sample=f"{n} calls at batch {batch}, {sec * 1e3:.0f} ms/call")
    return out


def gemm_bench(torch, hip, steps, warmup, cpu_budget_s=0.0):
    """Config 3: X [512 x 2048] ~ N(0,1) times W [8192 x 2048]^T Q4_K on MFMA: the row products on the
    weights' operand-layout copy (sc * q converted once, as the model keeps it; packing not timed), and
    the same products staging B from the GGUF rows per call (bit-identical results)."""
    rows, cols, batch = 8192, 2048, 512
    t = hip.GgmlType.Q4_K
    w_host = hip.synth_random_weights(t, 300, rows, cols, 0.02)
    x_host = hip.synth_normal(301, batch * cols)
    w = torch.from_numpy(w_host).cuda()
    x = torch.from_numpy(x_host).cuda()
    wg = torch.empty(hip.gemm_packed_size(t, rows, cols), dtype=torch.uint8, device="cuda")
    hip.pack_weights_gemm(t, w, wg, rows, cols)
    y = torch.empty(batch * rows, dtype=torch.float32, device="cuda")
    y2 = torch.empty(batch * rows, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    ms = timed(lambda: hip.quantized_matmul_rows_gemm_packed(y, t, w, wg, x, batch, rows, cols, stream=stream))
    ms_gguf = timed(lambda: hip.quantized_matmul_rows(y2, t, w, x, batch, rows, cols, stream=stream))
    torch.cuda.synchronize()
    flop = 2.0 * batch * rows * cols
    res = dict(batch=batch, rows=rows, cols=cols, algo_flop=flop, ms_per_call=ms,
               tflops=flop / (ms * 1e-3) / 1e12, frac_of_fp16_mfma_peak=flop / (ms * 1e-3) / 2.5e15,
               weight_layout="B operand converted once (mivi_hip_pack_weights_gemm, not timed)",
               bit_identical_to_gguf_rows=bool(torch.equal(y, y2)),
               gguf_rows=dict(ms_per_call=ms_gguf, tflops=flop / (ms_gguf * 1e-3) / 1e12),
               note="includes the activation split kernel (fp16 hi/lo + sub-block sums) run per call")
    if cpu_budget_s > 0:
        res["cpu_baseline"] = cpu_gemm_baseline(w_host, x_host, batch, rows, cols, cpu_budget_s)
    return res


def decode_bench(torch, hip, prefill, steps, cpu_budget_s):
    from mivi_hip.synthmodel import LFM2_1B2, build_hybrid, weight_bytes_per_token
    t0 = time.perf_counter()
    ctx = prefill + steps
    img = build_hybrid(**LFM2_1B2, ctx_len=65536, seed=2024)
    log(f"decode: model built ({img.nbytes / 1e6:.0f} MB) in {time.perf_counter() - t0:.1f}s")
    m = hip.Model(img, max_ctx=ctx, kv_precision=hip.KvPrecision.F16)
    rng = __import__("numpy").random.default_rng(11)
    prompt = rng.integers(0, LFM2_1B2["vocab"], prefill + 1)
    # prompt prefill: token by token once, then chunked (tiles of 512 rows,
    # PrefillStrategy::Chunked) warmed up and timed; the decode below runs
    # from the chunked prefill's state
    t1 = time.perf_counter()
    m.prefill(prompt[:-1])
    t_token = time.perf_counter() - t1
    m.generate_greedy([int(prompt[-1])], [prefill], 8)   # warm-up + graph capture (re-prefills below)
    m.reset_context()
    m.set_prefill_strategy(512)
    m.prefill(prompt[:-1])
    m.reset_context()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    m.prefill(prompt[:-1])
    t_chunked = time.perf_counter() - t1
    log(f"decode: prefill {prefill} tokens in {t_chunked * 1e3:.0f} ms chunked (tiles of 512), "
        f"{t_token:.2f} s token by token")
    state = m.export_state(prefill)
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    toks = m.generate_greedy([int(prompt[-1])], [prefill], steps)
    dt = time.perf_counter() - t2
    wb = weight_bytes_per_token(**LFM2_1B2)
    kv_per_tok = 2 * 6 * 512 * 2  # fp16 K+V bytes per cached token (6 attention layers)
    mean_t = prefill + (steps + 1) / 2
    out = dict(tok_s=steps / dt, ms_per_token=1e3 * dt / steps, prefill=prefill, steps=steps,
               prefill_tok_s=prefill / t_chunked, prefill_tile=512, prefill_token_path_tok_s=prefill / t_token,
               bytes_per_token=wb + kv_per_tok * mean_t, weight_bytes_per_token=wb, kv_precision="f16",
               working_ctx=ctx, first_tokens=[int(v) for v in toks[:8, 0]])
    out["gbs"] = out["bytes_per_token"] * out["tok_s"] / 1e9
    # the same steps from the same state with Sampler::sample on the device
    # (GenerationConfig::default: temperature 0.2, top-p 0.9, top-k 40,
    # repetition penalty 1.05) in place of the greedy argmax
    cfg = hip.SamplerConfig.make()
    m.import_state(prefill, *state)
    m.generate([int(prompt[-1])], [prefill], 4, cfg, [1])  # graph capture
    m.import_state(prefill, *state)
    torch.cuda.synchronize()
    t4 = time.perf_counter()
    stoks = m.generate([int(prompt[-1])], [prefill], steps, cfg, [1])
    ds = time.perf_counter() - t4
    out["sampled"] = dict(tok_s=steps / ds, ms_per_token=1e3 * ds / steps,
                          config="GenerationConfig::default (T 0.2, top-p 0.9, top-k 40, repetition 1.05), seed 1",
                          first_tokens=[int(v) for v in stoks[:8, 0]])
    log(f"decode: {steps / ds:.1f} tok/s with the device sampler (default GenerationConfig)")
    m.close()
    out["q4_k_m"] = mixed_decode_bench(torch, hip, prompt, prefill, steps, t_chunked)
    if cpu_budget_s > 0:
        out.update(decode_cpu_leg(img, state, prompt, prefill, steps, ctx, toks[:, 0], cpu_budget_s))
        out["speedup_vs_cpu"] = out["tok_s"] / out["cpu_tok_s"]
    return out


def config4_decode_only(torch, hip, prefill, steps):
    """Config 4's chunked prefill and greedy steps and nothing else, for
    counter and trace runs: every batch-1 attention launch of the run is then
    a decode step's (the token-path prefill launches the same grid)."""
    from mivi_hip.synthmodel import LFM2_1B2, build_hybrid
    img = build_hybrid(**LFM2_1B2, ctx_len=65536, seed=2024)
    m = hip.Model(img, max_ctx=prefill + steps, kv_precision=hip.KvPrecision.F16)
    prompt = __import__("numpy").random.default_rng(11).integers(0, LFM2_1B2["vocab"], prefill + 1)
    m.set_prefill_strategy(512)
    m.prefill(prompt[:-1])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    m.generate_greedy([int(prompt[-1])], [prefill], steps)
    dt = time.perf_counter() - t0
    m.close()
    return dict(tok_s=steps / dt, steps=steps, prefill=prefill)


def mixed_decode_bench(torch, hip, prompt, prefill, steps, q4k_prefill_s):
    """The same prompt and steps on the Q4_K_M layout of the 1.2B shape
    (8 ffn_down and 2 attn_v matrices in Q6_K, as the reference's 1.2B
    Q4_K_M file): chunked prefill time against the all-Q4_K model's, and
    greedy decode tok/s."""
    from mivi_hip.synthmodel import LFM2_1B2, build_hybrid, weight_bytes_per_token
    img = build_hybrid(**LFM2_1B2, ctx_len=65536, seed=2024, mixed="q4_k_m")
    m = hip.Model(img, max_ctx=prefill + steps, kv_precision=hip.KvPrecision.F16)
    m.set_prefill_strategy(512)
    m.prefill(prompt[:-1])
    m.generate_greedy([int(prompt[-1])], [prefill], 8)  # warm-up + graph capture
    m.reset_context()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    m.prefill(prompt[:-1])
    t_chunked = time.perf_counter() - t1
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    toks = m.generate_greedy([int(prompt[-1])], [prefill], steps)
    dt = time.perf_counter() - t2
    m.close()
    wb = weight_bytes_per_token(**LFM2_1B2, mixed="q4_k_m")
    log(f"decode Q4_K_M: prefill {prefill} tokens in {t_chunked * 1e3:.0f} ms "
        f"({t_chunked / q4k_prefill_s:.2f}x the Q4_K model), {steps / dt:.1f} tok/s")
    return dict(layout="Q4_K_M: ffn_down of layers 0,1,4,7,10,13,14,15 and attn_v of layers 8,15 in Q6_K",
                prefill_tok_s=prefill / t_chunked, prefill_time_vs_q4k=t_chunked / q4k_prefill_s,
                tok_s=steps / dt, weight_bytes_per_token=wb, first_tokens=[int(v) for v in toks[:8, 0]])


def oracle_import(o, k, v, conv, tokens, row, n_layers, f16):
    """State rows [n_layers, tokens, row] (the export layout) into the
    oracle's [n_layers, max_seq, row] caches (fp16 rows widened to f32)."""
    import numpy as np
    ok, ov = o.kv_views()
    per = ok.size // n_layers
    for l in range(n_layers):
        kk = k[l * tokens * row:(l + 1) * tokens * row]
        vv = v[l * tokens * row:(l + 1) * tokens * row]
        if f16:
            kk = kk.view(np.float16).astype(np.float32).view(np.uint8)
            vv = vv.view(np.float16).astype(np.float32).view(np.uint8)
        ok[l * per:l * per + kk.size] = kk
        ov[l * per:l * per + vv.size] = vv
    o.conv_view()[:] = conv


def oracle_greedy(pyoracle, o, tok, pos, n, budget_s):
    """Up to n greedy steps of the oracle (stops after budget_s); returns
    (tokens, seconds per step)."""
    toks, t0 = [], time.perf_counter()
    while len(toks) < n:
        tok = pyoracle.argmax(o.forward(tok, pos + len(toks)))
        toks.append(tok)
        if time.perf_counter() - t0 > budget_s:
            break
    return toks, (time.perf_counter() - t0) / max(1, len(toks))


def parity_record(got, want):
    """Token-by-token comparison of the device's greedy tokens with the
    oracle's over the steps the oracle ran."""
    n = len(want)
    div = next((i for i in range(n) if int(got[i]) != int(want[i])), None)
    return dict(steps_compared=n, tokens_equal=div is None, first_divergence=div)


def decode_cpu_leg(img, state, prompt, prefill, steps, ctx, gpu_toks, budget_s):
    """Config 4 on the CPU: the oracle's forward_step continuing greedily from
    the GPU-built state (the 4096-token prefill on the CPU would take minutes).
    Parity: all `steps` greedy tokens against the device's, with the oracle's
    attention heads spread over its threads (the same bits as one after
    another; not timed). Timed: the reference's own schedule, attention heads
    one after another (transformer.rs:128) and the projections over the
    threads, at the process's threads and at the reference default's 2, each
    within its budget."""
    pyoracle = _oracle()
    threads, vis = cpu_threads()
    k, v, conv = state
    out = {}
    pyoracle.set_threads(threads)
    o = pyoracle.Model(img, max_ctx=ctx, kv_precision=pyoracle.KV_F16RT)
    oracle_import(o, k, v, conv, prefill, 2 * 512, 6, True)
    toks, sec_par = oracle_greedy(pyoracle, o, int(prompt[-1]), prefill, steps, 10 * budget_s)
    o.close()
    out["parity"] = parity_record(gpu_toks, toks)
    pyoracle.set_serial_attention(True)
    try:
        for th, budget in ((threads, budget_s), (REF_THREADS, budget_s / 2)):
            pyoracle.set_threads(th)
            o = pyoracle.Model(img, max_ctx=ctx, kv_precision=pyoracle.KV_F16RT)
            oracle_import(o, k, v, conv, prefill, 2 * 512, 6, True)
            tt, sec = oracle_greedy(pyoracle, o, int(prompt[-1]), prefill, steps, budget)
            o.close()
            if th == threads:
                out.update(cpu_tok_s=1.0 / sec, cpu_threads=th, host_cpus_visible=vis,
                           cpu_sample=f"{len(tt)} greedy steps of the oracle forward_step after importing the "
                                      f"GPU-built state; attention heads one after another as transformer.rs:128, "
                                      f"projections over {th} threads",
                           cpu_tok_s_heads_over_threads=1.0 / sec_par)
            else:
                out["cpu_at_reference_default_threads"] = dict(tok_s=1.0 / sec, threads=th, steps=len(tt))
    finally:
        pyoracle.set_serial_attention(False)
    return out


def hbm_traffic():
    """HBM bytes per launch of the config-2 kernel from the committed counter
    profile (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, each scaled by the same
    counter on a kernel of known traffic); None when absent or when the kernel
    source changed since it was measured."""
    import hashlib
    path = os.path.join(ROOT, "profiles", "q6k_head_gemv_traffic.json")
    src = os.path.join(ROOT, "mivi-v4_amd", "csrc", "quant.hip")
    try:
        t = json.load(open(path))
        if t.get("quant_hip_sha256") != hashlib.sha256(open(src, "rb").read()).hexdigest():
            return None
        return t["fetch_kib"] * 1024 / t["fetch_factor"] + t["write_kib"] * 1024 / t["write_factor"]
    except (OSError, KeyError, ValueError):
        return None


def copy_calibration(torch, mib, reps):
    """Kernels of known HBM traffic for scaling the counters: a fill (writes
    `mib` MiB), plain copies (read + write `mib` MiB each) and full reductions
    (read `mib` MiB each)."""
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    for _ in range(reps):
        src.sum()
    torch.cuda.synchronize()
    log(f"counter calibration: fill, {reps} copies and {reps} reductions of {n * 4} bytes")


def config5_weight_bytes(cfg, batch):
    """Weight bytes one batched step streams with the current column grouping:
    the d = 2048 Q4_K projections take all the batch's columns (up to 8) in one
    launch and read their weights once; the K = 8192 FFN down runs groups of
    four columns side by side, each reading the matrix; the packed Q6_K head
    takes up to eight columns per launch and reads each row quad once."""
    from mivi_hip.synthmodel import weight_bytes_per_token
    wb = weight_bytes_per_token(**cfg)
    down = cfg["n_layers"] * cfg["dim"] * cfg["hidden"] // 256 * 144
    head = cfg["vocab"] * cfg["dim"] // 256 * 210
    rest = wb - down - head
    return rest * -(-batch // 8) + down * -(-batch // 4) + head * -(-batch // 8)


def batched_decode_bench(torch, hip, batch, ctx, steps, cpu_budget_s=0.0):
    """Config 5: 8 sequences, each a seeded uniform-random prompt of `ctx`
    tokens prefilled in tiles of 512 rows (PrefillStrategy::Chunked) into its
    own Q8_0 cache and ShortConv state, then `steps` greedy steps of the 8
    together (one batched decode step per position), timed."""
    import numpy as np
    from mivi_hip.synthmodel import LFM2_1B2, build_hybrid
    img = build_hybrid(**LFM2_1B2, ctx_len=65536, seed=2024)
    m = hip.Model(img, max_ctx=ctx + steps, kv_precision=hip.KvPrecision.Q8_0, max_batch=batch)
    info = m.info
    m.set_prefill_strategy(512)
    prompts = np.random.default_rng(12).integers(0, LFM2_1B2["vocab"], (batch, ctx + 1))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for b in range(batch):
        m.prefill(prompts[b, :-1], 0, seq=b)
    torch.cuda.synchronize()
    t_pf = time.perf_counter() - t0
    log(f"config 5: {batch} prompts of {ctx} tokens prefilled in {t_pf:.1f} s (tiles of 512)")
    states = [m.export_state(ctx, seq=b) for b in range(batch)]
    toks = [int(prompts[b, -1]) for b in range(batch)]
    m.generate_greedy(toks, [ctx] * batch, 4)  # graph capture; rewrites positions ctx.. below
    # the warm-up advanced each sequence's ShortConv state: back to the
    # prefilled one (an interval import of no rows with the state)
    empty = np.empty(0, np.uint8)
    for b in range(batch):
        m.import_state_at(0, 0, empty, empty, states[b][2], seq=b)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    out = m.generate_greedy(toks, [ctx] * batch, steps)
    dt = time.perf_counter() - t1
    kv_row = info.kv_dim // 32 * 34
    mean_t = ctx + (steps + 1) / 2
    kv_bytes = batch * info.n_attn_layers * 2 * kv_row * mean_t
    wbs = config5_weight_bytes(LFM2_1B2, batch)
    res = dict(batch=batch, cached_tokens=ctx, steps=steps, kv_precision="q8_0", tok_s=batch * steps / dt,
               ms_per_step=1e3 * dt / steps, kv_bytes_per_step=kv_bytes,
               kv_gbs_over_whole_step=kv_bytes * steps / dt / 1e9, weight_bytes_per_step=wbs,
               gbs_whole_step=(kv_bytes + wbs) * steps / dt / 1e9,
               prefill_tok_s=batch * ctx / t_pf, prefill_tile=512,
               note=("caches and ShortConv states built by the chunked prefill of seeded uniform token ids; "
                     "weight_bytes_per_step: the d = 2048 projections read their weights once for the 8 columns, "
                     "the K = 8192 FFN down once per group of four columns, the packed head once per eight; "
                     "kv_gbs_over_whole_step divides the KV bytes by the whole step time, not the attention "
                     "kernels' time"),
               first_tokens=[int(v) for v in out[:4, 0]])
    m.close()
    if cpu_budget_s > 0:
        res.update(config5_cpu_leg(img, states, toks, ctx, steps, out, cpu_budget_s))
        res["speedup_vs_cpu"] = res["tok_s"] / res["cpu_tok_s"]
    return res


def config5_cpu_leg(img, states, toks, ctx, steps, gpu_out, budget_s, parity_steps=16):
    """Config 5 on the CPU, from each sequence's GPU-built state (the reference
    runs one Model per sequence). Parity: `parity_steps` greedy steps of every
    sequence against the device's batched tokens (attention heads over the
    threads, not timed). Timed: single-sequence decodes with the reference's
    schedule (attention heads one after another, transformer.rs:128) within
    the budget, at the process's threads and at the reference default's 2."""
    pyoracle = _oracle()
    threads, vis = cpu_threads()
    batch = len(toks)
    pyoracle.set_threads(threads)
    o = pyoracle.Model(img, max_ctx=ctx + steps, kv_precision=pyoracle.KV_Q8_0)
    row = o.info.kv_dim // 32 * 34
    par = []
    for b in range(batch):
        o.reset()
        oracle_import(o, *states[b], ctx, row, 6, False)
        got, _ = oracle_greedy(pyoracle, o, toks[b], ctx, min(steps, parity_steps), 10 * budget_s)
        par.append(parity_record(gpu_out[:, b], got))
    res = dict(parity=dict(steps_compared=sum(p["steps_compared"] for p in par),
                           tokens_equal=all(p["tokens_equal"] for p in par),
                           per_sequence_first_divergence=[p["first_divergence"] for p in par]))
    pyoracle.set_serial_attention(True)
    try:
        for th, budget in ((threads, budget_s), (REF_THREADS, budget_s / 2)):
            pyoracle.set_threads(th)
            secs, n_steps, b = 0.0, 0, 0
            while secs < budget and b < batch:
                o.reset()
                oracle_import(o, *states[b], ctx, row, 6, False)
                got, sec = oracle_greedy(pyoracle, o, toks[b], ctx, steps, budget - secs)
                secs += sec * len(got)
                n_steps += len(got)
                b += 1
            if th == threads:
                res.update(cpu_tok_s=n_steps / secs, cpu_threads=th, host_cpus_visible=vis,
                           cpu_sample=f"{n_steps} oracle forward_step calls over {b} sequence(s) at {ctx}+ cached "
                                      f"tokens from the GPU-built states; attention heads one after another as "
                                      f"transformer.rs:128, projections over {th} threads")
            else:
                res["cpu_at_reference_default_threads"] = dict(tok_s=n_steps / secs, threads=th, steps=n_steps)
    finally:
        pyoracle.set_serial_attention(False)
    o.close()
    return res


def sampler_bench(torch, hip, calls):
    """Sampler::sample on one row of 65536 logits (N(0, 9), a 64-token penalty
    window), µs per call between HIP events on the stream the calls run on:
    GenerationConfig::default on the split path (chunk kernel + pick kernel
    over the top-k candidates), and full-vocabulary categorical sampling
    (temperature 1, no top-k / top-p: chunk, exp, probability and pick
    kernels)."""
    n = 65536
    g = torch.Generator(device="cuda").manual_seed(5)
    base = torch.randn(n, device="cuda", generator=g) * 3
    rec = torch.randint(0, n, (1, 64), dtype=torch.int32, device="cuda", generator=g)
    rng = torch.tensor([1], dtype=torch.int64, device="cuda")
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = {"n": n, "calls": calls}
    for name, cfg in (("default_config_us", hip.SamplerConfig.make()),
                      ("categorical_us",
                       hip.SamplerConfig.make(temperature=1.0, top_p=1.0, top_k=0, repetition_penalty=1.0))):
        fn = lambda l: hip.sample(l, rec[0], cfg, rng, tok)  # noqa: E731
        rows = [base.clone() for _ in range(calls)]
        fn(base.clone())
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for l in rows:
            fn(l)
        e1.record()
        torch.cuda.synchronize()
        out[name] = e0.elapsed_time(e1) * 1e3 / calls
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--decode-prefill", type=int, default=4096)
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--only-q6k", action="store_true", help="config 2 only (counter runs)")
    ap.add_argument("--only-gemm", action="store_true", help="config 3 only (counter runs)")
    ap.add_argument("--only-config5", action="store_true", help="config 5 only (counter runs)")
    ap.add_argument("--only-config4", action="store_true",
                    help="config 4 chunked prefill + greedy decode only (counter runs)")
    ap.add_argument("--no-config5", action="store_true")
    ap.add_argument("--config5-ctx", type=int, default=32768)
    ap.add_argument("--config5-steps", type=int, default=128)
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="also run plain copies of MIB MiB (counter calibration)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the GEMV and decode would shard by rows / sequences without exchange)", file=sys.stderr)
        sys.exit(2)
    import torch
    import mivi_hip as hip
    torch.cuda.set_device(0)
    log(f"{hip.version()} on {torch.cuda.get_device_name(0)}")

    if a.only_gemm:
        g3 = gemm_bench(torch, hip, max(5, a.steps // 10), 3)
        log(f"Q4_K GEMM 512x8192x2048: {g3['ms_per_call'] * 1e3:.1f} us/call, {g3['tflops']:.0f} TFLOP/s "
            f"(GGUF rows staged per call {g3['gguf_rows']['ms_per_call'] * 1e3:.1f} us)")
        return
    if a.only_config4:
        c4 = config4_decode_only(torch, hip, a.decode_prefill, a.decode_steps)
        log(f"config 4: {c4['tok_s']:.1f} tok/s over {c4['steps']} greedy steps (graph capture included)")
        return
    if a.only_config5:
        c5 = batched_decode_bench(torch, hip, 8, a.config5_ctx, a.config5_steps)
        log(f"config 5: {c5['tok_s']:.0f} tok/s over 8 sequences, {c5['ms_per_step']:.2f} ms per step")
        return
    q6 = gemv_bench(torch, hip, hip.GgmlType.Q6_K, 65536, 2048, a.steps, a.warmup, 100, packed=True)
    log(f"Q6_K GEMV 65536x2048 (packed rows): {q6['ms_per_call'] * 1e3:.1f} us/call, {q6['gbs']:.0f} GB/s; "
        f"plain read of the same bytes {q6['read_floor_us']:.1f} us")
    q6r = gemv_bench(torch, hip, hip.GgmlType.Q6_K, 65536, 2048, a.steps, a.warmup, 100)
    log(f"Q6_K GEMV 65536x2048 (GGUF rows): {q6r['ms_per_call'] * 1e3:.1f} us/call, {q6r['gbs']:.0f} GB/s")
    if a.copy_calib:
        copy_calibration(torch, a.copy_calib, 10)
    if a.only_q6k:
        return
    q4 = gemv_bench(torch, hip, hip.GgmlType.Q4_K, 8192, 2048, a.steps * 4, a.warmup, 200)
    log(f"Q4_K GEMV 8192x2048 (GGUF rows): {q4['ms_per_call'] * 1e3:.2f} us/call, {q4['gbs']:.0f} GB/s "
        f"({q4['host_loop_ms_per_call'] * 1e3:.2f} us issued from Python); "
        f"plain read of the same bytes {q4['read_floor_us']:.2f} us")
    q4p = gemv_bench(torch, hip, hip.GgmlType.Q4_K, 8192, 2048, a.steps * 4, a.warmup, 200, packed=True)
    log(f"Q4_K GEMV 8192x2048 (packed row quads): {q4p['ms_per_call'] * 1e3:.2f} us/call, {q4p['gbs']:.0f} GB/s "
        f"({q4p['host_loop_ms_per_call'] * 1e3:.2f} us issued from Python)")
    cpu = None
    if not a.no_cpu:
        cpu = cpu_gemv_baseline(hip.GgmlType.Q6_K, q6["w_host"], q6["x_host"], 65536, 2048, a.cpu_seconds)
        log(f"CPU oracle Q6_K GEMV: {cpu['value']:.2f} GB/s on {cpu['cores']} threads")
    extra = {
        "q6k_gemv_config2_gguf_rows": {k: q6r[k] for k in ("ms_per_call", "host_loop_ms_per_call", "gbs")},
        "q4k_gemv_config1": {k: q4[k] for k in ("rows", "cols", "algo_bytes", "ms_per_call", "host_loop_ms_per_call",
                                                "gbs", "copies", "read_floor_us", "frac_of_read_floor")},
        "q6k_gemv_config2_read_floor": {"read_floor_us": q6["read_floor_us"],
                                        "read_floor_gbs": q6["weight_bytes"] / q6["read_floor_us"] / 1e3,
                                        "packed_frac_of_read_floor": q6["frac_of_read_floor"]},
    }
    extra["q6k_gemv_config2_gguf_rows"]["frac_of_peak"] = q6r["gbs"] / HBM_PEAK_GBS
    extra["q4k_gemv_config1"]["frac_of_peak"] = q4["gbs"] / HBM_PEAK_GBS
    # the same matrix packed once into row quads (mivi_hip_pack_weights, not
    # timed; the model's one-column decode GEMVs read this layout)
    extra["q4k_gemv_config1_packed"] = {k: q4p[k] for k in ("ms_per_call", "host_loop_ms_per_call", "gbs",
                                                            "read_floor_us", "frac_of_read_floor")}
    extra["q4k_gemv_config1_packed"]["frac_of_peak"] = q4p["gbs"] / HBM_PEAK_GBS
    extra["q4k_gemv_config1_packed"]["weight_layout"] = "packed row quads (matrix cores; bit-identical to GGUF rows)"
    if not a.no_cpu:
        extra["q4k_gemv_config1"]["cpu_baseline"] = cpu_gemv_baseline(hip.GgmlType.Q4_K, q4["w_host"], q4["x_host"],
                                                                       8192, 2048, a.cpu_seconds / 2)
    g3 = gemm_bench(torch, hip, max(5, a.steps // 10), 3, 0 if a.no_cpu else a.cpu_seconds / 2)
    log(f"Q4_K GEMM 512x8192x2048: {g3['ms_per_call'] * 1e3:.1f} us/call, {g3['tflops']:.0f} TFLOP/s "
        f"(GGUF rows staged per call {g3['gguf_rows']['ms_per_call'] * 1e3:.1f} us)")
    extra["q4k_gemm_config3"] = g3
    if not a.no_decode:
        dec = decode_bench(torch, hip, a.decode_prefill, a.decode_steps, 0 if a.no_cpu else a.cpu_seconds)
        log(f"decode: {dec['tok_s']:.1f} tok/s ({dec['gbs']:.0f} GB/s)"
            + (f", CPU {dec['cpu_tok_s']:.2f} tok/s" if "cpu_tok_s" in dec else ""))
        extra["decode_config4"] = dec
        sm = sampler_bench(torch, hip, 50)
        log(f"sampler (65536 logits): {sm['default_config_us']:.1f} us default config (split path), "
            f"{sm['categorical_us']:.1f} us full-vocabulary categorical")
        extra["sampler"] = sm
    if not a.no_decode and not a.no_config5:
        c5 = batched_decode_bench(torch, hip, 8, a.config5_ctx, a.config5_steps, 0 if a.no_cpu else a.cpu_seconds)
        log(f"config 5: {c5['tok_s']:.0f} tok/s over 8 sequences, {c5['ms_per_step']:.2f} ms per step")
        extra["decode_config5"] = c5
    line = {
        "metric": METRIC,
        "value": round(q6["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": q6["ms_per_call"],
        "host_loop_ms_per_step": q6["host_loop_ms_per_call"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        # x enters the GEMV as three int8 digit planes against one scale per
        # launch; codes x digits accumulate exactly in int32 (matrix cores),
        # sub-block scales and the output are f32
        "dtype": "i8x3 digit planes x 6-bit codes -> i32, f32 scales and output",
        "data": "synthetic (seeded N(0,0.02) weights quantized to Q6_K by this build's encoder; x ~ N(0,1))",
        "config": {"workload": "config2_q6k_head_gemv", "rows": 65536, "cols": 2048, "weight_type": "Q6_K",
                   "weight_layout": "packed row quads (mivi_hip_pack_weights, done once, not timed)",
                   "weight_copies": q6["copies"], "algo_bytes_per_call": q6["algo_bytes"]},
        "roofline": {"bound": "hbm", "achieved": round(q6["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(q6["gbs"] / HBM_PEAK_GBS, 4), "traffic": hbm_traffic()},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
