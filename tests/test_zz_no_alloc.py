"""mivi_hip_sample_noalloc (the sampler with the library's fixed device scratch
in place of an allocated workspace) against mivi_hip_sample on the same
logits, penalty window and generator state, through the C ABI: the token, the
generator state and the probabilities (or penalised logits) left in the row
must be identical bit for bit, since both run the same kernels. Two calls in a
row per configuration, the second on a smaller row, so the second call runs
over scratch the first left behind; sizes beyond the scratch are refused
before anything runs.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CONFIGS = {
    "default": dict(),
    "categorical_min_p": dict(temperature=0.9, top_p=1.0, top_k=0, min_p=0.1, presence_penalty=0.4,
                              frequency_penalty=0.2),
    "greedy_penalised": dict(temperature=0.0, presence_penalty=0.5, frequency_penalty=0.25),
    "nucleus": dict(temperature=0.8, top_p=0.95, top_k=0),
}


def call(fn, torch, logits, recent, cfg, state):
    """One call of fn (an entry point of the library) on copies of the inputs;
    returns (token, state after, row after)."""
    row = logits.clone()
    rng = torch.tensor([state], dtype=torch.int64, device="cuda")
    tok = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()
    rc = fn(C.c_void_p(row.data_ptr()), row.numel(), C.c_void_p(recent.data_ptr()), recent.numel(), C.byref(cfg),
            C.c_void_p(rng.data_ptr()), C.c_void_p(tok.data_ptr()), C.c_void_p(stream.cuda_stream))
    assert rc == 0
    torch.cuda.synchronize()
    return int(tok.item()), int(rng.item()), row.cpu().numpy()


@pytest.mark.parametrize("name", list(CONFIGS))
def test_noalloc_sample_matches_sample(hip, torch_mod, name):
    torch = torch_mod
    lib = hip.lib()
    cfg = hip.SamplerConfig.make(**CONFIGS[name])
    g = torch.Generator(device="cuda").manual_seed(31)
    for n, seed in ((65536, 12345), (4099, 777)):  # second call smaller, ragged last chunk
        logits = torch.randn(n, device="cuda", generator=g) * 3
        recent = torch.randint(0, n, (64,), dtype=torch.int32, device="cuda", generator=g)
        want = call(lib.mivi_hip_sample, torch, logits, recent, cfg, seed)
        got = call(lib.mivi_hip_sample_noalloc, torch, logits, recent, cfg, seed)
        assert got[0] == want[0] and 0 <= got[0] < n, (name, n)
        assert got[1] == want[1], (name, n)
        assert np.array_equal(got[2].view(np.uint32), want[2].view(np.uint32)), (name, n)


def test_noalloc_sample_refuses_rows_beyond_its_scratch(hip, torch_mod):
    torch = torch_mod
    lib = hip.lib()
    n = 262144 + 1
    logits = torch.zeros(n, device="cuda")
    before = logits.clone()
    rng = torch.tensor([1], dtype=torch.int64, device="cuda")
    tok = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    cfg = hip.SamplerConfig.make()
    rc = lib.mivi_hip_sample_noalloc(C.c_void_p(logits.data_ptr()), n, None, 0, C.byref(cfg),
                                     C.c_void_p(rng.data_ptr()), C.c_void_p(tok.data_ptr()), None)
    assert rc == 101 and "262144" in hip.last_error().message.decode()
    torch.cuda.synchronize()
    assert torch.equal(logits, before) and int(tok.item()) == -1 and int(rng.item()) == 1
