"""Shared test setup: repo paths on sys.path, the `gpu` marker, helpers."""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "mivi-v4_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


@pytest.fixture(scope="session")
def oracle():
    import pyoracle
    pyoracle.build()
    pyoracle.set_threads(min(8, os.cpu_count() or 1))
    return pyoracle


@pytest.fixture(scope="session")
def hip():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    import mivi_hip
    return mivi_hip


@pytest.fixture(scope="session")
def torch_mod():
    import torch
    return torch


def import_into_oracle(o, k, v, conv, tokens, row, n_layers, f16=False):
    """A state exported by the device (rows [n_layers, tokens, row], the
    export layout) into the oracle's [n_layers, max_seq, row] caches and its
    ShortConv state; fp16 rows widen to the oracle's f32 cache."""
    import numpy as np
    ok, ov = o.kv_views()
    per = ok.size // n_layers
    orow = row * 2 if f16 else row
    for l in range(n_layers):
        src = slice(l * tokens * row, (l + 1) * tokens * row)
        kk, vv = k[src], v[src]
        if f16:
            kk = kk.view(np.float16).astype(np.float32).view(np.uint8)
            vv = vv.view(np.float16).astype(np.float32).view(np.uint8)
        ok[l * per: l * per + tokens * orow] = kk
        ov[l * per: l * per + tokens * orow] = vv
    o.conv_view()[:] = conv


def q8_rows_close(a, b, tokens, n_layers, row, max_frac=0.05):
    """Two Q8_0 caches (rows of 34-byte blocks) built by different float
    arithmetic: every int8 code within one step of the other's, fewer than
    max_frac of them different, block scales within 5e-3 relative. (The
    oracle's AVX2 and scalar kernels, both the reference's, give caches 1.5 %
    of whose codes differ by one step and whose f16 scales differ by up to
    1.5e-3 on a 120-token QK-norm prompt.)"""
    import numpy as np
    blk = a[:n_layers * tokens * row].reshape(-1, 34)
    blb = b[:n_layers * tokens * row].reshape(-1, 34)
    qa = blk[:, 2:].view(np.int8).astype(np.int32)
    qb = blb[:, 2:].view(np.int8).astype(np.int32)
    da = blk[:, :2].copy().view(np.float16).astype(np.float64).ravel()
    db = blb[:, :2].copy().view(np.float16).astype(np.float64).ravel()
    return (np.max(np.abs(qa - qb)) <= 1 and np.mean(qa != qb) < max_frac
            and np.all(np.abs(da - db) <= 5e-3 * np.maximum(np.abs(da), 1e-30)))
