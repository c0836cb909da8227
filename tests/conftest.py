"""Shared fixtures. GPU tests are marked ``gpu``; everything else runs on CPU."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

# Qwen3.5 attention facts used throughout (src/llm/qwen35.jl:15-23)
HQ, HK, D, HALF, THETA, EPS = 16, 4, 256, 32, 1.0e7, 1.0e-6
S = 2 * HQ + 2 * HK
TOL_MAX, TOL_MEAN = 2e-2, 2e-3   # north-star parity bar on bf16 outputs


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def vm():
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle


def maxmean(a, b):
    d = np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))
    return float(d.max()), float(d.mean())


# ---- GPU helpers (torch is only device-memory plumbing) ---------------------
def to_dev(bits):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(torch.bfloat16)


def from_dev(t):
    import torch
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def dev_f32(t):
    from oracle.rng import bf16_to_f32
    return bf16_to_f32(from_dev(t)).reshape(tuple(t.shape))


def i32(a):
    import torch
    return torch.as_tensor(np.asarray(a, np.int32)).cuda()


def banner(msg):
    """Name the case before each GPU step so a failure is attributable."""
    print(f"[case] {msg}", flush=True)
