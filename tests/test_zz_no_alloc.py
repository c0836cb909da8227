"""vm_gated_attn_decode_noalloc against vm_gated_attn_decode (GPU, through the C ABI).

The no-allocation entry point runs the same decode step with its workspace in
the library's static per-GPU array. Two calls in a row, the second on a smaller
input (the array keeps the first call's contents), each compared with the
existing entry point on copies of the same inputs: the outputs and the appended
cache rows are bit-identical (same kernels, same partition), and both meet the
parity bar against the CPU oracle.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from conftest import (D, EPS, HALF, THETA, TOL_MAX, TOL_MEAN, banner, dev_f32, from_dev, i32,
                      maxmean, to_dev)
from oracle.rng import normal_bf16

pytestmark = pytest.mark.gpu

HQ, HK = 16, 4
S = 2 * HQ + 2 * HK


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _step(vm, entry, B, ctx, pos, seed, ws=None):
    lib = vm._lib.load()
    qw = to_dev(normal_bf16((D,), seed + 1, scale=0.05))
    kw = to_dev(normal_bf16((D,), seed + 2, scale=0.05))
    K = to_dev(normal_bf16((B, HK, ctx, D), seed + 3))
    V = to_dev(normal_bf16((B, HK, ctx, D), seed + 4))
    qkv = to_dev(normal_bf16((B, S, D), seed + 5))
    cos = torch.empty((ctx, HALF), dtype=torch.float32, device="cuda")
    sin = torch.empty_like(cos)
    vm._lib.call("vm_rope_tables", _p(cos), _p(sin), HALF, ctx, THETA, None)
    positions = i32(pos)
    out = torch.empty((B, HQ, D), dtype=torch.bfloat16, device="cuda")
    args = [_p(out), HQ * D, _p(qkv), S * D, _p(K), _p(V), D, ctx * D, HK * ctx * D, ctx,
            _p(qw), _p(kw), _p(cos), _p(sin), _p(positions), 1, B, HQ, HK, D, HALF, EPS, 1.0, 0]
    if entry == "vm_gated_attn_decode":
        args += [_p(ws), ws.numel()]
    vm._lib.call(entry, *args, None)
    torch.cuda.synchronize()
    return out, K, V, positions, (qkv, qw, kw)


def _compare(vm, orc, B, ctx, pos, seed):
    lib = vm._lib.load()
    need = lib.vm_decode_scratch_bytes(B, HQ, HK, D, ctx, 0)
    assert 0 < need <= (16 << 20)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    banner(f"no-alloc decode B={B} ctx={ctx}: existing entry point")
    o1, K1, V1, p1, _ = _step(vm, "vm_gated_attn_decode", B, ctx, pos, seed, ws)
    banner(f"no-alloc decode B={B} ctx={ctx}: vm_gated_attn_decode_noalloc")
    o2, K2, V2, p2, (qkv, qw, kw) = _step(vm, "vm_gated_attn_decode_noalloc", B, ctx, pos, seed)
    assert torch.equal(o1, o2)
    assert torch.equal(K1, K2) and torch.equal(V1, V2)
    assert torch.equal(p1, p2) and np.array_equal(p2.cpu().numpy(), np.asarray(pos) + 1)
    kc0 = normal_bf16((B, HK, ctx, D), seed + 3)
    vc0 = normal_bf16((B, HK, ctx, D), seed + 4)
    c, s = orc.rope_tables(HALF, ctx, THETA)
    ref, _, _ = orc.gated_decode(from_dev(qkv), kc0, vc0, np.asarray(pos, np.int32), from_dev(qw),
                                 from_dev(kw), c, s, Hq=HQ, Hk=HK, eps=EPS, w_offset=1.0)
    mx, mn = maxmean(dev_f32(o2), ref)
    print(f"no-alloc B={B}: out max {mx:.3e} mean {mn:.3e}")
    assert mx <= TOL_MAX and mn <= TOL_MEAN


def test_noalloc_decode_matches_existing_entry_point(vm, orc):
    """Two calls in a row, the second smaller than the first."""
    _compare(vm, orc, 8, 4096, [4096, 1, 77, 2048, 3000, 129, 4000, 512], 900)
    _compare(vm, orc, 2, 1024, [1024, 300], 910)
