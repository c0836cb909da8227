"""Row kernels on the GPU vs the oracle: RoPE tables (a1), qnorm_rope! (a3),
knorm_rope_append! (a4), the sigmoid gate (a6), the device clock (a12) and the
synthetic-input generator."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import (D, EPS, HALF, HK, HQ, S, THETA, TOL_MAX, TOL_MEAN, banner, dev_f32,
                      from_dev, i32, maxmean, to_dev)
from oracle.rng import bf16_to_f32, normal_bf16

pytestmark = pytest.mark.gpu


class Cfg:
    rot_half, theta, Ctx = HALF, THETA, 131328


def test_rope_tables_match_oracle(vm, orc):
    banner("rope_tables ctx=131328")
    t = vm.rope_tables(Cfg)
    c, s = orc.rope_tables(HALF, Cfg.Ctx, THETA)
    assert np.max(np.abs(t["cos"].cpu().numpy() - c)) <= 1.2e-7
    assert np.max(np.abs(t["sin"].cpu().numpy() - s)) <= 1.2e-7


def test_fill_normal_matches_host_stream(vm):
    banner("fill_normal n=1_000_001")
    x = torch.empty(1_000_001, dtype=torch.bfloat16, device="cuda")
    vm.fill_normal_(x, 1234)
    assert np.array_equal(from_dev(x), normal_bf16((1_000_001,), 1234))
    y = torch.empty(4097, dtype=torch.bfloat16, device="cuda")
    vm.fill_normal_(y, 99, scale=0.05)
    assert np.array_equal(from_dev(y), normal_bf16((4097,), 99, scale=0.05))


def test_qnorm_rope_in_place_strided(vm, orc):
    banner("qnorm_rope_ B=3 strided q view")
    B, ctx = 3, 600
    qkv_bits = normal_bf16((B, S, D), 7)
    qw = normal_bf16((D,), 8, scale=0.05)
    pos = np.array([1, 257, 600], np.int32)
    tabs = vm.rope_tables(type("C", (), {"rot_half": HALF, "theta": THETA, "Ctx": ctx}))
    qkv = to_dev(qkv_bits)
    q = qkv[:, 0:2 * HQ:2, :]
    vm.qnorm_rope_(q, to_dev(qw), tabs["cos"], tabs["sin"], positions=i32(pos), eps=EPS, offset=1.0)
    torch.cuda.synchronize()
    got = dev_f32(qkv)
    c, s = orc.rope_tables(HALF, ctx, THETA)
    ref = np.stack([np.stack([orc.head_norm_rope(bf16_to_f32(qkv_bits[b, 2 * h]),
                                                 bf16_to_f32(qw), EPS, 1.0, c, s, pos[b] - 1)
                              for h in range(HQ)]) for b in range(B)])
    mx, mn = maxmean(got[:, 0:2 * HQ:2], ref)
    assert mx <= TOL_MAX and mn <= TOL_MEAN
    # gate / k / v slots untouched
    assert np.array_equal(from_dev(qkv)[:, 1::2][:, :HQ], qkv_bits[:, 1:2 * HQ:2])
    assert np.array_equal(from_dev(qkv)[:, 2 * HQ:], qkv_bits[:, 2 * HQ:])


def test_knorm_rope_append_writes_one_column(vm, orc):
    banner("knorm_rope_append_ B=2")
    B, ctx = 2, 300
    qkv_bits = normal_bf16((B, S, D), 17)
    kw = normal_bf16((D,), 18, scale=0.05)
    kc_bits = normal_bf16((B, HK, ctx, D), 19)
    vc_bits = normal_bf16((B, HK, ctx, D), 20)
    pos = np.array([300, 45], np.int32)
    tabs = vm.rope_tables(type("C", (), {"rot_half": HALF, "theta": THETA, "Ctx": ctx}))
    qkv, kc, vc = to_dev(qkv_bits), to_dev(kc_bits), to_dev(vc_bits)
    k = qkv[:, 2 * HQ:2 * HQ + HK]
    v = qkv[:, 2 * HQ + HK:]
    vm.knorm_rope_append_(kc, vc, k, v, to_dev(kw), tabs["cos"], tabs["sin"],
                          positions=i32(pos), eps=EPS, offset=1.0)
    torch.cuda.synchronize()
    c, s = orc.rope_tables(HALF, ctx, THETA)
    kg, vg = from_dev(kc), from_dev(vc)
    for b in range(B):
        col = pos[b] - 1
        for j in range(HK):
            ref = orc.head_norm_rope(bf16_to_f32(qkv_bits[b, 2 * HQ + j]), bf16_to_f32(kw), EPS,
                                     1.0, c, s, col)
            mx, mn = maxmean(bf16_to_f32(kg[b, j, col]), ref)
            assert mx <= TOL_MAX and mn <= TOL_MEAN
            assert np.array_equal(vg[b, j, col], qkv_bits[b, 2 * HQ + HK + j])
        others = np.ones(ctx, bool)
        others[col] = False
        assert np.array_equal(kg[b][:, others], kc_bits[b][:, others])
        assert np.array_equal(vg[b][:, others], vc_bits[b][:, others])


def test_sigmoid_gate(vm):
    banner("sigmoid_gate_ B=4")
    B = 4
    qkv_bits = normal_bf16((B, S, D), 27)
    o_bits = normal_bf16((B, HQ, D), 28)
    qkv, o = to_dev(qkv_bits), to_dev(o_bits)
    vm.sigmoid_gate_(o, qkv[:, 1:2 * HQ:2])
    torch.cuda.synchronize()
    ref = bf16_to_f32(o_bits) / (1 + np.exp(-bf16_to_f32(qkv_bits[:, 1:2 * HQ:2]).astype(np.float64)))
    mx, mn = maxmean(dev_f32(o), ref)
    assert mx <= 1e-2 and mn <= 1e-3


def test_advance_positions(vm):
    banner("advance")
    gen = vm.Generation(5)
    gen.positions.copy_(i32([1, 2, 3, 4, 5]))
    gen.advance_().advance_()
    assert gen.positions.cpu().tolist() == [3, 4, 5, 6, 7]
