"""Decode path on the GPU vs the oracle: decode!(::AttnLayer) fused step (a7 =
a3+a4+a5+a6), decode_attention! (a5) alone, split-count invariance, GQA group
sizes, ragged/edge lengths, BASELINE config 1 and config 3 at full size (sampled
sequences against the oracle), and config 4 as a hipGraph replayed with the
position advancing on the device (replays == eager steps, bit for bit)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import (D, EPS, HALF, HK, HQ, S, THETA, TOL_MAX, TOL_MEAN, banner, dev_f32,
                      from_dev, i32, maxmean, to_dev)
from oracle.rng import bf16_to_f32, f32_to_bf16, normal_bf16

pytestmark = pytest.mark.gpu


def make_layer(vm, B, ctx, Hq=HQ, Hk=HK, seed=0, n_splits=0, caches=None, kw_big=None):
    cfg = vm.AttnConfig(Hq=Hq, Hkv=Hk, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=ctx, B=B)
    qw = normal_bf16((D,), seed + 1, scale=0.05)
    kw = normal_bf16((D,), seed + 2, scale=0.05)
    if kw_big is not None:
        kw[0] = f32_to_bf16(np.array([kw_big], np.float32))[0]
    if caches is None:
        kc = normal_bf16((B, Hk, ctx, D), seed + 3)
        vc = normal_bf16((B, Hk, ctx, D), seed + 4)
        K, V = to_dev(kc), to_dev(vc)
    else:
        K, V = caches
    m = vm.AttnModel(cfg, n_splits=n_splits)
    layer = vm.AttnLayer(qw=to_dev(qw), kw=to_dev(kw), K_cache=K, V_cache=V)
    return cfg, m, layer, qw, kw


def run_decode_vs_oracle(vm, orc, B, ctx, pos, Hq=HQ, Hk=HK, seed=0, n_splits=0, kw_big=None):
    S_ = 2 * Hq + 2 * Hk
    cfg, m, layer, qw, kw = make_layer(vm, B, ctx, Hq, Hk, seed, n_splits, kw_big=kw_big)
    kc, vc = from_dev(layer.K_cache), from_dev(layer.V_cache)
    qkv = normal_bf16((B, S_, D), seed + 5)
    gen = vm.Generation(B)
    gen.positions.copy_(i32(pos))
    O = torch.empty((B, Hq, D), dtype=torch.bfloat16, device="cuda")
    vm.gated_attn_decode_(O, layer, m, gen, to_dev(qkv))
    torch.cuda.synchronize()
    c, s = orc.rope_tables(HALF, ctx, THETA)
    ref, kn, vn = orc.gated_decode(qkv, kc, vc, np.asarray(pos, np.int32), qw, kw, c, s, Hq=Hq,
                                   Hk=Hk, eps=EPS, w_offset=1.0)
    got = dev_f32(O)
    mx, mn = maxmean(got, ref)
    kg, vg = from_dev(layer.K_cache), from_dev(layer.V_cache)
    cols = np.asarray(pos) - 1
    live = [b for b in range(B) if cols[b] >= 0]   # position 0: no token appended
    kmx, kmn = (maxmean(np.stack([bf16_to_f32(kg[b, :, cols[b]]) for b in live]), kn[live])
                if live else (0.0, 0.0))
    vexact = all(np.array_equal(bf16_to_f32(vg[b, :, cols[b]]), vn[b]) for b in live)
    vexact &= all(np.array_equal(kg[b], kc[b]) and np.array_equal(vg[b], vc[b])
                  for b in range(B) if cols[b] < 0)
    return (mx, mn), (kmx, kmn), vexact, got, ref


def test_config1_decode_parity(vm, orc):
    """B=1, 16/4 heads, ctx 512, position 511 (0-based)."""
    banner("config1 decode B=1 ctx=512 pos=512")
    (mx, mn), (kmx, kmn), vexact, _, _ = run_decode_vs_oracle(vm, orc, 1, 512, [512], seed=100)
    print(f"config1: out max {mx:.3e} mean {mn:.3e}; K max {kmx:.3e} mean {kmn:.3e}")
    assert mx <= TOL_MAX and mn <= TOL_MEAN
    assert kmx <= TOL_MAX and kmn <= TOL_MEAN and vexact


@pytest.mark.parametrize("pos", [[1, 2, 31, 32, 33, 127, 128, 129],
                                 [700, 1000, 1023, 1024, 5, 64, 333, 999]])
def test_ragged_edge_lengths(vm, orc, pos):
    banner(f"ragged decode B=8 ctx=1024 pos={pos}")
    (mx, mn), (kmx, _), vexact, _, _ = run_decode_vs_oracle(vm, orc, 8, 1024, pos, seed=200)
    assert mx <= TOL_MAX and mn <= TOL_MEAN and kmx <= TOL_MAX and vexact


@pytest.mark.parametrize("Hq,Hk", [(8, 8), (16, 2), (12, 4), (24, 4)])
def test_gqa_groups(vm, orc, Hq, Hk):
    banner(f"decode GQA Hq={Hq} Hk={Hk}")
    (mx, mn), _, vexact, _, _ = run_decode_vs_oracle(vm, orc, 2, 640, [640, 77], Hq=Hq, Hk=Hk,
                                                     seed=300)
    assert mx <= TOL_MAX and mn <= TOL_MEAN and vexact


def test_fused_decode_running_max_path(vm, orc):
    """A norm weight of 4 (|kw + 1| = 5) lifts the QK-norm logit bound past the
    static limit of 64 (log2 units), so the fused decode takes its running-max
    path (appended row first, from m = -inf); checked against the oracle."""
    banner("fused decode running-max path (kw[0] = 4)")
    (mx, mn), (kmx, kmn), vexact, _, _ = run_decode_vs_oracle(
        vm, orc, 4, 2048, [2048, 1, 700, 1500], seed=250, kw_big=4.0)
    print(f"running-max decode: out max {mx:.3e} mean {mn:.3e}; K max {kmx:.3e}")
    assert mx <= TOL_MAX and mn <= TOL_MEAN and kmx <= TOL_MAX and kmn <= TOL_MEAN and vexact


def test_fused_decode_zero_position(vm, orc):
    """positions[b] = 0 in a batch: that sequence attends no key, so its output is
    0 (attention_decode.jl:114-128) and its cache is not written; the others are
    unaffected. A whole batch at 0 gives all zeros."""
    banner("fused decode with zero positions")
    (mx, mn), (kmx, _), ok, got, _ = run_decode_vs_oracle(vm, orc, 4, 1024, [0, 513, 0, 1024],
                                                          seed=260)
    assert np.all(got[0] == 0.0) and np.all(got[2] == 0.0)
    assert mx <= TOL_MAX and mn <= TOL_MEAN and kmx <= TOL_MAX and ok
    _, _, ok, got, _ = run_decode_vs_oracle(vm, orc, 2, 256, [0, 0], seed=270)
    assert np.all(got == 0.0) and ok


def test_decode_attention_zero_length(vm, orc):
    """decode_attention! with lengths[b] = 0: o = 0 for that sequence (the empty-split
    guards, attention_decode.jl:80-82, 114-128); the rest match the oracle."""
    banner("decode_attention_ zero lengths")
    B, H, Hk, ctx = 4, 16, 4, 1024
    q_bits = normal_bf16((B, H, D), 511)
    kc, vc = normal_bf16((B, Hk, ctx, D), 512), normal_bf16((B, Hk, ctx, D), 513)
    lengths = np.array([0, 700, 0, 1], np.int32)
    out = vm.decode_attention(to_dev(q_bits), to_dev(kc), to_dev(vc), lengths=i32(lengths))["O"]
    torch.cuda.synchronize()
    got = dev_f32(out)
    ref = orc.attention(bf16_to_f32(q_bits).reshape(B, H, 1, D), bf16_to_f32(kc).reshape(kc.shape),
                        bf16_to_f32(vc).reshape(vc.shape), causal=False, k_lengths=lengths)[:, :, 0]
    assert np.all(ref[[0, 2]] == 0.0)
    assert np.all(got[0] == 0.0) and np.all(got[2] == 0.0)
    mx, mn = maxmean(got, ref)
    assert mx <= TOL_MAX and mn <= TOL_MEAN


def test_split_count_invariance(vm, orc):
    """attention_decode.jl:80-82,114-120: the result does not depend on how the
    keys are split (empty splits included)."""
    outs = []
    for ns in (1, 2, 3, 8, 40, 0):
        banner(f"decode split invariance n_splits={ns}")
        (mx, mn), _, _, got, ref = run_decode_vs_oracle(vm, orc, 3, 5000, [5000, 129, 2711],
                                                        seed=400, n_splits=ns)
        assert mx <= TOL_MAX and mn <= TOL_MEAN, ns
        outs.append(got)
    for o in outs[1:]:
        assert np.max(np.abs(o - outs[0])) <= 2 * 2 ** -8 * np.max(np.abs(outs[0])) + 1e-3


def test_decode_attention_operator(vm, orc):
    """decode_attention! (a5) on already-normalised Q, caches with a head stride
    of the full capacity and lengths shorter than it."""
    banner("decode_attention_ operator B=4 ctx=2048")
    B, H, Hk, ctx = 4, 16, 4, 2048
    q_bits = normal_bf16((B, H, D), 501)
    kc, vc = normal_bf16((B, Hk, ctx, D), 502), normal_bf16((B, Hk, ctx, D), 503)
    lengths = np.array([2048, 1, 1000, 77], np.int32)
    out = vm.decode_attention(to_dev(q_bits), to_dev(kc), to_dev(vc), lengths=i32(lengths))["O"]
    torch.cuda.synchronize()
    ref = orc.attention(bf16_to_f32(q_bits).reshape(B, H, 1, D), bf16_to_f32(kc).reshape(kc.shape),
                        bf16_to_f32(vc).reshape(vc.shape), causal=False, k_lengths=lengths)
    mx, mn = maxmean(dev_f32(out), ref[:, :, 0])
    assert mx <= TOL_MAX and mn <= TOL_MEAN


def test_config3_batched_decode_full_size(vm, orc):
    """BASELINE config 3 at full size: B=32, capacity 32768, attended lengths
    ~U{1024..32768} (seeded); every sequence re-evaluated by the oracle (its
    caches copied to the host one sequence at a time), with its appended row."""
    banner("config3 decode B=32 ctx=32768")
    B, ctx = 32, 32768
    rng = np.random.default_rng(3)
    pos = rng.integers(1024, 32769, size=B).astype(np.int32)
    pos[0], pos[1] = 32768, 1024
    K = torch.empty((B, HK, ctx, D), dtype=torch.bfloat16, device="cuda")
    V = torch.empty_like(K)
    vm.fill_normal_(K, 3001)
    vm.fill_normal_(V, 3002)
    cfg, m, layer, qw, kw = make_layer(vm, B, ctx, seed=3000, caches=(K, V))
    qkv = normal_bf16((B, S, D), 3005)
    gen = vm.Generation(B)
    gen.positions.copy_(i32(pos))
    O = torch.empty((B, HQ, D), dtype=torch.bfloat16, device="cuda")
    vm.gated_attn_decode_(O, layer, m, gen, to_dev(qkv))
    torch.cuda.synchronize()
    got = dev_f32(O)
    assert np.all(np.isfinite(got))
    c, s = orc.rope_tables(HALF, ctx, THETA)
    errs, kerrs = [], []
    for b in range(B):
        # the step appended row pos[b] - 1: the oracle re-does the append from the
        # raw projection, so the prior rows it reads are the cache as written
        kc, vc = from_dev(K[b:b + 1]), from_dev(V[b:b + 1])
        ref, kn, _ = orc.gated_decode(qkv[b:b + 1], kc, vc, pos[b:b + 1], qw, kw, c, s, Hq=HQ, Hk=HK,
                                      eps=EPS, w_offset=1.0)
        errs.append(np.abs(got[b:b + 1].astype(np.float64) - ref))
        kerrs.append(np.abs(bf16_to_f32(kc[0][:, pos[b] - 1]).astype(np.float64) - kn[0]))
    e, ke = np.concatenate([x.ravel() for x in errs]), np.concatenate([x.ravel() for x in kerrs])
    worst = int(np.argmax([x.max() for x in errs]))
    print(f"config3, all {B} sequences: out max {e.max():.3e} (sequence {worst}, length "
          f"{pos[worst]}) mean {e.mean():.3e}; K max {ke.max():.3e} mean {ke.mean():.3e}")
    assert e.max() <= TOL_MAX and e.mean() <= TOL_MEAN
    assert ke.max() <= TOL_MAX and ke.mean() <= TOL_MEAN


def test_config4_graph_replay_matches_eager(vm, orc):
    """one decode step (append, split-K, merge, gate, advance)
    captured once in a hipGraph; replays advance the device clock. 256 replays
    (positions 131072..131327) equal 256 eager steps bit for bit (outputs and the
    256 appended cache rows), and the last step matches the oracle."""
    banner("config4 graph replay B=1 ctx=131328, 256 replays")
    B, ctx, p0, n = 1, 131328, 131072, 256
    K = torch.empty((B, HK, ctx, D), dtype=torch.bfloat16, device="cuda")
    V = torch.empty_like(K)
    vm.fill_normal_(K, 4001)
    vm.fill_normal_(V, 4002)
    K0, V0 = K.clone(), V.clone()
    cfg, m, layer, qw, kw = make_layer(vm, B, ctx, seed=4000, caches=(K, V))
    qkv_bits = normal_bf16((B, S, D), 4005)
    qkv = to_dev(qkv_bits)
    O = torch.empty((B, HQ, D), dtype=torch.bfloat16, device="cuda")

    gen = vm.Generation(B)
    gen.positions.fill_(p0)
    eager = []
    for _ in range(n):
        vm.gated_attn_decode_(O, layer, m, gen, qkv, advance=True)
        eager.append(O.clone())
    torch.cuda.synchronize()
    assert gen.positions.item() == p0 + n
    K_eager, V_eager = K.clone(), V.clone()

    K.copy_(K0)
    V.copy_(V0)
    gen.positions.fill_(p0)
    torch.cuda.synchronize()
    sess = vm.CaptureSession().capture(lambda: vm.gated_attn_decode_(O, layer, m, gen, qkv, advance=True))
    assert gen.positions.item() == p0          # capture records without executing
    replay = []
    for _ in range(n):
        sess.launch()
        replay.append(O.clone())
    torch.cuda.synchronize()
    sess.close()
    assert gen.positions.item() == p0 + n
    for a, b in zip(eager, replay):
        assert torch.equal(a, b)
    assert torch.equal(K_eager, K) and torch.equal(V_eager, V)
    # oracle on the last step (its cache holds the 255 rows appended before it)
    c, s = orc.rope_tables(HALF, ctx, THETA)
    kc, vc = from_dev(K), from_dev(V)
    ref, _, _ = orc.gated_decode(qkv_bits, kc, vc, np.array([p0 + n - 1], np.int32), qw, kw, c, s,
                                 Hq=HQ, Hk=HK, eps=EPS, w_offset=1.0)
    mx, mn = maxmean(dev_f32(replay[-1]), ref)
    print(f"config4 last replay: out max {mx:.3e} mean {mn:.3e}")
    assert mx <= TOL_MAX and mn <= TOL_MEAN
