"""Prefill path on the GPU vs the oracle: attention! (a8) alone, the fused
forward(::AttnLayer) (a9 prologue + a8 + a10 gate epilogue, a11) including
ragged chunked prefill, BASELINE configs 2 and 5 at full size (sampled query
rows against the oracle, every appended cache row checked), and the
cross-kernel identities: decode == last prefill row, chunked == full prefill."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import (D, EPS, HALF, HK, HQ, S, THETA, TOL_MAX, TOL_MEAN, banner, dev_f32,
                      from_dev, i32, maxmean, to_dev)
from oracle.rng import bf16_to_f32, normal_bf16

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("H,Hk,L,Lk", [(16, 4, 200, 300), (8, 8, 130, 130), (16, 2, 1, 77),
                                       (4, 1, 257, 1000)])
def test_attention_operator(vm, orc, causal, H, Hk, L, Lk):
    banner(f"attention_ causal={causal} H={H} Hk={Hk} L={L} Lk={Lk}")
    B = 2
    q = normal_bf16((B, H, L, D), 11)
    k = normal_bf16((B, Hk, Lk, D), 12)
    v = normal_bf16((B, Hk, Lk, D), 13)
    o = vm.attention(to_dev(q), to_dev(k), to_dev(v), causal=causal)["O"]
    torch.cuda.synchronize()
    ref = orc.attention(bf16_to_f32(q).reshape(q.shape), bf16_to_f32(k).reshape(k.shape),
                        bf16_to_f32(v).reshape(v.shape), causal=causal)
    mx, mn = maxmean(dev_f32(o), ref)
    assert mx <= TOL_MAX and mn <= TOL_MEAN


def test_attention_ragged_rows_untouched(vm, orc):
    banner("attention_ ragged k/q lengths")
    B, H, Hk, L, Lk = 3, 16, 4, 300, 700
    q = normal_bf16((B, H, L, D), 21)
    k = normal_bf16((B, Hk, Lk, D), 22)
    v = normal_bf16((B, Hk, Lk, D), 23)
    kl = np.array([700, 300, 129], np.int32)
    ql = np.array([300, 1, 129], np.int32)
    O = torch.full((B, H, L, D), 7.0, dtype=torch.bfloat16, device="cuda")
    vm.attention_({"O": O}, to_dev(q), to_dev(k), to_dev(v), causal=True, k_lengths=i32(kl),
                  q_lengths=i32(ql))
    torch.cuda.synchronize()
    ref = orc.attention(bf16_to_f32(q).reshape(q.shape), bf16_to_f32(k).reshape(k.shape),
                        bf16_to_f32(v).reshape(v.shape), causal=True, k_lengths=kl, q_lengths=ql)
    got = dev_f32(O)
    fin = ~np.isnan(ref)
    mx, mn = maxmean(got[fin], ref[fin])
    assert mx <= TOL_MAX and mn <= TOL_MEAN
    assert np.all(got[~fin] == 7.0)


def _fused(vm, orc, B, T, ctx, prior, qlen, seed, row_step=1, fill_gpu=False):
    cfg = vm.AttnConfig(Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=ctx, B=B)
    qw = normal_bf16((D,), seed + 1, scale=0.05)
    kw = normal_bf16((D,), seed + 2, scale=0.05)
    if fill_gpu:
        K = torch.empty((B, HK, ctx, D), dtype=torch.bfloat16, device="cuda")
        V = torch.empty_like(K)
        vm.fill_normal_(K, seed + 3)
        vm.fill_normal_(V, seed + 4)
    else:
        K = to_dev(normal_bf16((B, HK, ctx, D), seed + 3))
        V = to_dev(normal_bf16((B, HK, ctx, D), seed + 4))
    kc, vc = from_dev(K), from_dev(V)
    qkv = normal_bf16((B, T, S, D), seed + 5)
    m = vm.AttnModel(cfg)
    layer = vm.AttnLayer(qw=to_dev(qw), kw=to_dev(kw), K_cache=K, V_cache=V)
    out = vm.gated_attn_prefill(layer, m, to_dev(qkv), T, B, prior=i32(prior), q_lengths=i32(qlen))
    torch.cuda.synchronize()
    got = dev_f32(out).reshape(B, T, HQ, D)
    c, s = orc.rope_tables(HALF, ctx, THETA)
    ref, kn, vn = orc.gated_prefill(qkv, kc, vc, prior, qlen, qw, kw, c, s, Hq=HQ, Hk=HK, eps=EPS,
                                    w_offset=1.0, row_step=row_step)
    fin = ~np.isnan(ref)
    mx, mn = maxmean(got[fin], ref[fin])
    kg, vg = from_dev(layer.K_cache), from_dev(layer.V_cache)
    kerr = []
    vex = True
    for b in range(B):
        P, C = int(prior[b]), int(qlen[b])
        kerr.append(np.abs(bf16_to_f32(kg[b, :, P:P + C]).reshape(HK, C, D) - kn[b, :, :C]))
        vex &= np.array_equal(bf16_to_f32(vg[b, :, P:P + C]).reshape(HK, C, D), vn[b, :, :C])
        # columns outside [P, P+C) untouched
        keep = np.ones(ctx, bool)
        keep[P:P + C] = False
        vex &= np.array_equal(kg[b][:, keep], kc[b][:, keep])
        vex &= np.array_equal(vg[b][:, keep], vc[b][:, keep])
    kerr = np.concatenate([e.ravel() for e in kerr])
    return (mx, mn), (float(kerr.max()), float(kerr.mean())), vex, out


def test_fused_prefill_small_ragged(vm, orc):
    banner("fused prefill B=3 ragged")
    (mx, mn), (kmx, kmn), ok, _ = _fused(vm, orc, 3, 300, 1024, np.array([0, 129, 700], np.int32),
                                         np.array([300, 31, 257], np.int32), 50)
    assert mx <= TOL_MAX and mn <= TOL_MEAN and kmx <= TOL_MAX and kmn <= TOL_MEAN and ok


def test_config2_prefill_full_size(vm, orc):
    """causal prefill, B=1, T=4096, offset 0; every query row
    re-evaluated by the oracle, every appended K/V row checked."""
    banner("config2 prefill T=4096")
    (mx, mn), (kmx, kmn), ok, _ = _fused(vm, orc, 1, 4096, 4096, np.array([0], np.int32),
                                         np.array([4096], np.int32), 60, row_step=1)
    print(f"config2: out max {mx:.3e} mean {mn:.3e}; K max {kmx:.3e} mean {kmn:.3e}")
    assert mx <= TOL_MAX and mn <= TOL_MEAN and kmx <= TOL_MAX and kmn <= TOL_MEAN and ok


def test_config5_chunked_prefill_full_size(vm, orc):
    """B=4 ragged chunks (a seeded permutation of
    {512, 1024, 2048, 2048}) after prior caches ~U{8192..32768}; every query row
    of every sequence re-evaluated by the oracle."""
    rng = np.random.default_rng(5)
    qlen = rng.permutation(np.array([512, 1024, 2048, 2048], np.int32)).astype(np.int32)
    prior = rng.integers(8192, 32769, size=4).astype(np.int32)
    ctx = int((prior + qlen).max())
    banner(f"config5 chunked prefill prior={prior.tolist()} chunks={qlen.tolist()} ctx={ctx}")
    (mx, mn), (kmx, kmn), ok, _ = _fused(vm, orc, 4, 2048, ctx, prior, qlen, 70, row_step=1,
                                         fill_gpu=True)
    print(f"config5: out max {mx:.3e} mean {mn:.3e}; K max {kmx:.3e} mean {kmn:.3e}")
    assert mx <= TOL_MAX and mn <= TOL_MEAN and kmx <= TOL_MAX and kmn <= TOL_MEAN and ok


def test_fused_append_equals_standalone_append(vm):
    """The gated prefill appends K/V inside its V^T staging kernel; the cache it
    leaves is bit-identical to vm_prefill_kv_append's (a9, qwen35.jl:306-307),
    ragged, with a prior prefix and a chunk that stops short of the cache end."""
    banner("fused append == vm_prefill_kv_append")
    ops, call = vm.ops, vm._lib.call
    B, T, ctx = 3, 300, 1024
    prior = np.array([0, 129, 700], np.int32)
    qlen = np.array([300, 31, 257], np.int32)
    cfg = vm.AttnConfig(Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=ctx, B=B)
    m = vm.AttnModel(cfg)
    qw = to_dev(normal_bf16((D,), 71, scale=0.05))
    kw = to_dev(normal_bf16((D,), 72, scale=0.05))
    kc0 = to_dev(normal_bf16((B, HK, ctx, D), 73))
    vc0 = to_dev(normal_bf16((B, HK, ctx, D), 74))
    qkv = to_dev(normal_bf16((B, T, S, D), 75))
    la = vm.AttnLayer(qw=qw, kw=kw, K_cache=kc0.clone(), V_cache=vc0.clone())
    vm.gated_attn_prefill(la, m, qkv, T, B, prior=i32(prior), q_lengths=i32(qlen))
    K, V = kc0.clone(), vc0.clone()
    pr, ql = i32(prior), i32(qlen)  # held: the C ABI takes bare device pointers
    call("vm_prefill_kv_append", ops._p(K), ops._p(V), K.stride(2), K.stride(1), K.stride(0), ctx,
         ops._p(qkv), qkv.stride(1), qkv.stride(0), ops._p(kw), ops._p(m.rope["cos"]),
         ops._p(m.rope["sin"]), ops._p(pr), ops._p(ql), B, T, HQ, HK, D, HALF, float(EPS), 1.0,
         ops._stream())
    torch.cuda.synchronize()
    assert torch.equal(la.K_cache, K) and torch.equal(la.V_cache, V)
    assert not torch.equal(K, kc0)  # the append did write


def test_decode_equals_last_prefill_row(vm):
    """A decode step at position p equals the last row of a causal prefill over
    p tokens (both on the GPU; same cache contents)."""
    banner("decode == last prefill row")
    B, T, ctx = 2, 333, 512
    cfg = vm.AttnConfig(Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=ctx, B=B)
    qw, kw = to_dev(normal_bf16((D,), 81, scale=0.05)), to_dev(normal_bf16((D,), 82, scale=0.05))
    qkv = to_dev(normal_bf16((B, T, S, D), 83))
    m = vm.AttnModel(cfg)
    la = vm.attn_layer(cfg, qw, kw)
    full = vm.gated_attn_prefill(la, m, qkv, T, B)
    lb = vm.attn_layer(cfg, qw, kw)
    vm.gated_attn_prefill(lb, m, qkv[:, :T - 1].contiguous(), T - 1, B)
    gen = vm.Generation(B)
    gen.positions.fill_(T)
    O = torch.empty((B, HQ, D), dtype=torch.bfloat16, device="cuda")
    vm.gated_attn_decode_(O, lb, m, gen, qkv[:, T - 1].contiguous())
    torch.cuda.synchronize()
    a = full.reshape(B, T, HQ, D)[:, T - 1].float().cpu().numpy()
    b = O.float().cpu().numpy()
    mx, mn = maxmean(a, b)
    assert mx <= TOL_MAX and mn <= TOL_MEAN
    assert torch.equal(la.K_cache, lb.K_cache) and torch.equal(la.V_cache, lb.V_cache)


def test_chunked_equals_full_prefill(vm):
    """attention.jl:3-7 — chunk after P cached tokens == rows P.. of the full prefill."""
    banner("chunked == full prefill")
    B, T, P, ctx = 1, 700, 300, 1024
    cfg = vm.AttnConfig(Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=ctx, B=B)
    qw, kw = to_dev(normal_bf16((D,), 91, scale=0.05)), to_dev(normal_bf16((D,), 92, scale=0.05))
    qkv = to_dev(normal_bf16((B, T, S, D), 93))
    m = vm.AttnModel(cfg)
    la = vm.attn_layer(cfg, qw, kw)
    full = vm.gated_attn_prefill(la, m, qkv, T, B)
    lb = vm.attn_layer(cfg, qw, kw)
    vm.gated_attn_prefill(lb, m, qkv[:, :P].contiguous(), P, B)
    part = vm.gated_attn_prefill(lb, m, qkv[:, P:].contiguous(), T - P, B, offset=P)
    torch.cuda.synchronize()
    mx, mn = maxmean(full[:, P:].float().cpu().numpy(), part.float().cpu().numpy())
    assert mx <= 1e-2 and mn <= 1e-3
    assert torch.equal(la.K_cache, lb.K_cache)


def test_fused_prefill_prior_null_attends_chunk_only(vm, orc):
    """prior == NULL means no prior tokens (vallmo_attn.h): the fused prefill must
    attend cache columns 1..q_len only, never the rest of a larger cache (filled
    here with keys that would dominate every softmax if they were attended)."""
    banner("fused prefill prior=NULL ctx > T")
    B, T, ctx = 2, 200, 512
    qw = normal_bf16((D,), 101, scale=0.05)
    kw = normal_bf16((D,), 102, scale=0.05)
    qkv = normal_bf16((B, T, S, D), 103)
    stale = np.full((B, HK, ctx, D), 0x4200, np.uint16)  # bf16 32.0
    K, V = to_dev(stale), to_dev(stale)
    cos = torch.empty((ctx, HALF), dtype=torch.float32, device="cuda")
    sin = torch.empty_like(cos)
    vm._lib.call("vm_rope_tables", cos.data_ptr(), sin.data_ptr(), HALF, ctx, THETA, None)
    out = torch.empty((B, T, HQ * D), dtype=torch.bfloat16, device="cuda")
    dq, dqw, dkw = to_dev(qkv), to_dev(qw), to_dev(kw)  # held: the call takes raw pointers
    nws = vm._lib.load().vm_prefill_scratch_bytes(B, HK, D, ctx)
    ws = torch.empty(nws, dtype=torch.uint8, device="cuda")
    vm._lib.call("vm_gated_attn_prefill", out.data_ptr(), out.stride(1), out.stride(0),
                 dq.data_ptr(), S * D, T * S * D, K.data_ptr(), V.data_ptr(), D, ctx * D,
                 HK * ctx * D, ctx, dqw.data_ptr(), dkw.data_ptr(), cos.data_ptr(),
                 sin.data_ptr(), None, None, B, T, HQ, HK, D, HALF, EPS, 1.0, ws.data_ptr(),
                 nws, None)
    torch.cuda.synchronize()
    c, s = orc.rope_tables(HALF, ctx, THETA)
    ref, _, _ = orc.gated_prefill(qkv, stale, stale, np.zeros(B, np.int32),
                                  np.full(B, T, np.int32), qw, kw, c, s, Hq=HQ, Hk=HK, eps=EPS,
                                  w_offset=1.0)
    mx, mn = maxmean(dev_f32(out).reshape(B, T, HQ, D), ref)
    assert mx <= TOL_MAX and mn <= TOL_MEAN


def test_fused_prefill_online_max_path(vm, orc):
    """One large K-norm weight (kw[0] = 4, so max|kw + 1| = 5) lifts the QK-norm
    logit bound to ~118 log2 units, past the static-shift limit of 64, while the
    actual logits stay moderate: the fused kernel then runs its online running max
    with lazy rescaling, and must still match the oracle."""
    banner("fused prefill online-max path (one large k-norm weight)")
    B, T, ctx = 2, 384, 640
    cfg = vm.AttnConfig(Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=ctx, B=B)
    qw = normal_bf16((D,), 111, scale=0.05)
    kw = normal_bf16((D,), 112, scale=0.05)
    kw[0] = 0x4080  # bf16 4.0
    kc = normal_bf16((B, HK, ctx, D), 113)
    vc = normal_bf16((B, HK, ctx, D), 114)
    qkv = normal_bf16((B, T, S, D), 115)
    prior = np.array([0, 256], np.int32)
    qlen = np.array([384, 300], np.int32)
    m = vm.AttnModel(cfg)
    layer = vm.AttnLayer(qw=to_dev(qw), kw=to_dev(kw), K_cache=to_dev(kc), V_cache=to_dev(vc))
    out = vm.gated_attn_prefill(layer, m, to_dev(qkv), T, B, prior=i32(prior), q_lengths=i32(qlen))
    torch.cuda.synchronize()
    c, s = orc.rope_tables(HALF, ctx, THETA)
    ref, _, _ = orc.gated_prefill(qkv, kc, vc, prior, qlen, qw, kw, c, s, Hq=HQ, Hk=HK, eps=EPS,
                                  w_offset=1.0)
    got = dev_f32(out).reshape(B, T, HQ, D)
    fin = ~np.isnan(ref)
    mx, mn = maxmean(got[fin], ref[fin])
    print(f"online-max path: out max {mx:.3e} mean {mn:.3e}")
    assert mx <= TOL_MAX and mn <= TOL_MEAN


def test_attention_zero_k_length(vm, orc):
    """attention! with k_lengths[b] = 0: no key is valid, so every row of that
    sequence is 0 (the l == 0 guard, attention.jl:86), causal or not; a sequence
    with q_lengths[b] = 0 is not written at all; the rest match the oracle."""
    B, H, Hk, L, Lk = 3, 16, 4, 96, 256
    q = normal_bf16((B, H, L, D), 31)
    k = normal_bf16((B, Hk, Lk, D), 32)
    v = normal_bf16((B, Hk, Lk, D), 33)
    kl = np.array([0, 200, 0], np.int32)
    ql = np.array([96, 96, 0], np.int32)
    for causal in (False, True):
        banner(f"attention_ zero k_length causal={causal}")
        O = torch.full((B, H, L, D), 7.0, dtype=torch.bfloat16, device="cuda")
        vm.attention_({"O": O}, to_dev(q), to_dev(k), to_dev(v), causal=causal,
                      k_lengths=i32(kl), q_lengths=i32(ql))
        torch.cuda.synchronize()
        got = dev_f32(O)
        assert np.all(got[0] == 0.0)
        assert np.all(got[2] == 7.0)
        ref = orc.attention(bf16_to_f32(q).reshape(q.shape), bf16_to_f32(k).reshape(k.shape),
                            bf16_to_f32(v).reshape(v.shape), causal=causal, k_lengths=kl,
                            q_lengths=ql)
        assert np.all(ref[0] == 0.0)
        mx, mn = maxmean(got[1], ref[1])
        assert mx <= TOL_MAX and mn <= TOL_MEAN


def test_prefill_q_norm_rope_operator(vm, orc):
    """vm_prefill_q_norm_rope (the unfused prefill prologue for attention!,
    qwen35.jl:297-304): per-head RMSNorm (w + 1) and partial RoPE of q read from
    the packed projection, at position prior[b] + t, into Q :: (D, T, Hq, B);
    rows t >= q_lengths[b] are not written."""
    banner("vm_prefill_q_norm_rope ragged")
    B, T, ctx = 2, 150, 1024
    prior = np.array([0, 700], np.int32)
    qlen = np.array([150, 61], np.int32)
    qw = normal_bf16((D,), 121, scale=0.05)
    qkv = normal_bf16((B, T, S, D), 122)
    cos = torch.empty((ctx, HALF), dtype=torch.float32, device="cuda")
    sin = torch.empty_like(cos)
    vm._lib.call("vm_rope_tables", cos.data_ptr(), sin.data_ptr(), HALF, ctx, THETA, None)
    Q = torch.full((B, HQ, T, D), 7.0, dtype=torch.bfloat16, device="cuda")
    dq, dqw, pr, ql = to_dev(qkv), to_dev(qw), i32(prior), i32(qlen)
    vm._lib.call("vm_prefill_q_norm_rope", Q.data_ptr(), Q.stride(2), Q.stride(1), Q.stride(0),
                 dq.data_ptr(), S * D, T * S * D, dqw.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                 pr.data_ptr(), ql.data_ptr(), B, T, HQ, HK, D, HALF, EPS, 1.0, None)
    torch.cuda.synchronize()
    got = dev_f32(Q)
    c, s = orc.rope_tables(HALF, ctx, THETA)
    wf = bf16_to_f32(qw)
    ref = np.full((B, HQ, T, D), np.nan, np.float32)
    for b in range(B):
        for t in range(int(qlen[b])):
            for h in range(HQ):
                x = bf16_to_f32(qkv[b, t, 2 * h])
                ref[b, h, t] = orc.head_norm_rope(x, wf, EPS, 1.0, c, s, int(prior[b]) + t)
    fin = ~np.isnan(ref)
    mx, mn = maxmean(got[fin], ref[fin])
    print(f"prefill q norm+rope: max {mx:.3e} mean {mn:.3e}")
    assert mx <= TOL_MAX and mn <= TOL_MEAN
    assert np.all(got[~fin] == 7.0)


# ---- paired items: one sequence, causal, >= 2 items per CU (H n_qt >= 2 x 256) --
# Each workgroup of the fused kernel then runs a heavy and a light q-block of
# one head; B > 1 keeps one item per workgroup. Per item the arithmetic is the
# same either way.

def test_paired_prefill_equals_one_item_per_workgroup(vm):
    """B = 1, T = 4096 (paired workgroups) against the same sequence twice at
    B = 2 (one item per workgroup): outputs and appended cache rows bit-equal."""
    banner("paired prefill == unpaired (B=1 vs B=2 copies, T=4096)")
    T, ctx = 4096, 4096
    qw, kw = to_dev(normal_bf16((D,), 301, scale=0.05)), to_dev(normal_bf16((D,), 302, scale=0.05))
    qkv1 = torch.empty((1, T, S, D), dtype=torch.bfloat16, device="cuda")
    vm.fill_normal_(qkv1, 303)
    outs, caches = [], []
    for B in (1, 2):
        cfg = vm.AttnConfig(Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=ctx, B=B)
        m = vm.AttnModel(cfg)
        layer = vm.attn_layer(cfg, qw, kw)
        qkv = qkv1.expand(B, -1, -1, -1).contiguous()
        outs.append(vm.gated_attn_prefill(layer, m, qkv, T, B))
        caches.append((layer.K_cache, layer.V_cache))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][0], outs[1][1])
    assert torch.equal(caches[0][0][0], caches[1][0][0]) and torch.equal(caches[0][1][0], caches[1][1][0])


def test_paired_prefill_prior_and_short_chunk(vm, orc):
    """Paired workgroups after 300 cached tokens with q_lengths = 2999 of T = 4096:
    the heavy q-blocks past the chunk return at once and their light partners
    still run; every 16th row against the oracle, every appended row checked."""
    banner("paired prefill prior=300 q_len=2999 T=4096")
    (mx, mn), (kmx, kmn), ok, _ = _fused(vm, orc, 1, 4096, 4396, np.array([300], np.int32),
                                         np.array([2999], np.int32), 310, row_step=16,
                                         fill_gpu=True)
    print(f"paired prior: out max {mx:.3e} mean {mn:.3e}; K max {kmx:.3e} mean {kmn:.3e}")
    assert mx <= TOL_MAX and mn <= TOL_MEAN and kmx <= TOL_MAX and kmn <= TOL_MEAN and ok


def test_paired_prefill_online_max_path(vm, orc):
    """The online running-max path (kw[0] = 4 lifts the logit bound past 64) on
    paired workgroups (B = 1, T = 4096); every 16th row against the oracle."""
    banner("paired prefill online-max path T=4096")
    B, T, ctx = 1, 4096, 4096
    cfg = vm.AttnConfig(Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=ctx, B=B)
    qw = normal_bf16((D,), 321, scale=0.05)
    kw = normal_bf16((D,), 322, scale=0.05)
    kw[0] = 0x4080  # bf16 4.0
    K = torch.empty((B, HK, ctx, D), dtype=torch.bfloat16, device="cuda")
    V = torch.empty_like(K)
    vm.fill_normal_(K, 323)
    vm.fill_normal_(V, 324)
    kc, vc = from_dev(K), from_dev(V)
    qkv = normal_bf16((B, T, S, D), 325)
    m = vm.AttnModel(cfg)
    layer = vm.AttnLayer(qw=to_dev(qw), kw=to_dev(kw), K_cache=K, V_cache=V)
    prior, qlen = np.zeros(1, np.int32), np.full(1, T, np.int32)
    out = vm.gated_attn_prefill(layer, m, to_dev(qkv), T, B, prior=i32(prior), q_lengths=i32(qlen))
    torch.cuda.synchronize()
    c, s = orc.rope_tables(HALF, ctx, THETA)
    ref, _, _ = orc.gated_prefill(qkv, kc, vc, prior, qlen, qw, kw, c, s, Hq=HQ, Hk=HK, eps=EPS,
                                  w_offset=1.0, row_step=16)
    got = dev_f32(out).reshape(B, T, HQ, D)
    fin = ~np.isnan(ref)
    mx, mn = maxmean(got[fin], ref[fin])
    print(f"paired online-max: out max {mx:.3e} mean {mn:.3e}")
    assert mx <= TOL_MAX and mn <= TOL_MEAN


def test_staged_prefill_chunks_equal_full_staging(vm):
    """vm_gated_attn_prefill_staged over a chunk-by-chunk, ragged prefill (B = 2):
    each chunk stages only its own rows into the kept V^T workspace, and rows
    written at a sequence's end between chunks (as decode steps append them) are
    staged by the next chunk. Every output and both caches equal those of the
    per-call full staging, bit for bit, and rows[b] = prior[b] + q_len[b] after
    each call. After reset_(b), a rewritten prefix of sequence b is staged
    again."""
    banner("staged V^T prefill: chunks == full staging")
    B, T, ctx = 2, 384, 2048
    cfg = vm.AttnConfig(Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=ctx, B=B)
    qw, kw = to_dev(normal_bf16((D,), 351, scale=0.05)), to_dev(normal_bf16((D,), 352, scale=0.05))
    m = vm.AttnModel(cfg)
    la = vm.attn_layer(cfg, qw, kw)  # full staging on every call
    lb = vm.attn_layer(cfg, qw, kw)  # kept V^T workspace
    st = vm.StagedV(cfg, B)

    def chunk(prior, qlen, seed):
        qkv = to_dev(normal_bf16((B, T, S, D), seed))
        p, q = i32(np.array(prior, np.int32)), i32(np.array(qlen, np.int32))
        oa = vm.gated_attn_prefill(la, m, qkv, T, B, prior=p, q_lengths=q)
        ob = vm.gated_attn_prefill(lb, m, qkv, T, B, prior=p, q_lengths=q, staged=st)
        torch.cuda.synchronize()
        print(f"chunk prior={prior} q_len={qlen}: rows held {st.rows.tolist()}", flush=True)
        for bb in range(B):  # rows past q_len[b] are not written
            assert torch.equal(oa[bb, :qlen[bb]].view(torch.int16), ob[bb, :qlen[bb]].view(torch.int16))
        assert torch.equal(la.K_cache, lb.K_cache) and torch.equal(la.V_cache, lb.V_cache)
        assert st.rows.tolist() == [a + b for a, b in zip(prior, qlen)]
        assert st.state[B:].tolist() == [0] * B  # arrival counters left zero

    def write_rows(b, r0, r1, seed):
        for c, s in ((la.K_cache, seed), (la.V_cache, seed + 1)):
            c[b, :, r0:r1, :] = to_dev(normal_bf16((HK, r1 - r0, D), s))
        lb.K_cache.copy_(la.K_cache)
        lb.V_cache.copy_(la.V_cache)

    chunk([0, 0], [384, 200], 353)
    chunk([384, 200], [100, 384], 354)
    write_rows(0, 484, 491, 355)  # 7 rows past each sequence's end, not staged yet
    write_rows(1, 584, 591, 357)
    chunk([491, 591], [250, 31], 359)
    write_rows(0, 0, 64, 360)  # a rewritten prefix: sequence 0 must be staged again
    st.reset_(0)
    chunk([741, 622], [64, 64], 362)
    # the same StagedV used with another layer's cache (same prefix length, other
    # rows) forgets what it held: that cache's prefix is staged
    lc, ld = vm.attn_layer(cfg, qw, kw), vm.attn_layer(cfg, qw, kw)
    for c, sd in ((lc.K_cache, 364), (lc.V_cache, 365)):
        c[:, :, :64, :] = to_dev(normal_bf16((B, HK, 64, D), sd))
    ld.K_cache.copy_(lc.K_cache)
    ld.V_cache.copy_(lc.V_cache)
    qkv = to_dev(normal_bf16((B, T, S, D), 363))
    p, q = i32(np.array([64, 64], np.int32)), i32(np.array([100, 50], np.int32))
    oc = vm.gated_attn_prefill(lc, m, qkv, T, B, prior=p, q_lengths=q)
    od = vm.gated_attn_prefill(ld, m, qkv, T, B, prior=p, q_lengths=q, staged=st)
    torch.cuda.synchronize()
    assert st.rows.tolist() == [164, 114]
    for bb, n in enumerate([100, 50]):
        assert torch.equal(oc[bb, :n].view(torch.int16), od[bb, :n].view(torch.int16))
