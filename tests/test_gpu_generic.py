"""The attention operators at head shapes outside the tuned kernels, on the GPU
vs the CPU oracle: qnorm_rope! and knorm_rope_append!
(src/kernels/qknorm_rope_append.jl:100-141) at power-of-two head dims 16..512
and other rotary widths, attention! (src/kernels/attention.jl:93-129) and
decode_attention! (src/kernels/attention_decode.jl:134-200) at Dk != Dv, other
head dims and GQA groups above 8; fused_deltanet_decode!, deltanet_sequence! and
deltanet_recurrent_decode! (deltanet_fused.jl, deltanet_recurrent.jl) at Dk, Dv
other than 128. The oracle is pinned at these shapes by tests/test_oracle.py
(torch rms_norm + complex rotation, SDPA) and tests/test_oracle_deltanet.py
(the float64 product form at Dk, Dv = 16, 24, 32, 8, 12).

Bar: the north-star parity bar on bf16 outputs (max-abs 2e-2, mean-abs 2e-3);
cache columns and rows that must not be written are compared bit for bit."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import EPS, THETA, TOL_MAX, TOL_MEAN, banner, dev_f32, from_dev, i32, maxmean, to_dev
from oracle.rng import bf16_to_f32, normal_bf16

pytestmark = pytest.mark.gpu


def _tabs(vm, half, ctx):
    return vm.rope_tables(type("C", (), {"rot_half": half, "theta": THETA, "Ctx": ctx}))


@pytest.mark.parametrize("Dh,half", [(16, 8), (64, 8), (128, 64), (512, 32), (256, 16)])
def test_qnorm_rope_head_dims(vm, orc, Dh, half):
    """In place on a strided view (every other head of a packed row); the other
    heads untouched."""
    banner(f"qnorm_rope_ D={Dh} half={half}")
    B, H, ctx = 3, 4, 700
    bits = normal_bf16((B, 2 * H, Dh), 400 + Dh)
    qw = normal_bf16((Dh,), 401, scale=0.05)
    pos = np.array([1, 333, 700], np.int32)
    tabs = _tabs(vm, half, ctx)
    buf = to_dev(bits)
    q = buf[:, 0::2, :]
    vm.qnorm_rope_(q, to_dev(qw), tabs["cos"], tabs["sin"], positions=i32(pos), eps=EPS,
                   offset=1.0)
    torch.cuda.synchronize()
    c, s = orc.rope_tables(half, ctx, THETA)
    ref = np.stack([np.stack([orc.head_norm_rope(bf16_to_f32(bits[b, 2 * h]), bf16_to_f32(qw),
                                                 EPS, 1.0, c, s, pos[b] - 1)
                              for h in range(H)]) for b in range(B)])
    got = dev_f32(buf)
    mx, mn = maxmean(got[:, 0::2], ref)
    print(f"max {mx:.3e} mean {mn:.3e}")
    assert mx <= TOL_MAX and mn <= TOL_MEAN
    assert np.array_equal(from_dev(buf)[:, 1::2], bits[:, 1::2])


@pytest.mark.parametrize("Dk,Dv,half", [(128, 64, 16), (64, 256, 32), (256, 256, 16),
                                        (512, 128, 64)])
def test_knorm_rope_append_head_dims(vm, orc, Dk, Dv, half):
    """One cache column written per sequence: K normed and rotated, V copied bit
    for bit; every other column untouched."""
    banner(f"knorm_rope_append_ Dk={Dk} Dv={Dv} half={half}")
    B, Hk, ctx = 2, 3, 129
    k_bits = normal_bf16((B, Hk, Dk), 410 + Dk)
    v_bits = normal_bf16((B, Hk, Dv), 411 + Dv)
    kw = normal_bf16((Dk,), 412, scale=0.05)
    kc_bits = normal_bf16((B, Hk, ctx, Dk), 413)
    vc_bits = normal_bf16((B, Hk, ctx, Dv), 414)
    pos = np.array([129, 17], np.int32)
    tabs = _tabs(vm, half, ctx)
    kc, vc = to_dev(kc_bits), to_dev(vc_bits)
    vm.knorm_rope_append_(kc, vc, to_dev(k_bits), to_dev(v_bits), to_dev(kw), tabs["cos"],
                          tabs["sin"], positions=i32(pos), eps=EPS, offset=1.0)
    torch.cuda.synchronize()
    c, s = orc.rope_tables(half, ctx, THETA)
    kg, vg = from_dev(kc), from_dev(vc)
    for b in range(B):
        col = pos[b] - 1
        for j in range(Hk):
            ref = orc.head_norm_rope(bf16_to_f32(k_bits[b, j]), bf16_to_f32(kw), EPS, 1.0, c, s,
                                     col)
            mx, mn = maxmean(bf16_to_f32(kg[b, j, col]), ref)
            assert mx <= TOL_MAX and mn <= TOL_MEAN
            assert np.array_equal(vg[b, j, col], v_bits[b, j])
        others = np.ones(ctx, bool)
        others[col] = False
        assert np.array_equal(kg[b][:, others], kc_bits[b][:, others])
        assert np.array_equal(vg[b][:, others], vc_bits[b][:, others])


@pytest.mark.parametrize("Dk,Dv,H,Hk,causal", [(64, 64, 8, 2, True), (128, 128, 8, 2, False),
                                               (128, 128, 16, 4, True), (128, 128, 4, 4, True),
                                               (64, 128, 8, 2, True), (128, 32, 4, 4, True),
                                               (512, 512, 4, 1, True), (16, 16, 16, 1, False),
                                               (256, 128, 32, 2, True)])
def test_attention_head_dims(vm, orc, Dk, Dv, H, Hk, causal):
    """attention! on cache-prefix views (Lk of a longer cache), ragged k/q
    lengths, queries the suffix of the keys; rows past q_len untouched. Dk = Dv
    = 128 or 64 runs the MFMA kernel, the other shapes the generic one."""
    banner(f"attention_ Dk={Dk} Dv={Dv} H={H} Hk={Hk} causal={causal}")
    B, L, Lk, ctx = 2, 37, 100, 128
    q_bits = normal_bf16((B, H, L, Dk), 420)
    k_bits = normal_bf16((B, Hk, ctx, Dk), 421)
    v_bits = normal_bf16((B, Hk, ctx, Dv), 422)
    o_bits = normal_bf16((B, H, L, Dv), 423)
    kl = np.array([100, 40], np.int32)
    ql = np.array([37, 25], np.int32)
    O = to_dev(o_bits)
    vm.attention_({"O": O}, to_dev(q_bits), to_dev(k_bits)[:, :, :Lk], to_dev(v_bits)[:, :, :Lk],
                  causal=causal, k_lengths=i32(kl), q_lengths=i32(ql))
    torch.cuda.synchronize()
    ref = orc.attention(bf16_to_f32(q_bits), bf16_to_f32(k_bits[:, :, :Lk]),
                        bf16_to_f32(v_bits[:, :, :Lk]), causal=causal, k_lengths=kl,
                        q_lengths=ql)
    got = dev_f32(O)
    fin = ~np.isnan(ref)
    mx, mn = maxmean(got[fin], ref[fin])
    print(f"max {mx:.3e} mean {mn:.3e}")
    assert mx <= TOL_MAX and mn <= TOL_MEAN
    assert np.array_equal(from_dev(O)[~fin.any(axis=-1)], o_bits[~fin.any(axis=-1)])


@pytest.mark.parametrize("Dh,causal", [(128, True), (128, False), (64, True), (64, False)])
def test_attention_mfma_head_dims_long(vm, orc, Dh, causal):
    """The MFMA kernel at D = 128 and 64 over many tiles and query blocks (B =
    2, 300 queries against 1000 keys, ragged), every row checked."""
    banner(f"attention_ D={Dh} long causal={causal}")
    B, H, Hk, L, Lk = 2, 8, 2, 300, 1000
    q_bits = normal_bf16((B, H, L, Dh), 425)
    k_bits = normal_bf16((B, Hk, Lk, Dh), 426)
    v_bits = normal_bf16((B, Hk, Lk, Dh), 427)
    kl = np.array([1000, 517], np.int32)
    ql = np.array([300, 129], np.int32)
    O = torch.zeros((B, H, L, Dh), dtype=torch.bfloat16, device="cuda")
    vm.attention_({"O": O}, to_dev(q_bits), to_dev(k_bits), to_dev(v_bits), causal=causal,
                  k_lengths=i32(kl), q_lengths=i32(ql))
    torch.cuda.synchronize()
    ref = orc.attention(bf16_to_f32(q_bits), bf16_to_f32(k_bits), bf16_to_f32(v_bits),
                        causal=causal, k_lengths=kl, q_lengths=ql)
    got = dev_f32(O)
    fin = ~np.isnan(ref)
    mx, mn = maxmean(got[fin], ref[fin])
    print(f"max {mx:.3e} mean {mn:.3e}")
    assert mx <= TOL_MAX and mn <= TOL_MEAN
    assert not got[~fin].any()


@pytest.mark.parametrize("Dk,Dv,H,Hk,n_splits", [(128, 128, 16, 1, 0), (64, 256, 8, 2, 8),
                                                 (256, 256, 32, 2, 0), (128, 64, 4, 4, 1),
                                                 (32, 32, 16, 4, 3)])
def test_decode_attention_head_dims(vm, orc, Dk, Dv, H, Hk, n_splits):
    """decode_attention! at other head dims and groups above 8 (the generic
    split-KV kernel and its merge), ragged lengths including 0 (O = 0) and one
    at the cache's end; each sequence's query is the last of its keys."""
    banner(f"decode_attention_ Dk={Dk} Dv={Dv} H={H} Hk={Hk} n_splits={n_splits}")
    B, ctx = 4, 3000
    q_bits = normal_bf16((B, H, Dk), 430)
    k_bits = normal_bf16((B, Hk, ctx, Dk), 431)
    v_bits = normal_bf16((B, Hk, ctx, Dv), 432)
    lens = np.array([3000, 1, 0, 1777], np.int32)
    O = torch.empty((B, H, Dv), dtype=torch.bfloat16, device="cuda")
    vm.decode_attention_({"O": O}, to_dev(q_bits), to_dev(k_bits), to_dev(v_bits),
                         lengths=i32(lens), n_splits=n_splits)
    torch.cuda.synchronize()
    ref = orc.attention(bf16_to_f32(q_bits)[:, :, None], bf16_to_f32(k_bits),
                        bf16_to_f32(v_bits), causal=False, k_lengths=lens)[:, :, 0]
    got = dev_f32(O)
    mx, mn = maxmean(got, ref)
    print(f"max {mx:.3e} mean {mn:.3e}")
    assert mx <= TOL_MAX and mn <= TOL_MEAN
    assert not got[2].any()  # no key: O = 0


def test_decode_splits_agree(vm):
    """The generic decode's result does not depend on its split count beyond
    fp32 rounding of the merge."""
    banner("decode_attention_ generic split invariance")
    B, H, Hk, Dk, Dv, ctx = 2, 16, 1, 128, 128, 5000
    q = to_dev(normal_bf16((B, H, Dk), 440))
    k = to_dev(normal_bf16((B, Hk, ctx, Dk), 441))
    v = to_dev(normal_bf16((B, Hk, ctx, Dv), 442))
    lens = i32(np.array([5000, 2049], np.int32))
    outs = []
    for n in (1, 2, 7, 0):
        O = torch.empty((B, H, Dv), dtype=torch.bfloat16, device="cuda")
        vm.decode_attention_({"O": O}, q, k, v, lengths=lens, n_splits=n)
        outs.append(dev_f32(O))
    torch.cuda.synchronize()
    for o in outs[1:]:
        mx, _ = maxmean(o, outs[0])
        assert mx <= 4e-3


# ---------------------------------------------------------------- DeltaNet
def _f32dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


@pytest.mark.parametrize("Dk,Dv,Hk,Hv,inplace", [(64, 64, 4, 8, True), (256, 128, 2, 4, False),
                                                 (128, 256, 2, 2, True), (16, 48, 1, 3, True),
                                                 (192, 64, 1, 2, False)])
def test_fused_deltanet_decode_head_dims(vm, orc, Dk, Dv, Hk, Hv, inplace):
    """fused_deltanet_decode! at head dims other than Dk = Dv = 128
    (deltanet_fused.jl:109-141 tiles any Dk by 16): the generic kernel against
    the oracle, state in place or into a new buffer."""
    from oracle.rng import normal_f32
    banner(f"fused_deltanet_decode Dk={Dk} Dv={Dv} Hk={Hk} Hv={Hv} inplace={inplace}")
    B = 3
    q, k = normal_bf16((B, Hk, Dk), 450), normal_bf16((B, Hk, Dk), 451)
    v, z = normal_bf16((B, Hv, Dv), 452), normal_bf16((B, Hv, Dv), 453)
    ab = normal_bf16((B, 2 * Hv), 454)
    a_log, dt_bias = normal_f32(Hv, 455, scale=0.5), normal_f32(Hv, 456, scale=0.5)
    norm_w = normal_bf16((Dv,), 457, scale=0.2, shift=1.0)
    s = normal_f32(B * Hv * Dv * Dk, 458, scale=0.05).reshape(B, Hv, Dv, Dk)
    o_ref, s_ref = orc.fused_deltanet_decode(q, k, v, ab[:, :Hv], ab[:, Hv:], z, a_log, dt_bias,
                                             norm_w, s, eps=EPS)
    AB = to_dev(ab)
    S = _f32dev(s)
    out = vm.fused_deltanet_decode(to_dev(q), to_dev(k), to_dev(v), AB[:, :Hv], AB[:, Hv:],
                                   to_dev(z), _f32dev(a_log), _f32dev(dt_bias), to_dev(norm_w), S,
                                   eps=EPS, Sp=S if inplace else None)
    torch.cuda.synchronize()
    s_got = (S if inplace else out["Sp"]).cpu().numpy()
    np.testing.assert_allclose(s_got, s_ref, rtol=2e-5, atol=2e-6)
    got = dev_f32(out["O"])
    bar = 2.0 ** -8 * np.abs(o_ref) + 1e-5
    assert np.max(np.abs(got - o_ref) / bar) <= 1.0


@pytest.mark.parametrize("Dk,Dv,Hk,Hv,B,T", [(64, 32, 2, 4, 2, 20), (192, 128, 1, 2, 1, 9),
                                             (32, 256, 2, 2, 3, 5)])
def test_deltanet_sequence_head_dims(vm, orc, Dk, Dv, Hk, Hv, B, T):
    """deltanet_sequence! at other head dims (the generic kernel, state in
    registers across the T steps), in place; T single steps of
    deltanet_recurrent_decode! give the same rows."""
    from oracle.rng import normal_f32
    banner(f"deltanet_sequence Dk={Dk} Dv={Dv} Hk={Hk} Hv={Hv} B={B} T={T}")
    cv = normal_bf16((B, T, 2 * Hk * Dk + Hv * Dv), 460)
    ab = normal_bf16((B, T, 2 * Hv), 461)
    a_log, dt_bias = normal_f32(Hv, 462, scale=0.5), normal_f32(Hv, 463, scale=0.5)
    p = orc.deltanet_prep(cv, ab, a_log, dt_bias, Dk=Dk, Dv=Dv, Hk=Hk, Hv=Hv)
    s = normal_f32(B * Hv * Dv * Dk, 464, scale=0.05).reshape(B, Hv, Dv, Dk)
    o_ref, s_ref = orc.deltanet_sequence(p["q"], p["k"], p["v"], p["beta"], p["gate"], s)
    S = _f32dev(s)
    qd, kd, vd = _f32dev(p["q"]), _f32dev(p["k"]), _f32dev(p["v"])
    bd, gd = _f32dev(p["beta"]), _f32dev(p["gate"])
    out = vm.deltanet_sequence(qd, kd, vd, bd, gd, S, Sp=S)
    S2 = _f32dev(s)
    rows = []
    for t in range(T):
        r = vm.deltanet_recurrent_decode(qd[:, :, t].contiguous(), kd[:, :, t].contiguous(),
                                         vd[:, :, t].contiguous(), bd[:, t].contiguous(),
                                         gd[:, t].contiguous(), S2, Sp=S2)
        rows.append(r["O"])
    torch.cuda.synchronize()
    np.testing.assert_allclose(S.cpu().numpy(), s_ref, rtol=5e-4, atol=5e-5)
    np.testing.assert_allclose(out["O"].cpu().numpy(), o_ref, rtol=5e-4, atol=5e-5)
    assert torch.equal(S2, S)
    assert torch.equal(torch.stack(rows, 2), out["O"])
