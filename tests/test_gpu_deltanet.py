"""The linear-attention layer parts on the GPU vs the CPU oracle (oracle/deltanet.c):
causal_conv1d! and causal_conv1d_sequence! (src/kernels/causal_conv1d.jl),
fused_deltanet_decode! (deltanet_fused.jl), deltanet_recurrent_decode! and
deltanet_sequence! (deltanet_recurrent.jl), and the prefill's prep and gated
RMSNorm (src/llm/qwen35.jl:347-364), at the Qwen3.5 DeltaNet shape (Dk = Dv =
128, Hk = 16, Hv = 32, conv kernel 4, 8192 conv channels) and at odd sizes.

Bars: the conv ring (raw bf16 inputs) bit-exact; fp32 states and outputs
within rtol 2e-5 of the oracle per step (5e-4 after 64 steps); bf16 outputs
within one bf16 ulp of the fp32 oracle plus fp32 reassociation."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import banner, dev_f32, from_dev, to_dev
from oracle.rng import bf16_to_f32, f32_to_bf16, normal_bf16, normal_f32

pytestmark = pytest.mark.gpu

DK = DV = 128
HK, HV, KC = 16, 32, 4
NCH = 2 * HK * DK + HV * DV  # conv channels q | k | v
EPS = 1e-6


def f32dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def bf16_bar(ref, extra=0.0):
    """One bf16 ulp of the fp32 reference (2^-8 relative) plus an absolute floor."""
    return 2.0 ** -8 * np.abs(ref) + 1e-6 + extra


def assert_bf16_close(got, ref, what, extra=0.0):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    worst = float(np.max(np.abs(got - ref) / bf16_bar(ref, extra)))
    print(f"{what}: worst |err| / bar = {worst:.3f}")
    assert worst <= 1.0, what


# ---------------------------------------------------------------- conv1d
@pytest.mark.parametrize("B,bias,act", [(1, True, True), (3, False, True), (5, True, False)])
def test_conv1d_update(vm, orc, B, bias, act):
    """One decode step on the in-place ring; X a strided view (the q | k | v rows
    of the projection, token stride NCH + HV * DV)."""
    banner(f"conv1d update B={B} bias={bias} act={act}")
    qz = normal_bf16((B, NCH + HV * DV), 900 + B)
    ring = normal_bf16((B, KC, NCH), 901 + B)
    w = normal_bf16((KC, NCH), 902, scale=0.5)
    b = normal_bf16((NCH,), 903, scale=0.1) if bias else None
    y_ref, ring_ref = orc.conv1d_update(qz[:, :NCH], ring, w, b, act=act)
    X = to_dev(qz)[:, :NCH]
    S = to_dev(ring)
    out = vm.causal_conv1d(X, S, to_dev(w), None if b is None else to_dev(b),
                           sigma="silu" if act else None, Sp=S)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(S), ring_ref)
    assert_bf16_close(dev_f32(out["Y"]), y_ref, "conv1d update")


def _narrow_bar(x, W, ref):
    """One bf16 ulp (2^-8 |y|) plus fp32 reassociation (2^-20 sum_k |x_k w_k|)."""
    xa = np.abs(bf16_to_f32(x).astype(np.float64))
    wa = np.abs(bf16_to_f32(W).astype(np.float64))
    return 2.0 ** -8 * np.abs(ref) + 2.0 ** -20 * (xa @ wa.T) + 1e-30


@pytest.mark.parametrize("B,Kdim,bias", [(32, 2560, False), (1, 2560, True), (5, 640, True),
                                         (40, 256, False)])
def test_linear_causal_conv1d(vm, orc, B, Kdim, bias):
    """linear! + causal_conv1d! in one call (the DeltaNet layer's decode step,
    qwen35.jl:212-223) at the Qwen3.5 shape: W_in 12352 x K, the conv on the first
    8192 channels, the ring in place. The projection within one bf16 ulp plus
    fp32 reassociation of the oracle's; the conv output and ring equal to the
    oracle's conv step on that bf16 projection (bit-exact ring); a second call
    from the same ring bitwise equal. B = 40 is linear! + causal_conv1d!."""
    banner(f"linear_causal_conv1d B={B} K={Kdim} bias={bias}")
    M = NCH + HV * DV + 2 * HV
    x = normal_bf16((B, Kdim), 940 + B)
    W = normal_bf16((M, Kdim), 941, scale=Kdim ** -0.5)
    ring = normal_bf16((B, KC, NCH), 942 + B)
    w = normal_bf16((KC, NCH), 943, scale=0.5)
    b = normal_bf16((NCH,), 944, scale=0.1) if bias else None
    xd, Wd, wd = to_dev(x), to_dev(W), to_dev(w)
    bd = None if b is None else to_dev(b)
    outs = []
    for _ in range(2):
        S = to_dev(ring)
        y = torch.empty((B, M), dtype=torch.bfloat16, device="cuda")
        Y = torch.empty((B, NCH), dtype=torch.bfloat16, device="cuda")
        vm.linear_causal_conv1d_({"y": y, "Y": Y, "Sp": S}, xd, Wd, S, wd, bd, sigma="silu")
        outs.append((y, Y, S))
    torch.cuda.synchronize()
    y, Y, S = outs[0]
    ref = orc.linear(x, W).astype(np.float64)
    got = dev_f32(y).astype(np.float64)
    worst = float(np.max(np.abs(got - ref) / _narrow_bar(x, W, ref)))
    print(f"projection: worst |err| / bar = {worst:.3f}")
    assert worst <= 1.0
    yb = from_dev(y)
    y_ref, ring_ref = orc.conv1d_update(yb[:, :NCH], ring, w, b, act=True)
    assert np.array_equal(from_dev(S), ring_ref)
    assert_bf16_close(dev_f32(Y), y_ref, "conv of the projection")
    for t0, t1 in zip(outs[0], outs[1]):
        assert torch.equal(t0.view(torch.int16), t1.view(torch.int16))


def test_conv1d_update_chain_equals_sequence(vm, orc):
    """T decode steps from a zero ring == one sequence run (rows and ring)."""
    banner("conv1d update chain == sequence")
    B, T, D = 2, 9, 512
    x = normal_bf16((B, T, D), 910)
    w = normal_bf16((KC, D), 911, scale=0.5)
    b = normal_bf16((D,), 912, scale=0.1)
    X, W, Bi = to_dev(x), to_dev(w), to_dev(b)
    seq = vm.causal_conv1d_sequence(X, W, Bi, sigma="silu",
                                    Sp=torch.zeros((B, KC, D), dtype=torch.bfloat16,
                                                   device="cuda"))
    S = torch.zeros((B, KC, D), dtype=torch.bfloat16, device="cuda")
    rows = []
    for t in range(T):
        rows.append(vm.causal_conv1d(X[:, t], S, W, Bi, sigma="silu", Sp=S)["Y"])
    torch.cuda.synchronize()
    y_ref, ring_ref = orc.conv1d_sequence(x, w, b, act=True)
    assert_bf16_close(dev_f32(seq["Y"]), y_ref, "sequence")
    assert_bf16_close(dev_f32(torch.stack(rows, 1)), y_ref, "update chain")
    assert np.array_equal(from_dev(S), ring_ref)


@pytest.mark.parametrize("B,T,prefix,bias", [(1, 37, False, True), (2, 16, False, False),
                                             (2, 3, True, True), (3, 50, True, False),
                                             (1, 1, True, True)])
def test_conv1d_sequence(vm, orc, B, T, prefix, bias):
    """The whole-sequence conv over a strided X, with the seeded ring; with a
    prefix ring (the suffix prefill) read and overwritten in place."""
    banner(f"conv1d sequence B={B} T={T} prefix={prefix} bias={bias}")
    qz = normal_bf16((B, T, NCH + HV * DV), 920 + T)
    x = np.ascontiguousarray(qz[..., :NCH])
    w = normal_bf16((KC, NCH), 921, scale=0.5)
    b = normal_bf16((NCH,), 922, scale=0.1) if bias else None
    ring0 = normal_bf16((B, KC, NCH), 923) if prefix else None
    y_ref, ring_ref = orc.conv1d_sequence(x, w, b, s_in=ring0, act=True)
    X = to_dev(qz)[..., :NCH]
    S = to_dev(ring0) if prefix else torch.empty((B, KC, NCH), dtype=torch.bfloat16,
                                                  device="cuda")
    out = vm.causal_conv1d_sequence(X, to_dev(w), None if b is None else to_dev(b),
                                    sigma="silu", Sp=S, S=S if prefix else None)
    torch.cuda.synchronize()
    assert_bf16_close(dev_f32(out["Y"]), y_ref, "conv1d sequence")
    assert np.array_equal(from_dev(S), ring_ref)


# ---------------------------------------------------------------- delta rule
def _fused_inputs(B, seed):
    qz = normal_bf16((B, NCH + HV * DV), seed)  # conv output rows (q | k | v) + z
    ab = normal_bf16((B, 2 * HV), seed + 1)
    a_log = normal_f32(HV, seed + 2, scale=0.5)
    dt_bias = normal_f32(HV, seed + 3, scale=0.5)
    norm_w = normal_bf16((DV,), seed + 4, scale=0.2, shift=1.0)
    s = normal_f32(B * HV * DV * DK, seed + 5, scale=0.05).reshape(B, HV, DV, DK)
    return qz, ab, a_log, dt_bias, norm_w, s


def _split(qz):
    q = qz[..., :HK * DK]
    k = qz[..., HK * DK:2 * HK * DK]
    v = qz[..., 2 * HK * DK:NCH]
    z = qz[..., NCH:]
    return q, k, v, z


@pytest.mark.parametrize("B,inplace", [(1, True), (4, False), (32, True), (33, True)])
def test_fused_deltanet_decode(vm, orc, B, inplace):
    """The layer's decode step: q, k, v, z, alpha, beta as strided views of the
    projection outputs, the state updated in place or into a new buffer."""
    banner(f"fused deltanet decode B={B} inplace={inplace}")
    qz, ab, a_log, dt_bias, norm_w, s = _fused_inputs(B, 930 + B)
    q, k, v, z = _split(qz)
    o_ref, s_ref = orc.fused_deltanet_decode(
        q.reshape(B, HK, DK), k.reshape(B, HK, DK), v.reshape(B, HV, DV), ab[:, :HV], ab[:, HV:],
        z.reshape(B, HV, DV), a_log, dt_bias, norm_w, s, eps=EPS)
    QZ, AB = to_dev(qz), to_dev(ab)
    Qd, Kd, Vd, Zd = (t.unflatten(-1, (-1, DK)) for t in _split(QZ))
    S = f32dev(s)
    out = vm.fused_deltanet_decode(Qd, Kd, Vd, AB[:, :HV], AB[:, HV:], Zd, f32dev(a_log),
                                   f32dev(dt_bias), to_dev(norm_w), S, eps=EPS,
                                   Sp=S if inplace else None)
    torch.cuda.synchronize()
    s_got = (S if inplace else out["Sp"]).cpu().numpy()
    np.testing.assert_allclose(s_got, s_ref, rtol=2e-5, atol=2e-6)
    assert_bf16_close(dev_f32(out["O"]), o_ref, "fused decode O", extra=1e-5)


@pytest.mark.parametrize("B,hk,hv,bias", [(32, HK, HV, False), (1, HK, HV, True),
                                           (5, 16, 16, True), (3, 8, 32, False),
                                           (40, HK, HV, True)])
def test_linear_deltanet_decode(vm, orc, B, hk, hv, bias):
    """The DeltaNet layer's decode step up to its out projection in one call
    (qwen35.jl:212-232): O, the state and the ring bit for bit equal to
    linear_causal_conv1d_ followed by fused_deltanet_decode_ on the same inputs,
    for Hv / Hk = 2, 1, 4 (one kernel per (qk head, sequence) at B <= 32; B = 40
    runs the two calls); O and the state also within the bars of the oracle's
    conv step and fused decode on the two-call path's bf16 projection. Two steps
    in a row from the in-place ring and state."""
    banner(f"linear_deltanet_decode B={B} Hk={hk} Hv={hv} bias={bias}")
    Kdim = 640
    nch = 2 * hk * DK + hv * DV
    M = nch + hv * DV + 2 * hv
    x = normal_bf16((2, B, Kdim), 960 + B)
    W = normal_bf16((M, Kdim), 961, scale=Kdim ** -0.5)
    ring = normal_bf16((B, KC, nch), 962 + B)
    w = normal_bf16((KC, nch), 963, scale=0.5)
    b = normal_bf16((nch,), 964, scale=0.1) if bias else None
    a_log = normal_f32(hv, 965, scale=0.5)
    dt_bias = normal_f32(hv, 966, scale=0.5)
    norm_w = normal_bf16((DV,), 967, scale=0.2, shift=1.0)
    s = normal_f32(B * hv * DV * DK, 968, scale=0.05).reshape(B, hv, DV, DK)
    Wd, wd, nd = to_dev(W), to_dev(w), to_dev(norm_w)
    bd = None if b is None else to_dev(b)
    al, dt = f32dev(a_log), f32dev(dt_bias)
    m = nch + hv * DV

    def two_calls():
        S_ring, S = to_dev(ring), f32dev(s)
        y = torch.empty((B, M), dtype=torch.bfloat16, device="cuda")
        Y = torch.empty((B, nch), dtype=torch.bfloat16, device="cuda")
        O = torch.empty((B, hv, DV), dtype=torch.bfloat16, device="cuda")
        ys, Os = [], []
        for t in range(2):
            vm.linear_causal_conv1d_({"y": y, "Y": Y, "Sp": S_ring}, to_dev(x[t]), Wd, S_ring,
                                     wd, bd, sigma="silu")
            q = Y[:, :hk * DK].unflatten(-1, (hk, DK))
            k = Y[:, hk * DK:2 * hk * DK].unflatten(-1, (hk, DK))
            v = Y[:, 2 * hk * DK:].unflatten(-1, (hv, DV))
            z = y[:, nch:m].unflatten(-1, (hv, DV))
            vm.fused_deltanet_decode_({"O": O, "Sp": S}, q, k, v, y[:, m:m + hv],
                                      y[:, m + hv:], z, al, dt, nd, S, eps=EPS)
            ys.append((y.clone(), Y.clone()))
            Os.append(O.clone())
        return Os, S, S_ring, ys

    def one_call():
        S_ring, S = to_dev(ring), f32dev(s)
        y = torch.empty((B, M), dtype=torch.bfloat16, device="cuda")
        Y = torch.empty((B, nch), dtype=torch.bfloat16, device="cuda")
        O = torch.empty((B, hv, DV), dtype=torch.bfloat16, device="cuda")
        Os = []
        for t in range(2):
            vm.linear_deltanet_decode_({"O": O, "y": y, "Y": Y, "Sp_ring": S_ring, "Sp": S},
                                       to_dev(x[t]), Wd, S_ring, wd, bd, al, dt, nd, S, Dk=DK,
                                       Dv=DV, Hk=hk, Hv=hv, eps=EPS)
            Os.append(O.clone())
        return Os, S, S_ring

    O2, S2, R2, ys = two_calls()
    O1, S1, R1 = one_call()
    torch.cuda.synchronize()
    for t in range(2):
        assert torch.equal(O1[t].view(torch.int16), O2[t].view(torch.int16)), f"O step {t}"
    assert torch.equal(S1, S2)
    assert torch.equal(R1.view(torch.int16), R2.view(torch.int16))
    # the first step against the oracle's fused decode on the two-call path's
    # bf16 projection and conv output (those two are pinned by
    # test_linear_causal_conv1d)
    yb, cv = from_dev(ys[0][0]), from_dev(ys[0][1])
    o_ref, s_ref = orc.fused_deltanet_decode(
        cv[:, :hk * DK].reshape(B, hk, DK), cv[:, hk * DK:2 * hk * DK].reshape(B, hk, DK),
        cv[:, 2 * hk * DK:].reshape(B, hv, DV), yb[:, m:m + hv], yb[:, m + hv:],
        yb[:, nch:m].reshape(B, hv, DV), a_log, dt_bias, norm_w, s, eps=EPS)
    assert_bf16_close(dev_f32(O1[0]), o_ref, "one-call decode O", extra=1e-5)
    if B == 1:
        s1 = f32dev(s)
        vm.linear_deltanet_decode_({"O": O1[0], "y": ys[0][0], "Y": ys[0][1], "Sp_ring": R1,
                                    "Sp": s1}, to_dev(x[0]), Wd, to_dev(ring), wd, bd, al, dt, nd,
                                   f32dev(s), Dk=DK, Dv=DV, Hk=hk, Hv=hv, eps=EPS)
        torch.cuda.synchronize()
        np.testing.assert_allclose(s1.cpu().numpy(), s_ref, rtol=2e-5, atol=2e-6)


def _prepped(B, T, seed):
    cv = normal_bf16((B, T, NCH), seed)
    ab = normal_bf16((B, T, 2 * HV), seed + 1)
    a_log = normal_f32(HV, seed + 2, scale=0.5)
    dt_bias = normal_f32(HV, seed + 3, scale=0.5)
    return cv, ab, a_log, dt_bias


@pytest.mark.parametrize("B,T", [(1, 64), (2, 17), (16, 4), (17, 3)])
def test_deltanet_sequence(vm, orc, B, T):
    """deltanet_sequence! on the prefill's prepped inputs: both launch shapes
    (16 waves per head for B * Hv < 512, 4 above), in place."""
    banner(f"deltanet sequence B={B} T={T}")
    cv, ab, a_log, dt_bias = _prepped(B, T, 950 + B + T)
    p = orc.deltanet_prep(cv, ab, a_log, dt_bias, Dk=DK, Dv=DV, Hk=HK, Hv=HV)
    s = normal_f32(B * HV * DV * DK, 951, scale=0.05).reshape(B, HV, DV, DK)
    o_ref, s_ref = orc.deltanet_sequence(p["q"], p["k"], p["v"], p["beta"], p["gate"], s)
    S = f32dev(s)
    out = vm.deltanet_sequence(f32dev(p["q"]), f32dev(p["k"]), f32dev(p["v"]), f32dev(p["beta"]),
                               f32dev(p["gate"]), S, Sp=S)
    torch.cuda.synchronize()
    tol = 2e-5 if T <= 4 else 5e-4
    np.testing.assert_allclose(S.cpu().numpy(), s_ref, rtol=tol, atol=tol * 0.1)
    np.testing.assert_allclose(out["O"].cpu().numpy(), o_ref, rtol=tol, atol=tol * 0.1)


def test_deltanet_recurrent_decode_chain(vm, orc):
    """deltanet_recurrent_decode!: T single steps == the sequence run's rows."""
    banner("deltanet recurrent decode chain")
    B, T = 3, 5
    cv, ab, a_log, dt_bias = _prepped(B, T, 960)
    p = orc.deltanet_prep(cv, ab, a_log, dt_bias, Dk=DK, Dv=DV, Hk=HK, Hv=HV)
    s = normal_f32(B * HV * DV * DK, 961, scale=0.05).reshape(B, HV, DV, DK)
    o_ref, s_ref = orc.deltanet_sequence(p["q"], p["k"], p["v"], p["beta"], p["gate"], s)
    S = f32dev(s)
    for t in range(T):
        o = vm.deltanet_recurrent_decode(
            f32dev(p["q"][:, :, t]), f32dev(p["k"][:, :, t]), f32dev(p["v"][:, :, t]),
            f32dev(p["beta"][:, t]), f32dev(p["gate"][:, t]), S, Sp=S)["O"]
        np.testing.assert_allclose(o.cpu().numpy(), o_ref[:, :, t], rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(S.cpu().numpy(), s_ref, rtol=1e-4, atol=1e-5)


def test_deltanet_sequence_zero_length_copies_state(vm):
    banner("deltanet sequence T=0")
    B = 2
    s = normal_f32(B * HV * DV * DK, 970).reshape(B, HV, DV, DK)
    e = torch.empty((B, HK, 0, DK), dtype=torch.float32, device="cuda")
    ev = torch.empty((B, HV, 0, DV), dtype=torch.float32, device="cuda")
    g = torch.empty((B, 0, HV), dtype=torch.float32, device="cuda")
    out = vm.deltanet_sequence(e, e, ev, g, g, f32dev(s))
    torch.cuda.synchronize()
    assert np.array_equal(out["Sp"].cpu().numpy(), s)


@pytest.mark.parametrize("off", [0, 4])
def test_prep_and_gated_norm(vm, orc, off):
    """The prefill's prep from strided conv rows and its gated-norm epilogue
    reading z from the projection. off = 0: 16-byte aligned rows (the vectorised
    kernels); off = 4: rows 8-byte aligned only (the one-wave-per-head kernels)."""
    banner(f"deltanet prep + gated norm, rows at element offset {off}")
    B, T = 2, 7
    cv, ab, a_log, dt_bias = _prepped(B, T, 980)
    p_ref = orc.deltanet_prep(cv, ab, a_log, dt_bias, Dk=DK, Dv=DV, Hk=HK, Hv=HV)
    wide = np.zeros((B, T, NCH + 64), np.uint16)
    wide[..., off:off + NCH] = cv
    CV = to_dev(wide)[..., off:off + NCH]
    outs = {"Q": torch.empty((B, HK, T, DK), dtype=torch.float32, device="cuda"),
            "K": torch.empty((B, HK, T, DK), dtype=torch.float32, device="cuda"),
            "V": torch.empty((B, HV, T, DV), dtype=torch.float32, device="cuda"),
            "Beta": torch.empty((B, T, HV), dtype=torch.float32, device="cuda"),
            "Gate": torch.empty((B, T, HV), dtype=torch.float32, device="cuda")}
    vm.deltanet_prefill_prep_(outs, CV, to_dev(ab), f32dev(a_log), f32dev(dt_bias), Dk=DK,
                              Dv=DV, Hk=HK, Hv=HV)
    torch.cuda.synchronize()
    for key, rk in (("Q", "q"), ("K", "k"), ("V", "v"), ("Beta", "beta"), ("Gate", "gate")):
        np.testing.assert_allclose(outs[key].cpu().numpy(), p_ref[rk], rtol=2e-6, atol=1e-7,
                                   err_msg=key)
    o = normal_f32(B * HV * T * DV, 981).reshape(B, HV, T, DV)
    qz = normal_bf16((B, T, NCH + off + HV * DV), 982)
    norm_w = normal_bf16((DV,), 983, scale=0.2, shift=1.0)
    y_ref = orc.gated_rms_norm(o, np.ascontiguousarray(qz[..., NCH + off:]), norm_w, eps=EPS)
    Z = to_dev(qz)[..., NCH + off:].unflatten(-1, (HV, DV))
    Yw = torch.empty((B, T, HV * DV + off), dtype=torch.bfloat16, device="cuda")
    Y = Yw[..., off:].unflatten(-1, (HV, DV))
    vm.gated_rms_norm_(Y, f32dev(o), Z, to_dev(norm_w), eps=EPS)
    torch.cuda.synchronize()
    assert_bf16_close(dev_f32(Y), y_ref, "gated norm", extra=1e-6)


@pytest.mark.parametrize("B,T,prefix,bias,hk,hv", [(1, 37, False, True, HK, HV),
                                                   (2, 16, True, False, HK, HV),
                                                   (3, 5, True, True, HK, HV),
                                                   (1, 100, False, False, HK, HV),
                                                   (2, 33, True, True, 2, 6)])
def test_deltanet_conv_prep(vm, orc, B, T, prefix, bias, hk, hv):
    """The prefill's conv and prep in one pass equal, bit for bit, the conv
    (silu) followed by the prep on the GPU, from strided projection rows, with
    and without a prefix ring; the prep of the conv's output also against the
    oracle's, and the ring against the oracle's."""
    banner(f"deltanet conv + prep B={B} T={T} prefix={prefix} bias={bias} Hk={hk} Hv={hv}")
    nch = 2 * hk * DK + hv * DV
    qz = normal_bf16((B, T, nch + hv * DV), 1990 + T)  # q | k | v | z projection rows
    abw = normal_bf16((B, T, 2 * hv + 8), 1991)
    w = normal_bf16((KC, nch), 1992, scale=0.5)
    b = normal_bf16((nch,), 1993, scale=0.1) if bias else None
    ring0 = normal_bf16((B, KC, nch), 1994) if prefix else None
    a_log = normal_f32(hv, 1995, scale=0.5)
    dt_bias = normal_f32(hv, 1996, scale=0.5)
    X = to_dev(qz)[..., :nch]
    AB = to_dev(abw)[..., 4:4 + 2 * hv]
    W, Bb = to_dev(w), (None if b is None else to_dev(b))
    A, Dt = f32dev(a_log), f32dev(dt_bias)

    def outs():
        f = dict(dtype=torch.float32, device="cuda")
        return {"Q": torch.empty((B, hk, T, DK), **f), "K": torch.empty((B, hk, T, DK), **f),
                "V": torch.empty((B, hv, T, DV), **f), "Beta": torch.empty((B, T, hv), **f),
                "Gate": torch.empty((B, T, hv), **f)}

    def ring():
        return to_dev(ring0) if prefix else torch.zeros((B, KC, nch), dtype=torch.bfloat16,
                                                         device="cuda")
    S1, S2 = ring(), ring()
    conv = vm.causal_conv1d_sequence(X, W, Bb, sigma="silu", Sp=S1, S=S1 if prefix else None)["Y"]
    two = outs()
    vm.deltanet_prefill_prep_(two, conv, AB, A, Dt, Dk=DK, Dv=DV, Hk=hk, Hv=hv)
    one = outs()
    vm.deltanet_conv_prep_(one, X, W, AB, A, Dt, Bb, Dk=DK, Dv=DV, Hk=hk, Hv=hv, Sp=S2,
                           S=S2 if prefix else None)
    torch.cuda.synchronize()
    for key in ("Q", "K", "V", "Beta", "Gate"):
        assert torch.equal(one[key], two[key]), key
    assert torch.equal(S1, S2)
    _, ring_ref = orc.conv1d_sequence(np.ascontiguousarray(qz[..., :nch]), w, b, s_in=ring0,
                                      act=True)
    assert np.array_equal(from_dev(S2), ring_ref)
    p_ref = orc.deltanet_prep(from_dev(conv), np.ascontiguousarray(abw[..., 4:4 + 2 * hv]),
                              a_log, dt_bias, Dk=DK, Dv=DV, Hk=hk, Hv=hv)
    for key, rk in (("Q", "q"), ("K", "k"), ("V", "v"), ("Beta", "beta"), ("Gate", "gate")):
        np.testing.assert_allclose(one[key].cpu().numpy(), p_ref[rk], rtol=2e-6, atol=1e-7,
                                   err_msg=key)


def test_prep_many_value_heads(vm, orc):
    """The prep with more value heads than a wave has lanes (Hk = 2, Hv = 72): the
    gates of heads 64 .. 71 too."""
    banner("deltanet prep, Hv = 72")
    B, T, hk, hv = 1, 3, 2, 72
    n = 2 * hk * DK + hv * DV
    cv = normal_bf16((B, T, n), 990)
    ab = normal_bf16((B, T, 2 * hv), 991)
    a_log = normal_f32(hv, 992, scale=0.5)
    dt_bias = normal_f32(hv, 993, scale=0.5)
    ref = orc.deltanet_prep(cv, ab, a_log, dt_bias, Dk=DK, Dv=DV, Hk=hk, Hv=hv)
    outs = {"Q": torch.empty((B, hk, T, DK), dtype=torch.float32, device="cuda"),
            "K": torch.empty((B, hk, T, DK), dtype=torch.float32, device="cuda"),
            "V": torch.empty((B, hv, T, DV), dtype=torch.float32, device="cuda"),
            "Beta": torch.empty((B, T, hv), dtype=torch.float32, device="cuda"),
            "Gate": torch.empty((B, T, hv), dtype=torch.float32, device="cuda")}
    vm.deltanet_prefill_prep_(outs, to_dev(cv), to_dev(ab), f32dev(a_log), f32dev(dt_bias), Dk=DK,
                              Dv=DV, Hk=hk, Hv=hv)
    torch.cuda.synchronize()
    for key, rk in (("Q", "q"), ("K", "k"), ("V", "v"), ("Beta", "beta"), ("Gate", "gate")):
        np.testing.assert_allclose(outs[key].cpu().numpy(), ref[rk], rtol=2e-6, atol=1e-7,
                                   err_msg=key)


def test_shape_errors(vm):
    """The reference's DimensionMismatch on Hv % Hk, and head sizes no kernel
    takes (Dk a multiple of 16 up to 256, deltanet_recurrent.jl:86 tiles by 16);
    checked before any launch."""
    banner("deltanet shape errors")
    B = 1
    S = torch.zeros((B, 6, DV, DK), dtype=torch.float32, device="cuda")
    q = torch.zeros((B, 4, DK), dtype=torch.float32, device="cuda")
    v = torch.zeros((B, 6, DV), dtype=torch.float32, device="cuda")
    g = torch.zeros((B, 6), dtype=torch.float32, device="cuda")
    with pytest.raises(vm.DimensionMismatch):
        vm.deltanet_recurrent_decode(q, q, v, g, g, S)
    g2 = torch.zeros((B, 2), dtype=torch.float32, device="cuda")
    for dk in (24, 320):
        Sx = torch.zeros((B, 2, 64, dk), dtype=torch.float32, device="cuda")
        qx = torch.zeros((B, 1, dk), dtype=torch.float32, device="cuda")
        vx = torch.zeros((B, 2, 64), dtype=torch.float32, device="cuda")
        with pytest.raises(vm.UnsupportedShape):
            vm.deltanet_recurrent_decode(qx, qx, vx, g2, g2, Sx)


@pytest.mark.parametrize("B,T", [(1, 1), (1, 63), (1, 64), (2, 65), (1, 200), (17, 70),
                                 (1, 1000)])
def test_deltanet_sequence_chunked(vm, orc, B, T):
    """deltanet_sequence! in its chunked form (triangular solve + fp32 MFMA per
    64-token chunk, one scan over chunks) against the sequential oracle: every
    output and the final state within rtol 5e-4 (chunk edges, partial last
    chunks, B > 1, the state updated in place)."""
    banner(f"deltanet sequence chunked B={B} T={T}")
    cv, ab, a_log, dt_bias = _prepped(B, T, 1950 + B + T)
    p = orc.deltanet_prep(cv, ab, a_log, dt_bias, Dk=DK, Dv=DV, Hk=HK, Hv=HV)
    s = normal_f32(B * HV * DV * DK, 1951, scale=0.05).reshape(B, HV, DV, DK)
    o_ref, s_ref = orc.deltanet_sequence(p["q"], p["k"], p["v"], p["beta"], p["gate"], s)
    S = f32dev(s)
    o = torch.empty((B, HV, T, DV), dtype=torch.float32, device="cuda")
    ws = torch.full((vm.deltanet_sequence_workspace_bytes(T, HV, B),), 255, dtype=torch.uint8,
                    device="cuda")   # garbage: every byte read is written first
    vm.deltanet_sequence_chunked_({"O": o, "Sp": S}, f32dev(p["q"]), f32dev(p["k"]),
                                  f32dev(p["v"]), f32dev(p["beta"]), f32dev(p["gate"]), S,
                                  workspace=ws)
    torch.cuda.synchronize()
    for got, ref, name in ((o.cpu().numpy(), o_ref, "O"), (S.cpu().numpy(), s_ref, "S")):
        err = np.abs(got - ref).max() / np.abs(ref).max()
        print(f"chunked {name}: max err / max |ref| = {err:.2e}")
        assert err <= 5e-4, name


@pytest.mark.parametrize("B,T,off", [(1, 100, 0), (2, 65, 8), (1, 1, 0), (3, 129, 0)])
def test_deltanet_sequence_chunked_gated_norm(vm, orc, B, T, off):
    """forward(::DeltaNetLayer)'s recurrence and gated norm as one call
    (qwen35.jl:357-364): y = O rstd NormWeight silu(z) formed where each chunk's
    O is. The output kernel forms O the same way with or without the norm, so y
    is checked against the oracle's gated norm of the unfused call's O (itself
    checked against the sequential oracle), to one bf16 ulp; z is read from the
    projection's rows, y written as a strided view, the state updated in place
    and equal to the unfused call's bit for bit."""
    banner(f"deltanet chunked + gated norm B={B} T={T} off={off}")
    cv, ab, a_log, dt_bias = _prepped(B, T, 2950 + B + T)
    p = orc.deltanet_prep(cv, ab, a_log, dt_bias, Dk=DK, Dv=DV, Hk=HK, Hv=HV)
    s = normal_f32(B * HV * DV * DK, 2951, scale=0.05).reshape(B, HV, DV, DK)
    o_ref, s_ref = orc.deltanet_sequence(p["q"], p["k"], p["v"], p["beta"], p["gate"], s)
    args = [f32dev(p[n]) for n in ("q", "k", "v", "beta", "gate")]
    S1 = f32dev(s)
    o = torch.empty((B, HV, T, DV), dtype=torch.float32, device="cuda")
    vm.deltanet_sequence_chunked_({"O": o, "Sp": S1}, *args, S1)
    qz = normal_bf16((B, T, NCH + HV * DV), 2952)
    norm_w = normal_bf16((DV,), 2953, scale=0.2, shift=1.0)
    Z = to_dev(qz)[..., NCH:].unflatten(-1, (HV, DV))
    Yw = torch.full((B, T, HV * DV + off), 5.0, dtype=torch.bfloat16, device="cuda")
    Y = Yw[..., off:].unflatten(-1, (HV, DV))
    S2 = f32dev(s)
    vm.deltanet_sequence_chunked_gated_norm_({"Y": Y, "Sp": S2}, Z, to_dev(norm_w), *args, S2,
                                             eps=EPS)
    torch.cuda.synchronize()
    og = o.cpu().numpy()
    err = np.abs(og - o_ref).max() / np.abs(o_ref).max()
    print(f"unfused O: max err / max |ref| = {err:.2e}")
    assert err <= 5e-4
    y_ref = orc.gated_rms_norm(og, np.ascontiguousarray(qz[..., NCH:]), norm_w, eps=EPS)
    assert_bf16_close(dev_f32(Y), y_ref, "gated y", extra=1e-6)
    if off:
        assert bool((Yw[..., :off] == 5.0).all())
    assert torch.equal(S1, S2)
    err = np.abs(S2.cpu().numpy() - s_ref).max() / np.abs(s_ref).max()
    print(f"chunked + norm S: max err / max |ref| = {err:.2e}")
    assert err <= 5e-4


def test_deltanet_sequence_chunked_overflowing_softplus(vm, orc):
    """A gate input past softplus' fp32 overflow (alpha + dt_bias > 88.7: the
    prep's log1p(exp(x)) is +inf, the log decay -inf, the decay exactly 0, as in
    the reference's prefill, qwen35.jl:30, :354) in the middle of a chunk: the
    chunked form still matches the sequential oracle, with no NaN in O or the
    carried state (tokens before it stop contributing; those after it do)."""
    banner("deltanet chunked with an overflowing softplus")
    B, T = 1, 100
    cv, ab, a_log, dt_bias = _prepped(B, T, 1970)
    # alpha of value head 3 at token 37 (chunk 0) and of head 9 at token 70 (chunk 1)
    big = f32_to_bf16(np.array([200.0], np.float32))[0]
    ab = ab.copy()
    ab[0, 37, 3] = big
    ab[0, 70, 9] = big
    p = orc.deltanet_prep(cv, ab, a_log, dt_bias, Dk=DK, Dv=DV, Hk=HK, Hv=HV)
    assert np.isneginf(p["gate"][0, 37, 3]) and np.isneginf(p["gate"][0, 70, 9])
    s = normal_f32(B * HV * DV * DK, 1971, scale=0.05).reshape(B, HV, DV, DK)
    o_ref, s_ref = orc.deltanet_sequence(p["q"], p["k"], p["v"], p["beta"], p["gate"], s)
    assert np.isfinite(o_ref).all() and np.isfinite(s_ref).all()
    S = f32dev(s)
    o = torch.empty((B, HV, T, DV), dtype=torch.float32, device="cuda")
    vm.deltanet_sequence_chunked_({"O": o, "Sp": S}, f32dev(p["q"]), f32dev(p["k"]),
                                  f32dev(p["v"]), f32dev(p["beta"]), f32dev(p["gate"]), S)
    torch.cuda.synchronize()
    for got, ref, name in ((o.cpu().numpy(), o_ref, "O"), (S.cpu().numpy(), s_ref, "S")):
        assert np.isfinite(got).all(), name
        err = np.abs(got - ref).max() / np.abs(ref).max()
        print(f"chunked {name} with -inf log decays: max err / max |ref| = {err:.2e}")
        assert err <= 5e-4, name


def test_deltanet_sequence_chunked_equals_sequential_at_4096(vm):
    """At the prefill size (T = 4096, B = 1) the chunked and the sequential
    kernels agree: outputs and final state within 1e-3 of their maxima."""
    banner("deltanet sequence chunked vs sequential T=4096")
    B, T = 1, 4096
    f32 = dict(dtype=torch.float32, device="cuda")
    cv = torch.empty((B, T, NCH), dtype=torch.bfloat16, device="cuda")
    vm.fill_normal_(cv, 1960)
    ab = torch.empty((B, T, 2 * HV), dtype=torch.bfloat16, device="cuda")
    vm.fill_normal_(ab, 1961)
    p = {"Q": torch.empty((B, HK, T, DK), **f32), "K": torch.empty((B, HK, T, DK), **f32),
         "V": torch.empty((B, HV, T, DV), **f32), "Beta": torch.empty((B, T, HV), **f32),
         "Gate": torch.empty((B, T, HV), **f32)}
    vm.deltanet_prefill_prep_(p, cv, ab, f32dev(normal_f32(HV, 1962, scale=0.5)),
                              f32dev(normal_f32(HV, 1963, scale=0.5)), Dk=DK, Dv=DV, Hk=HK, Hv=HV)
    S0 = torch.randn((B, HV, DV, DK), **f32) * 0.05
    seq = vm.deltanet_sequence(p["Q"], p["K"], p["V"], p["Beta"], p["Gate"], S0)
    chk = {"O": torch.empty_like(seq["O"]), "Sp": torch.empty_like(S0)}
    vm.deltanet_sequence_chunked_(chk, p["Q"], p["K"], p["V"], p["Beta"], p["Gate"], S0)
    torch.cuda.synchronize()
    for name in ("O", "Sp"):
        a, b_ = chk[name], seq[name]
        err = float((a - b_).abs().max() / b_.abs().max())
        print(f"{name}: max err / max = {err:.2e}")
        assert err <= 1e-3, name
