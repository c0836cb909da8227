"""Pins of the oracle's model-level compositions -- CPU only.

orc.model_step (step!, src/llm/qwen35.jl:245-273) and orc.prefill_model
(prefill!, qwen35.jl:369-395) compose oracle pieces that are pinned one by one
elsewhere (test_oracle.py, test_oracle_deltanet.py). What those pins leave open
is the wiring: which norm goes where, the residual adds, the MLP, the DeltaNet
layer's conv / prep / recurrence / gated norm chain, the suffix conv's left
context, the bf16 buffers. Here both are checked against an independent torch
composition of the same model on a small mixed stack (DeltaNet, attention,
DeltaNet): torch rms_norm, SDPA with complex-multiplication RoPE, depthwise
conv1d, softplus and sigmoid from torch, the delta rule in its float64 product
form, fp32 matmuls -- with the reference's bf16 rounding points.

The same comparison is shown to fail for a composition with the MLP dropped or
with a layer's two norms swapped (planted in the torch composition), so it would
catch those slips in the oracle.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import D, EPS, HALF, HK, HQ, S, THETA

from oracle.rng import bf16_to_f32, f32_to_bf16, normal_bf16, normal_f32
from test_oracle import _torch_gated
from test_oracle_deltanet import _product_form

DM, INTER, VOCAB, CTX, KC = 128, 96, 300, 32, 4
LIN = dict(Dk=32, Dv=32, Hk=2, Hv=4)
NCH = 2 * LIN["Hk"] * LIN["Dk"] + LIN["Hv"] * LIN["Dv"]


def _model(seed):
    """E, head, final norm, layers [DeltaNet, attention, DeltaNet] as oracle dicts
    (bf16 bits; DeltaNet fp32 state and bf16 ring; attention caches)."""
    E = normal_bf16((VOCAB, DM), seed)
    head = normal_bf16((VOCAB, DM), seed + 1, scale=0.5)
    norm_w = normal_bf16((DM,), seed + 2, scale=0.1)
    Hv, Dv, Dk = LIN["Hv"], LIN["Dv"], LIN["Dk"]
    layers = []
    for i in range(3):
        s0 = seed + 10 * (i + 1)
        l = dict(norm1=normal_bf16((DM,), s0, scale=0.1), norm2=normal_bf16((DM,), s0 + 1, scale=0.1),
                 Wgu=normal_bf16((2 * INTER, DM), s0 + 2, scale=DM ** -0.5),
                 Wd=normal_bf16((DM, INTER), s0 + 3, scale=INTER ** -0.5))
        if i == 1:
            l.update(Wqkv=normal_bf16((S * D, DM), s0 + 4, scale=DM ** -0.5),
                     Wo=normal_bf16((DM, HQ * D), s0 + 5, scale=(HQ * D) ** -0.5),
                     qw=normal_bf16((D,), s0 + 6, scale=0.05), kw=normal_bf16((D,), s0 + 7, scale=0.05))
        else:
            l.update(kind="linear_attention",
                     Wqz=normal_bf16((NCH + Hv * Dv, DM), s0 + 4, scale=DM ** -0.5),
                     Wab=normal_bf16((2 * Hv, DM), s0 + 5, scale=DM ** -0.5),
                     Wout=normal_bf16((DM, Hv * Dv), s0 + 6, scale=(Hv * Dv) ** -0.5),
                     conv_w=normal_bf16((KC, NCH), s0 + 7, scale=0.5),
                     conv_b=normal_bf16((NCH,), s0 + 8, scale=0.1),
                     A_log=normal_f32(Hv, s0 + 9, scale=0.5),
                     dt_bias=normal_f32(Hv, s0 + 10, scale=0.5),
                     gnorm_w=normal_bf16((Dv,), s0 + 11, scale=0.2, shift=1.0))
        layers.append(l)
    return E, head, norm_w, layers


def _fresh_state(layers, B, seed, caches=True):
    """Per-layer state: random attention caches, zero or random DeltaNet state."""
    out = []
    for i, l in enumerate(layers):
        l = dict(l)
        if l.get("kind") == "linear_attention":
            l["S"] = normal_f32(B * LIN["Hv"] * LIN["Dv"] * LIN["Dk"], seed + i, scale=0.05).reshape(
                B, LIN["Hv"], LIN["Dv"], LIN["Dk"])
            l["ring"] = normal_bf16((B, KC, NCH), seed + 50 + i)
        else:
            shape = (B, HK, CTX, D)
            l["kc"] = normal_bf16(shape, seed + 100 + i) if caches else np.zeros(shape, np.uint16)
            l["vc"] = normal_bf16(shape, seed + 200 + i) if caches else np.zeros(shape, np.uint16)
        out.append(l)
    return out


# ---------------------------------------------------------------- torch pieces
def _t(bits):
    return torch.from_numpy(bf16_to_f32(np.asarray(bits)))


def _r16(x):
    """The reference stores this buffer as bf16 (round to nearest even)."""
    return x.to(torch.bfloat16).to(torch.float32)


def _lin(x, W):
    return x @ _t(W).t()


def _norm(x, w):
    return F.rms_norm(x, (x.shape[-1],), weight=_t(w) + 1.0, eps=EPS)


def _add_norm(x, dx, w):
    """x' = bf16(x + dx) (stored); y = x' rstd (w + 1), rstd from the fp32 sum."""
    s = x + dx
    rstd = torch.rsqrt(s.pow(2).mean(-1, keepdim=True) + EPS)
    xo = _r16(s)
    return xo, _r16(xo * rstd * (_t(w) + 1.0))


def _mlp(xn, l):
    gu = _r16(_lin(xn, l["Wgu"]))
    return _lin(_r16(F.silu(gu[..., :INTER]) * gu[..., INTER:]), l["Wd"])


def _l2(x):
    return x * torch.rsqrt(x.pow(2).sum(-1, keepdim=True) + 1e-6)


def _dn_tail(y, qz, ab, l, T, B, softplus):
    """From the conv output y [B][T][n] (bf16 values) on: l2 norms, gates, the
    delta rule in float64 product form, the gated norm with silu(z), Wout."""
    Dk, Dv, Hk, Hv = LIN["Dk"], LIN["Dv"], LIN["Hk"], LIN["Hv"]
    q = _l2(y[..., :Hk * Dk].reshape(B, T, Hk, Dk)) / np.sqrt(Dk)
    k = _l2(y[..., Hk * Dk:2 * Hk * Dk].reshape(B, T, Hk, Dk))
    v = y[..., 2 * Hk * Dk:].reshape(B, T, Hv, Dv)
    a, bt = ab[..., :Hv], ab[..., Hv:]
    gate = -torch.exp(torch.from_numpy(l["A_log"])) * softplus(a + torch.from_numpy(l["dt_bias"]))
    beta = torch.sigmoid(bt)
    o, S = _product_form(q.permute(0, 2, 1, 3).numpy(), k.permute(0, 2, 1, 3).numpy(),
                         v.permute(0, 2, 1, 3).numpy(), beta.numpy(), gate.numpy(), l["S"])
    o = torch.from_numpy(o).float().permute(0, 2, 1, 3)                 # [B][T][Hv][Dv]
    z = qz[..., NCH:].reshape(B, T, Hv, Dv)
    g = o * torch.rsqrt(o.pow(2).mean(-1, keepdim=True) + EPS) * _t(l["gnorm_w"]) * F.silu(z)
    return _lin(_r16(g).reshape(B, T, Hv * Dv), l["Wout"]), S


def _dn_decode(xn, l, B):
    qz, ab = _r16(_lin(xn, l["Wqz"])), _r16(_lin(xn, l["Wab"]))
    ring = torch.cat([_t(l["ring"])[:, 1:], qz[:, None, :NCH]], dim=1)     # newest in column K
    y = _r16(F.silu((ring * _t(l["conv_w"])).sum(1) + _t(l["conv_b"])))
    h, S = _dn_tail(y[:, None], qz[:, None], ab[:, None], l, 1, B, F.softplus)  # threshold 20
    return h[:, 0], S


def _dn_prefill(xn, l, T, B, offset):
    qz, ab = _r16(_lin(xn, l["Wqz"])), _r16(_lin(xn, l["Wab"]))
    X = qz[..., :NCH]
    left = _t(l["ring"])[:, 1:] if offset > 0 else torch.zeros(B, KC - 1, NCH)
    full = torch.cat([left, X], dim=1).transpose(1, 2)                 # [B][n][K-1+T]
    w = _t(l["conv_w"]).t()[:, None, :]                                 # [n][1][K]
    y = _r16(F.silu(F.conv1d(full, w, bias=_t(l["conv_b"]), groups=NCH).transpose(1, 2)))
    h, S = _dn_tail(y, qz, ab, l, T, B, lambda x: torch.log1p(torch.exp(x)))
    return h, S


def _attn(xn, l, prior, T, B):
    qkv = f32_to_bf16(_lin(xn, l["Wqkv"]).numpy()).reshape(B, T, S, D)
    o = _torch_gated(qkv, l["kc"], l["vc"], prior, np.full(B, T, np.int32), l["qw"], l["kw"])
    return _lin(_r16(torch.from_numpy(o).float()).reshape(B, T, HQ * D), l["Wo"])


def _torch_model(E, head, norm_w, layers, tokens, mode, *, positions=None, offset=0,
                 drop_mlp=False, swap_norms=False):
    """step! (mode "step": tokens [B], positions [B]) or prefill! (mode "prefill":
    tokens [B][T], offset) in torch. Returns (next tokens, final xn [B][DM])."""
    tokens = np.asarray(tokens)
    B = tokens.shape[0]
    T = 1 if mode == "step" else tokens.shape[1]
    x = _t(E[np.clip(tokens.reshape(B, T) - 1, 0, VOCAB - 1)])              # [B][T][DM]
    xn = _r16(_norm(x, layers[0]["norm1"]))
    for i, l in enumerate(layers):
        if l.get("kind") == "linear_attention":
            h = _dn_decode(xn[:, 0], l, B)[0][:, None] if mode == "step" else \
                _dn_prefill(xn, l, T, B, offset)[0]
        else:
            prior = positions - 1 if mode == "step" else np.full(B, offset, np.int32)
            h = _attn(xn, l, prior, T, B)
        nw2 = l["norm1"] if swap_norms else l["norm2"]
        x, xn = _add_norm(x, _r16(h), nw2)
        dh = torch.zeros_like(x) if drop_mlp else _mlp(xn, l)
        nw = norm_w if i == len(layers) - 1 else layers[i + 1]["norm1"]
        x, xn = _add_norm(x, _r16(dh), nw)
    last = xn[:, T - 1]
    logits = last.double() @ _t(head).double().t()
    return logits.argmax(1).numpy().astype(np.int32) + 1, last.numpy(), logits.numpy()


def _compare(res, xn, t_res, t_xn, t_logits, what):
    top2 = np.sort(t_logits, axis=1)[:, -2:]
    margin = top2[:, 1] - top2[:, 0]
    err = float(np.abs(xn - t_xn).max() / np.abs(t_xn).max())
    ok = margin > 0.05
    print(f"{what}: final xn max err / max {err:.2e}; tokens {res.tolist()} torch "
          f"{t_res.tolist()} margins {np.round(margin, 3).tolist()}")
    return err, ok


# ---------------------------------------------------------------- the pins
def test_model_step_is_the_torch_composition(orc):
    """One step! of the mixed stack: final xn within bf16 rounding of the torch
    composition, tokens equal where its top-2 margin is not tiny; a dropped MLP or
    swapped norms move xn by far more."""
    B = 3
    E, head, norm_w, layers0 = _model(400)
    layers = _fresh_state(layers0, B, 410)
    tok = np.array([1, 150, 300], np.int32)
    pos = np.array([5, 17, 32], np.int32)
    c, s = orc.rope_tables(HALF, CTX, THETA)
    res, _, xn = orc.model_step(E, layers, norm_w, head, tok, pos, c, s, Hq=HQ, Hk=HK, eps=EPS,
                                linear_cfg=LIN)
    t_res, t_xn, t_log = _torch_model(E, head, norm_w, layers, tok, "step", positions=pos)
    err, ok = _compare(res, xn, t_res, t_xn, t_log, "step")
    assert err <= 2e-2
    assert ok.sum() >= B - 1 and np.array_equal(res[ok], t_res[ok])
    for kw in (dict(drop_mlp=True), dict(swap_norms=True)):
        _, m_xn, _ = _torch_model(E, head, norm_w, layers, tok, "step", positions=pos, **kw)
        planted = float(np.abs(xn - m_xn).max() / np.abs(m_xn).max())
        print(f"step with {kw}: max err / max {planted:.2e}")
        assert planted > 10 * max(err, 1e-3)


def test_prefill_model_is_the_torch_composition(orc):
    """prefill! of the mixed stack over 9 tokens from zero DeltaNet state, then a
    5-token suffix on the states it left (offset 9: the conv's left context from
    the ring, the caches' prior rows): final xn and tokens against the torch
    composition, and the suffix's states against a 14-token prefill."""
    B, T1, T2 = 2, 9, 5
    E, head, norm_w, layers0 = _model(500)
    layers = _fresh_state(layers0, B, 510, caches=False)
    for l in layers:
        if l.get("kind") == "linear_attention":
            l["S"][:] = 0
            l["ring"][:] = 0
    ids = np.random.default_rng(520).integers(1, VOCAB + 1, size=(B, T1 + T2)).astype(np.int32)
    c, s = orc.rope_tables(HALF, CTX, THETA)
    res, _, xn, states = orc.prefill_model(E, layers, norm_w, head, ids[:, :T1], 0, c, s, Hq=HQ,
                                           Hk=HK, eps=EPS, linear_cfg=LIN)
    t_res, t_xn, t_log = _torch_model(E, head, norm_w, layers, ids[:, :T1], "prefill")
    err, ok = _compare(res, xn, t_res, t_xn, t_log, "prefill prefix")
    assert err <= 2e-2 and ok.sum() >= B - 1 and np.array_equal(res[ok], t_res[ok])
    for kw in (dict(drop_mlp=True), dict(swap_norms=True)):
        _, m_xn, _ = _torch_model(E, head, norm_w, layers, ids[:, :T1], "prefill", **kw)
        planted = float(np.abs(xn - m_xn).max() / np.abs(m_xn).max())
        print(f"prefill with {kw}: max err / max {planted:.2e}")
        assert planted > 10 * max(err, 1e-3)
    # the suffix on the prefix's states == the whole prefill's last rows
    cont = [dict(l) for l in layers]
    for l, st in zip(cont, states):
        if l.get("kind") == "linear_attention":
            l["ring"], l["S"] = st
        else:
            l["kc"], l["vc"] = st
    res2, _, xn2, states2 = orc.prefill_model(E, cont, norm_w, head, ids[:, T1:], T1, c, s, Hq=HQ,
                                              Hk=HK, eps=EPS, linear_cfg=LIN)
    t_res2, t_xn2, t_log2 = _torch_model(E, head, norm_w, cont, ids[:, T1:], "prefill", offset=T1)
    err2, ok2 = _compare(res2, xn2, t_res2, t_xn2, t_log2, "prefill suffix")
    assert err2 <= 2e-2 and ok2.sum() >= B - 1 and np.array_equal(res2[ok2], t_res2[ok2])
    resf, _, xnf, statesf = orc.prefill_model(E, layers, norm_w, head, ids, 0, c, s, Hq=HQ, Hk=HK,
                                              eps=EPS, linear_cfg=LIN)
    assert float(np.abs(xn2 - xnf).max() / np.abs(xnf).max()) <= 2e-2
    for (a1, a2), (b1, b2) in zip(states2, statesf):
        for u, w in ((a1, b1), (a2, b2)):
            u = bf16_to_f32(u) if u.dtype == np.uint16 else u
            w = bf16_to_f32(w) if w.dtype == np.uint16 else w
            assert float(np.abs(u - w).max()) <= 2e-2 * max(float(np.abs(w).max()), 1.0)
