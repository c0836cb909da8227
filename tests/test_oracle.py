"""Pins of the CPU oracle (oracle/oracle.c) — CPU only.

The reference holds no golden vectors or known-answer tests for this path
(its test/runtests.jl covers checkpoint loaders only), so each oracle function
is checked against an independent library or a closed form chosen so that a
plausible slip (dropped (w+1) offset, wrong rotate-half sign or pair index,
wrong scale, top-left instead of suffix causal alignment, wrong GQA head map,
wrong slot of the packed [q|g] projection, off-by-one position) fails:

  rope_tables     closed forms (position 0, inv_freq_i = theta^(-i/32)),
                  cos^2+sin^2 = 1, torch f32 cos/sin of the same angles
  head_norm_rope  torch.nn.functional.rms_norm(weight = w+1) followed by a
                  complex multiplication by exp(i*angle); scale invariance;
                  pair-norm preservation; relative-position property
  attention       torch.nn.functional.scaled_dot_product_attention (fp32, CPU)
                  with an explicit suffix-aligned causal mask and repeated KV
                  heads; one-key and identical-key closed forms; window
                  locality; GQA == MHA on repeated heads
  gated decode /  a composition of the torch checks above on the packed
  gated prefill   projection; decode == last row of a causal prefill; chunked
                  prefill == the matching rows of a full prefill
  rng             SplitMix64 published outputs; bf16 rounding == torch's
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import D, EPS, HALF, HK, HQ, S, THETA

from oracle.rng import _splitmix64, bf16_to_f32, f32_to_bf16, normal_bf16, normal_f32


# ---------------------------------------------------------------- rng / bf16
def test_splitmix64_published_vector():
    # Vigna's splitmix64.c with x = 1234567: the first five next() outputs.
    got = _splitmix64(1234567, np.arange(5, dtype=np.uint64)).tolist()
    assert got == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                   4593380528125082431, 16408922859458223821]


def test_normal_stream_statistics():
    x = normal_f32(1 << 20, 7).astype(np.float64)
    assert abs(x.mean()) < 5e-3 and abs(x.var() - 1) < 5e-3
    assert abs(np.mean(x ** 3)) < 1e-2 and abs(np.mean(x ** 4) - 3) < 3e-2


def test_bf16_rounding_matches_torch():
    x = normal_f32(100_000, 3, scale=7.0)
    x = np.concatenate([x, np.float32([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 0.0])])
    mine = f32_to_bf16(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(mine, theirs)
    assert np.array_equal(bf16_to_f32(mine), torch.from_numpy(x).to(torch.bfloat16).float().numpy())


# ---------------------------------------------------------------- rope tables
def test_rope_tables_closed_forms(orc):
    ctx = 4096
    c, s = orc.rope_tables(HALF, ctx, THETA)
    assert c.shape == (ctx, HALF) and c.dtype == np.float32
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)          # position 0 is the identity
    assert np.max(np.abs(c.astype(np.float64) ** 2 + s.astype(np.float64) ** 2 - 1)) < 3e-7
    # angle at position 1 is inv_freq_i = theta^(-i/32): 1 rad at i = 0, 1/sqrt(theta) at i = 16
    ang1 = np.arctan2(s[1].astype(np.float64), c[1].astype(np.float64))
    assert abs(ang1[0] - 1.0) < 1e-7
    assert abs(ang1[16] - THETA ** -0.5) < 1e-9
    ratio = ang1[1:] / ang1[:-1]
    assert np.allclose(ratio, THETA ** (-1 / 32), rtol=1e-6)
    # against torch's own f32 cos/sin of the f32 angles inv_freq * t
    inv = torch.tensor([THETA ** (-i / HALF) for i in range(HALF)], dtype=torch.float64).float()
    ang = torch.outer(torch.arange(ctx, dtype=torch.float32), inv)
    assert np.max(np.abs(c - torch.cos(ang).numpy())) < 2.5e-7
    assert np.max(np.abs(s - torch.sin(ang).numpy())) < 2.5e-7


# ---------------------------------------------------------------- norm + rope
def _torch_norm_rope(x, w, pos, ctx=2048, half=HALF):
    """Independent restatement: torch rms_norm with weight (w + 1), then the first
    2 half dims rotated as half complex numbers (x_i + i x_{i+half}) * exp(i angle_i)."""
    xt = torch.from_numpy(np.asarray(x, np.float32))
    wt = torch.from_numpy(np.asarray(w, np.float32)) + 1.0
    y = F.rms_norm(xt, (xt.shape[-1],), weight=wt, eps=EPS)
    inv = torch.tensor([THETA ** (-i / half) for i in range(half)], dtype=torch.float64).float()
    ang = (inv * torch.tensor(float(pos), dtype=torch.float32)).double()
    z = torch.complex(y[..., :half].double(), y[..., half:2 * half].double())
    z = z * torch.polar(torch.ones_like(ang), ang)
    out = y.clone().double()
    out[..., :half] = z.real
    out[..., half:2 * half] = z.imag
    return out.numpy()


@pytest.mark.parametrize("pos", [0, 1, 511, 4000])
def test_head_norm_rope_vs_torch(orc, pos):
    c, s = orc.rope_tables(HALF, 4096, THETA)
    x = bf16_to_f32(normal_bf16((D,), 100 + pos))
    w = bf16_to_f32(normal_bf16((D,), 200, scale=0.05))
    y = orc.head_norm_rope(x, w, EPS, 1.0, c, s, pos)
    ref = _torch_norm_rope(x, w, pos)
    assert np.max(np.abs(y - ref)) < 2e-5
    assert np.array_equal(y[2 * HALF:] != 0, ref[2 * HALF:] != 0)


@pytest.mark.parametrize("Dh,half", [(16, 8), (64, 8), (128, 64), (512, 32), (128, 1)])
def test_head_norm_rope_head_dims_vs_torch(orc, Dh, half):
    """Other head dims and rotary widths (qknorm_rope_append.jl:100-141 take any
    power-of-two D and any HALF_ROT up to D/2)."""
    c, s = orc.rope_tables(half, 4096, THETA)
    x = bf16_to_f32(normal_bf16((Dh,), 300 + Dh))
    w = bf16_to_f32(normal_bf16((Dh,), 301, scale=0.05))
    y = orc.head_norm_rope(x, w, EPS, 1.0, c, s, 777)
    ref = _torch_norm_rope(x, w, 777, half=half)
    assert np.max(np.abs(y - ref)) < 2e-5


def test_head_norm_invariants(orc):
    c, s = orc.rope_tables(HALF, 1024, THETA)
    x = bf16_to_f32(normal_bf16((D,), 5))
    w0 = np.zeros(D, np.float32)
    y = orc.head_norm_rope(x, w0, EPS, 1.0, c, s, 0)
    assert abs(np.mean(y.astype(np.float64) ** 2) - 1) < 1e-5      # w = 0 -> unit RMS
    y2 = orc.head_norm_rope(3.7 * x, w0, EPS, 1.0, c, s, 0)
    assert np.max(np.abs(y - y2)) < 1e-5                            # scale invariance
    yp = orc.head_norm_rope(x, w0, EPS, 1.0, c, s, 777)
    pair = lambda v: v[:HALF].astype(np.float64) ** 2 + v[HALF:2 * HALF].astype(np.float64) ** 2
    assert np.max(np.abs(pair(yp) - pair(y))) < 1e-5                # rotation keeps pair norms
    assert np.array_equal(yp[2 * HALF:], y[2 * HALF:])              # dims 65..256 pass through


def test_rope_relative_position(orc):
    c, s = orc.rope_tables(HALF, 2048, THETA)
    q = bf16_to_f32(normal_bf16((D,), 31))
    k = bf16_to_f32(normal_bf16((D,), 32))
    w = np.zeros(D, np.float32)
    dots = []
    for shift in (0, 100, 1000):
        qa = orc.head_norm_rope(q, w, EPS, 1.0, c, s, 300 + shift)
        ka = orc.head_norm_rope(k, w, EPS, 1.0, c, s, 120 + shift)
        dots.append(float(np.dot(qa[:2 * HALF], ka[:2 * HALF])))
    assert max(dots) - min(dots) < 2e-3 * max(1.0, abs(dots[0]))


# ---------------------------------------------------------------- attention
def _torch_attention(q, k, v, causal, k_lengths=None, q_lengths=None):
    """SDPA per sequence with KV heads repeated and a suffix-aligned causal mask."""
    B, H, L, _ = q.shape
    Hk, Lk = k.shape[1], k.shape[2]
    out = np.full((B, H, L, v.shape[3]), np.nan, np.float32)
    for b in range(B):
        kl = int(k_lengths[b]) if k_lengths is not None else Lk
        ql = int(q_lengths[b]) if q_lengths is not None else L
        qt = torch.from_numpy(q[b, :, :ql])
        kt = torch.from_numpy(k[b, :, :kl]).repeat_interleave(H // Hk, dim=0)
        vt = torch.from_numpy(v[b, :, :kl]).repeat_interleave(H // Hk, dim=0)
        mask = None
        if causal:
            off = kl - ql
            mask = torch.arange(kl)[None, :] <= (torch.arange(ql)[:, None] + off)
        o = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask)
        out[b, :, :ql] = o.numpy()
    return out


def _rand(shape, seed):
    return bf16_to_f32(normal_bf16(shape, seed)).reshape(shape)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("H,Hk", [(4, 2), (16, 4), (3, 3)])
def test_attention_vs_sdpa(orc, causal, H, Hk):
    B, L, Lk = 2, 9, 23
    q, k, v = _rand((B, H, L, D), 1), _rand((B, Hk, Lk, D), 2), _rand((B, Hk, Lk, D), 3)
    o = orc.attention(q, k, v, causal=causal)
    ref = _torch_attention(q, k, v, causal)
    assert np.max(np.abs(o - ref)) < 2e-6


def test_attention_ragged_vs_sdpa(orc):
    B, H, Hk, L, Lk = 3, 8, 2, 12, 40
    q, k, v = _rand((B, H, L, D), 4), _rand((B, Hk, Lk, D), 5), _rand((B, Hk, Lk, D), 6)
    kl = np.array([40, 13, 5], np.int32)
    ql = np.array([12, 13, 1], np.int32)
    ql[1] = 12  # q_len <= L
    o = orc.attention(q, k, v, causal=True, k_lengths=kl, q_lengths=ql)
    ref = _torch_attention(q, k, v, True, kl, ql)
    finite = ~np.isnan(ref)
    assert np.array_equal(finite, ~np.isnan(o))       # rows past q_len untouched
    assert np.max(np.abs(o[finite] - ref[finite])) < 2e-6


@pytest.mark.parametrize("Dk,Dv,causal", [(64, 128, True), (128, 32, False), (16, 512, True)])
def test_attention_head_dims_vs_sdpa(orc, Dk, Dv, causal):
    """Dk != Dv and head dims other than 256 (attention.jl:93-101 takes any):
    scores scaled by 1/sqrt(Dk), outputs Dv wide; ragged lengths, GQA 4:1."""
    B, H, Hk, L, Lk = 2, 8, 2, 11, 37
    q, k, v = _rand((B, H, L, Dk), 7), _rand((B, Hk, Lk, Dk), 8), _rand((B, Hk, Lk, Dv), 9)
    kl = np.array([37, 20], np.int32)
    ql = np.array([11, 6], np.int32)
    o = orc.attention(q, k, v, causal=causal, k_lengths=kl, q_lengths=ql)
    ref = _torch_attention(q, k, v, causal, kl, ql)
    assert o.shape == (B, H, L, Dv)
    finite = ~np.isnan(ref)
    assert np.array_equal(finite, ~np.isnan(o))
    assert np.max(np.abs(o[finite] - ref[finite])) < 2e-6


def test_attention_closed_forms(orc):
    B, H, Hk = 1, 4, 2
    q = _rand((B, H, 6, D), 7)
    v = _rand((B, Hk, 6, D), 8)
    # one key: o = v
    o = orc.attention(q[:, :, :1], _rand((B, Hk, 1, D), 9), v[:, :, :1], causal=True)
    assert np.max(np.abs(o - np.repeat(v[:, :, :1], 2, axis=1))) < 1e-6
    # identical keys: o = running mean of V over the causal window
    k = np.repeat(_rand((B, Hk, 1, D), 10), 6, axis=2)
    o = orc.attention(q, k, v, causal=True)
    means = np.cumsum(v, axis=2) / np.arange(1, 7)[None, None, :, None]
    assert np.max(np.abs(o - np.repeat(means, 2, axis=1))) < 1e-5
    # window locality: keys beyond t + off do not influence row t
    k = _rand((B, Hk, 6, D), 11)
    o1 = orc.attention(q, k, v, causal=True)
    v2 = v.copy()
    v2[:, :, 4:] += 100.0
    o2 = orc.attention(q, k, v2, causal=True)
    assert np.array_equal(o1[:, :, :4], o2[:, :, :4]) and not np.allclose(o1[:, :, 4:], o2[:, :, 4:])
    # GQA == MHA with repeated KV heads
    o_mha = orc.attention(q, np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1), causal=True)
    assert np.max(np.abs(o1 - o_mha)) == 0.0


# ---------------------------------------------------------------- gated layer
def _torch_gated(qkv_bits, kc_bits, vc_bits, prior, qlen, qw_bits, kw_bits):
    """forward(::AttnLayer) attention part from torch pieces: rms_norm + complex
    rope + cache append + SDPA over columns 0..prior+t + sigmoid gate."""
    qkv = bf16_to_f32(qkv_bits).reshape(qkv_bits.shape)
    B, T = qkv.shape[:2]
    qw, kw = bf16_to_f32(qw_bits), bf16_to_f32(kw_bits)
    out = np.full((B, T, HQ, D), np.nan)
    for b in range(B):
        P, C = int(prior[b]), int(qlen[b])
        kcache = bf16_to_f32(kc_bits[b]).reshape(HK, -1, D)[:, :P].astype(np.float64)
        vcache = bf16_to_f32(vc_bits[b]).reshape(HK, -1, D)[:, :P].astype(np.float64)
        knew = np.stack([np.stack([_torch_norm_rope(qkv[b, t, 2 * HQ + j], kw, P + t)
                                   for t in range(C)]) for j in range(HK)])
        vnew = qkv[b, :C, 2 * HQ + HK:].transpose(1, 0, 2).astype(np.float64)
        K = np.concatenate([kcache, knew], axis=1)
        V = np.concatenate([vcache, vnew], axis=1)
        qn = np.stack([np.stack([_torch_norm_rope(qkv[b, t, 2 * h], qw, P + t)
                                 for t in range(C)]) for h in range(HQ)])
        Kt = torch.from_numpy(K).repeat_interleave(HQ // HK, dim=0)
        Vt = torch.from_numpy(V).repeat_interleave(HQ // HK, dim=0)
        mask = torch.arange(P + C)[None, :] <= (torch.arange(C)[:, None] + P)
        o = F.scaled_dot_product_attention(torch.from_numpy(qn), Kt, Vt, attn_mask=mask).numpy()
        g = qkv[b, :C, 1:2 * HQ:2]                       # (C, HQ, D): the gate slots
        out[b, :C] = o.transpose(1, 0, 2) * torch.sigmoid(torch.from_numpy(g).double()).numpy()
    return out


def test_gated_prefill_vs_torch(orc):
    B, T, ctx = 2, 11, 64
    qkv = normal_bf16((B, T, S, D), 41)
    kc, vc = normal_bf16((B, HK, ctx, D), 42), normal_bf16((B, HK, ctx, D), 43)
    qw, kw = normal_bf16((D,), 44, scale=0.05), normal_bf16((D,), 45, scale=0.05)
    prior, qlen = np.array([5, 30], np.int32), np.array([11, 7], np.int32)
    c, s = orc.rope_tables(HALF, ctx, THETA)
    out, kn, vn = orc.gated_prefill(qkv, kc, vc, prior, qlen, qw, kw, c, s, Hq=HQ, Hk=HK,
                                    eps=EPS, w_offset=1.0)
    ref = _torch_gated(qkv, kc, vc, prior, qlen, qw, kw)
    fin = ~np.isnan(ref)
    assert np.array_equal(fin, ~np.isnan(out))
    assert np.max(np.abs(out[fin] - ref[fin])) < 3e-5
    # the appended K rows are norm+rope of the packed k slots
    k0 = _torch_norm_rope(bf16_to_f32(qkv[1, 3, 2 * HQ + 2]), bf16_to_f32(kw), 30 + 3)
    assert np.max(np.abs(kn[1, 2, 3] - k0)) < 2e-5
    assert np.array_equal(vn[0, 1, 4], bf16_to_f32(qkv[0, 4, 2 * HQ + HK + 1]))


def test_gated_decode_is_last_prefill_row(orc):
    B, ctx = 2, 96
    pos = np.array([40, 96], np.int32)         # 1-based column of the new token
    kc, vc = normal_bf16((B, HK, ctx, D), 51), normal_bf16((B, HK, ctx, D), 52)
    qkv1 = normal_bf16((B, S, D), 53)
    qw, kw = normal_bf16((D,), 54, scale=0.05), normal_bf16((D,), 55, scale=0.05)
    c, s = orc.rope_tables(HALF, ctx, THETA)
    dec, kn, vn = orc.gated_decode(qkv1, kc, vc, pos, qw, kw, c, s, Hq=HQ, Hk=HK, eps=EPS,
                                   w_offset=1.0)
    # the same token as a 1-row chunked prefill after pos-1 cached tokens
    pre, kp, vp = orc.gated_prefill(qkv1[:, None], kc, vc, pos - 1, np.ones(B, np.int32), qw, kw,
                                    c, s, Hq=HQ, Hk=HK, eps=EPS, w_offset=1.0)
    assert np.max(np.abs(dec - pre[:, 0])) < 1e-6
    assert np.array_equal(kn, kp[:, :, 0]) and np.array_equal(vn, vp[:, :, 0])
    ref = _torch_gated(qkv1[:, None], kc, vc, pos - 1, np.ones(B), qw, kw)
    assert np.max(np.abs(dec - ref[:, 0])) < 3e-5


def test_chunked_prefill_matches_full_prefill(orc):
    """attention.jl:3-7: a chunk after P cached tokens equals rows P.. of the full prefill."""
    B, T, ctx, P = 1, 48, 64, 20
    qkv = normal_bf16((B, T, S, D), 61)
    qw, kw = normal_bf16((D,), 62, scale=0.05), normal_bf16((D,), 63, scale=0.05)
    c, s = orc.rope_tables(HALF, ctx, THETA)
    zero = np.zeros((B, HK, ctx, D), np.uint16)
    full, kf, vf = orc.gated_prefill(qkv, zero, zero, np.zeros(B, np.int32),
                                     np.full(B, T, np.int32), qw, kw, c, s, Hq=HQ, Hk=HK,
                                     eps=EPS, w_offset=1.0)
    kc, vc = zero.copy(), zero.copy()
    kc[:, :, :P] = f32_to_bf16(kf[:, :, :P])
    vc[:, :, :P] = f32_to_bf16(vf[:, :, :P])
    part, _, _ = orc.gated_prefill(np.ascontiguousarray(qkv[:, P:]), kc, vc,
                                   np.full(B, P, np.int32), np.full(B, T - P, np.int32), qw, kw,
                                   c, s, Hq=HQ, Hk=HK, eps=EPS, w_offset=1.0)
    # the cached prefix went through one bf16 rounding of K
    assert np.max(np.abs(part[:, :T - P] - full[:, P:])) < 1e-2
    assert np.mean(np.abs(part[:, :T - P] - full[:, P:])) < 1e-3


def test_linear_matches_torch_matmul(orc):
    """orc.linear (y = W^T x, src/linear.jl:40-57) against torch.matmul in fp32 on
    the CPU, for a GEMV (one column), a thin and a square problem; and two closed
    forms: W = identity gives y = x, and scaling x by 2 scales y by 2 exactly."""
    import torch
    from oracle.rng import bf16_to_f32, f32_to_bf16, normal_bf16
    for (N, K, M) in [(1, 256, 96), (7, 320, 130), (64, 128, 64)]:
        x = normal_bf16((N, K), 500 + K)
        W = normal_bf16((M, K), 600 + M, scale=K ** -0.5)
        y = orc.linear(x, W)
        ref = (torch.from_numpy(bf16_to_f32(x)) @ torch.from_numpy(bf16_to_f32(W)).T).numpy()
        assert y.shape == (N, M)
        assert np.max(np.abs(y - ref)) <= 1e-4 * max(1.0, np.max(np.abs(ref)))
    x = normal_bf16((5, 64), 7)
    eye = f32_to_bf16(np.eye(64, dtype=np.float32))
    assert np.array_equal(orc.linear(x, eye), bf16_to_f32(x))
    x2 = f32_to_bf16(2.0 * bf16_to_f32(x))
    W = normal_bf16((33, 64), 8)
    assert np.array_equal(orc.linear(x2, W), 2.0 * orc.linear(x, W))


def test_decode_layer_is_the_composition(orc):
    """orc.decode_layer = Wo-projection of the bf16-rounded gated decode of the
    bf16-rounded qkv projection (qwen35.jl:193-206), recomposed here with torch
    matmuls for the two projections."""
    import torch
    from conftest import D, EPS, HALF, HK, HQ, S, THETA
    from oracle.rng import bf16_to_f32, f32_to_bf16, normal_bf16
    B, ctx, Dm = 2, 64, 96
    xn = normal_bf16((B, Dm), 11)
    Wqkv = normal_bf16((S * D, Dm), 12, scale=Dm ** -0.5)
    Wo = normal_bf16((Dm, HQ * D), 13, scale=(HQ * D) ** -0.5)
    kc, vc = normal_bf16((B, HK, ctx, D), 14), normal_bf16((B, HK, ctx, D), 15)
    qw, kw = normal_bf16((D,), 16, scale=0.05), normal_bf16((D,), 17, scale=0.05)
    pos = np.array([64, 9], np.int32)
    c, s = orc.rope_tables(HALF, ctx, THETA)
    h, _, _ = orc.decode_layer(xn, Wqkv, Wo, kc, vc, pos, qw, kw, c, s, Hq=HQ, Hk=HK, eps=EPS,
                               w_offset=1.0)
    t = lambda a: torch.from_numpy(bf16_to_f32(a))
    qkv = f32_to_bf16((t(xn) @ t(Wqkv).T).numpy()).reshape(B, S, D)
    o, _, _ = orc.gated_decode(qkv, kc, vc, pos, qw, kw, c, s, Hq=HQ, Hk=HK, eps=EPS, w_offset=1.0)
    ref = (t(f32_to_bf16(o).reshape(B, HQ * D)) @ t(Wo).T).numpy()
    # torch sums in another order, so a few bf16 roundings of qkv / o flip by one ulp
    assert np.max(np.abs(h - ref)) <= 2e-3 and np.mean(np.abs(h - ref)) <= 1e-4
    assert np.max(np.abs(ref)) > 0.1


# ---------------------------------------------------- the rest of the decode step
def test_rms_norm_invariants(orc):
    """rms_norm (rms_norm.jl:3-31): with w = 0 and offset 1 every output column
    has unit RMS (a wrong divisor, a dropped square root or offset fails); a
    power-of-two scale of x leaves y unchanged (eps negligible); the weight
    multiplies by (w + offset); a 2-row known answer."""
    x = normal_bf16((5, 2560), 11, scale=3.0)
    zero = np.zeros(2560, np.uint16)
    y = orc.rms_norm(x, zero, eps=1e-30, offset=1.0)
    assert np.allclose(np.sqrt((y.astype(np.float64) ** 2).mean(axis=1)), 1.0, rtol=1e-5)
    y2 = orc.rms_norm(f32_to_bf16(bf16_to_f32(x) * 4.0), zero, eps=1e-30, offset=1.0)
    assert np.allclose(y, y2, rtol=1e-6, atol=1e-7)
    w = normal_bf16((2560,), 12, scale=0.05)
    yw = orc.rms_norm(x, w, eps=1e-30, offset=1.0)
    assert np.allclose(yw, y * (bf16_to_f32(w) + 1.0), rtol=1e-6, atol=1e-7)
    k = orc.rms_norm(f32_to_bf16(np.array([[3.0, 4.0]], np.float32)), np.zeros(2, np.uint16),
                     eps=0.0, offset=2.0)
    r = np.sqrt(12.5)
    assert np.allclose(k, [[2 * 3 / r, 2 * 4 / r]], rtol=1e-6)


def test_fused_add_rms_norm_is_the_norm_of_the_sum(orc):
    """fused_add_rms_norm (residual_norm.jl:4-37): on integer-valued x, dx the sum
    is exact in bf16, so x' == x + dx and y == rms_norm(x') bit for bit."""
    rng = np.random.default_rng(13)
    x = f32_to_bf16(rng.integers(-40, 40, size=(3, 1024)).astype(np.float32))
    dx = f32_to_bf16(rng.integers(-40, 40, size=(3, 1024)).astype(np.float32))
    w = normal_bf16((1024,), 14, scale=0.05)
    y, xo = orc.rms_norm(x, w, eps=1e-6, offset=1.0, dx=dx)
    s = bf16_to_f32(x) + bf16_to_f32(dx)
    assert np.array_equal(xo, s)
    assert np.array_equal(y, orc.rms_norm(f32_to_bf16(s), w, eps=1e-6, offset=1.0))


def test_silu_mul_identities(orc):
    """mid = silu(gate) * up (qwen35.jl:234-243, kernels.jl:35): silu(g) - silu(-g)
    = g (a sign or sigmoid-argument slip fails), silu(0) = 0, silu(g) -> g for
    large g, linear in up; gate is the first half of each column."""
    g = normal_bf16((2, 512), 15, scale=3.0)
    one = f32_to_bf16(np.ones((2, 512), np.float32))
    pos = orc.silu_mul(np.concatenate([g, one], axis=1))
    neg = orc.silu_mul(np.concatenate([f32_to_bf16(-bf16_to_f32(g)), one], axis=1))
    assert np.allclose(pos - neg, bf16_to_f32(g), rtol=1e-5, atol=1e-6)
    z = orc.silu_mul(np.concatenate([np.zeros((1, 8), np.uint16), one[:1, :8]], axis=1))
    assert np.all(z == 0.0)
    big = orc.silu_mul(np.concatenate([f32_to_bf16(np.full((1, 8), 40.0, np.float32)),
                                       one[:1, :8]], axis=1))
    assert np.allclose(big, 40.0, rtol=1e-6)
    u = normal_bf16((2, 512), 16)
    two_u = f32_to_bf16(2 * bf16_to_f32(u))
    m1 = orc.silu_mul(np.concatenate([g, u], axis=1))
    m2 = orc.silu_mul(np.concatenate([g, two_u], axis=1))
    assert np.array_equal(m2, 2 * m1)


def test_lm_head_argmax_known_answers(orc):
    """lm_head_argmax (lm_head_topk.jl:27-101): 1-based; a planted column wins;
    duplicated best columns resolve to the smallest index; agrees with a float64
    numpy argmax wherever the margin is not tiny."""
    K, N, B = 256, 3001, 6
    x = normal_bf16((B, K), 17)
    W = normal_bf16((N, K), 18, scale=0.1)
    res, gap = orc.lm_head_argmax(x, W, nthreads=4)
    logits = bf16_to_f32(W).astype(np.float64) @ bf16_to_f32(x).astype(np.float64).T
    ref = logits.argmax(axis=0) + 1
    ok = gap > 1e-3
    assert ok.sum() >= B - 1 and np.array_equal(res[ok], ref[ok])
    # plant: column 2000 (1-based 2001) is 10 x_0; its copy at column 77 (1-based 78)
    W2 = W.copy()
    W2[2000] = f32_to_bf16(10 * bf16_to_f32(x[0]))
    res2, _ = orc.lm_head_argmax(x[:1], W2)
    assert res2[0] == 2001
    W2[77] = W2[2000]
    res3, gap3 = orc.lm_head_argmax(x[:1], W2)
    assert res3[0] == 78 and gap3[0] == 0.0


def test_model_step_identity_model(orc):
    """step! (qwen35.jl:245-273) with every projection zero and a tied head: the
    mixer and the MLP add nothing, xn = rms_norm(E[token]) (norm weights 0, offset
    1), and the greedy next token is the input token itself (|E_t|^2 ~ Dm dwarfs
    E_v . E_t): pins the 1-based embedding gather, the norm chain and the head's
    index convention together."""
    Dm, I, V, B, ctx = 256, 64, 500, 3, 16
    E = normal_bf16((V, Dm), 19)
    z = lambda *s: np.zeros(s, np.uint16)  # noqa: E731
    layer = dict(norm1=z(Dm), norm2=z(Dm), Wqkv=z(S * D, Dm), Wo=z(Dm, HQ * D), qw=z(D), kw=z(D),
                 kc=normal_bf16((B, HK, ctx, D), 20), vc=normal_bf16((B, HK, ctx, D), 21),
                 Wgu=z(2 * I, Dm), Wd=z(Dm, I))
    c, s = orc.rope_tables(HALF, ctx, THETA)
    tokens = np.array([1, 250, 500], np.int32)
    res, gap, xn = orc.model_step(E, [layer, dict(layer)], z(Dm), E, tokens,
                                  np.array([5, 9, 16], np.int32), c, s, Hq=HQ, Hk=HK, eps=EPS)
    assert np.array_equal(res, tokens)
    xe = bf16_to_f32(E[tokens - 1])
    want = xe / np.sqrt((xe.astype(np.float64) ** 2).mean(axis=1, keepdims=True) + EPS)
    assert np.allclose(xn, want, rtol=1e-2, atol=1e-2)
