"""CPU fp32 oracle for the gated full-attention path and the linear-attention
(DeltaNet + conv1d) layer parts — TEST INFRASTRUCTURE.

Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
may import this package, and only as the checker (never as the measured or
shipped path). ``liboracle.so`` is built from ``oracle.c`` and ``deltanet.c`` by
``oracle/Makefile``.

Parity pinning (the reference ships no golden vectors or known-answer tests for
this path; its tests cover checkpoint loaders only, test/runtests.jl:48-207):
every function here is checked in tests/test_oracle.py against an independent
library or closed form — torch.nn.functional.rms_norm, complex-number rotation,
torch scaled_dot_product_attention (fp32, CPU), the relative-position and
scale invariances, and brute-force special cases — see that file's docstrings.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

from .rng import normal_bf16, bf16_to_f32, f32_to_bf16  # noqa: F401

_HERE = Path(__file__).resolve().parent
_LIB = None

_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")


def build() -> Path:
    """Compile liboracle.so with the committed Makefile (gcc, OpenMP)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _HERE / "liboracle.so"


def lib():
    global _LIB
    if _LIB is None:
        path = _HERE / "liboracle.so"
        if not path.exists():
            build()
        L = ctypes.CDLL(str(path))
        i64, i32, f32, f64 = ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_double
        L.orc_rope_tables.argtypes = [_f32p, _f32p, i32, i64, f64]
        L.orc_rope_tables.restype = None
        L.orc_head_norm_rope.argtypes = [_f32p, _f32p, f32, f32, _f32p, _f32p, i64, i32, i32, _f32p]
        L.orc_head_norm_rope.restype = None
        L.orc_attention.argtypes = [_f32p, _f32p, _f32p, _f32p, ctypes.c_void_p, ctypes.c_void_p,
                                    i32, i32, i32, i32, i32, i32, i32, i32, i32, i32]
        L.orc_attention.restype = None
        L.orc_gated_decode.argtypes = [_u16p, _u16p, _u16p, i64, _i32p, _u16p, _u16p, _f32p, _f32p,
                                       i32, i32, i32, i32, i32, f32, f32, _f32p, _f32p, _f32p, i32]
        L.orc_gated_decode.restype = None
        L.orc_gated_prefill.argtypes = [_u16p, _u16p, _u16p, i64, _i32p, _i32p, _u16p, _u16p,
                                        _f32p, _f32p, i32, i32, i32, i32, i32, i32, f32, f32,
                                        _f32p, _f32p, _f32p, i32, i32]
        L.orc_gated_prefill.restype = None
        L.orc_linear.argtypes = [_u16p, _u16p, _f32p, i32, i32, i32, i32]
        L.orc_linear.restype = None
        L.orc_rms_norm.argtypes = [_u16p, ctypes.c_void_p, _u16p, ctypes.c_void_p, _f32p, i32, i32,
                                   f32, f32]
        L.orc_rms_norm.restype = None
        L.orc_silu_mul.argtypes = [_u16p, _f32p, i32, i32]
        L.orc_silu_mul.restype = None
        L.orc_lm_head_argmax.argtypes = [_u16p, _u16p, i32, i32, i32, _i32p, _f32p, i32]
        L.orc_lm_head_argmax.restype = None
        L.orc_max_threads.restype = i32
        vp = ctypes.c_void_p
        L.orc_conv1d_update.argtypes = [_u16p, _u16p, _u16p, _u16p, vp, _f32p, i32, i32, i32, i32]
        L.orc_conv1d_update.restype = None
        L.orc_conv1d_sequence.argtypes = [_u16p, _u16p, vp, vp, vp, _f32p, i32, i32, i32, i32, i32]
        L.orc_conv1d_sequence.restype = None
        L.orc_deltanet_decode.argtypes = [_f32p] * 8 + [i32] * 5
        L.orc_deltanet_decode.restype = None
        L.orc_deltanet_sequence.argtypes = [_f32p] * 8 + [i32] * 6
        L.orc_deltanet_sequence.restype = None
        L.orc_fused_deltanet_decode.argtypes = [_u16p] * 6 + [_f32p, _f32p, _u16p, _f32p, _f32p,
                                                              _f32p] + [i32] * 5 + [f32]
        L.orc_fused_deltanet_decode.restype = None
        L.orc_deltanet_prep.argtypes = [_u16p, _u16p, _f32p, _f32p] + [_f32p] * 5 + [i32] * 6
        L.orc_deltanet_prep.restype = None
        L.orc_gated_rms_norm.argtypes = [_f32p, _u16p, i64, _u16p, _f32p, i32, i32, i32, i32, f32]
        L.orc_gated_rms_norm.restype = None
        _LIB = L
    return _LIB


def max_threads() -> int:
    return int(lib().orc_max_threads())


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def rope_tables(half: int, ctx: int, theta: float):
    """(cos, sin) as [ctx][half] fp32 — src/llm/qwen35.jl:115-119."""
    c = np.empty((ctx, half), np.float32)
    s = np.empty((ctx, half), np.float32)
    lib().orc_rope_tables(c, s, half, ctx, float(theta))
    return c, s


def head_norm_rope(x, w, eps, w_offset, cos_tab, sin_tab, pos):
    """rope(rmsnorm(x) * (w + w_offset), pos) for one head vector (fp32)."""
    x = _c(x, np.float32)
    y = np.empty_like(x)
    half = cos_tab.shape[1]
    lib().orc_head_norm_rope(x, _c(w, np.float32), eps, w_offset, _c(cos_tab, np.float32),
                             _c(sin_tab, np.float32), int(pos), x.shape[0], half, y)
    return y


def attention(q, k, v, *, causal, k_lengths=None, q_lengths=None, row_step=1, nthreads=0):
    """o = softmax(q k^T / sqrt(Dk)) v per (b, h); q [B][H][L][Dk], k [B][Hk][Lk][Dk],
    v [B][Hk][Lk][Dv] fp32 -> o [B][H][L][Dv].

    src/kernels/attention.jl:12-91: GQA head h uses kv head h // (H/Hk); causal
    offset k_len - q_len; o = 0 for rows with no key. Rows t >= q_len (and rows
    skipped by row_step) are returned as NaN.
    """
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    B, H, L, Dk = q.shape
    Hk, Lk, Dv = k.shape[1], k.shape[2], v.shape[3]
    o = np.full((B, H, L, Dv), np.nan, np.float32)
    kl = _c(k_lengths, np.int32) if k_lengths is not None else None
    ql = _c(q_lengths, np.int32) if q_lengths is not None else None
    lib().orc_attention(q, k, v, o,
                        kl.ctypes.data if kl is not None else None,
                        ql.ctypes.data if ql is not None else None,
                        B, H, Hk, L, Lk, Dk, Dv, int(bool(causal)), int(row_step),
                        int(nthreads))
    return o


def gated_decode(qkv, kc, vc, positions, qw, kw, cos_tab, sin_tab, *, Hq, Hk, eps, w_offset,
                 nthreads=0):
    """One decode step of the attention layer (src/llm/qwen35.jl:187-208).

    qkv [B][2Hq+2Hk][D] bf16 bits, kc/vc [B][Hk][ctx][D] bf16 bits, positions
    [B] (1-based column of the new token). Returns (out [B][Hq][D],
    k_new [B][Hk][D], v_new [B][Hk][D]) in fp32.
    """
    qkv, kc, vc = _c(qkv, np.uint16), _c(kc, np.uint16), _c(vc, np.uint16)
    B, S, D = qkv.shape
    assert S == 2 * Hq + 2 * Hk
    ctx = kc.shape[2]
    out = np.empty((B, Hq, D), np.float32)
    kn = np.empty((B, Hk, D), np.float32)
    vn = np.empty((B, Hk, D), np.float32)
    lib().orc_gated_decode(qkv, kc, vc, ctx, _c(positions, np.int32), _c(qw, np.uint16),
                           _c(kw, np.uint16), _c(cos_tab, np.float32), _c(sin_tab, np.float32),
                           B, Hq, Hk, D, cos_tab.shape[1], eps, w_offset, out, kn, vn,
                           int(nthreads))
    return out, kn, vn


def gated_prefill(qkv, kc, vc, prior, q_len, qw, kw, cos_tab, sin_tab, *, Hq, Hk, eps, w_offset,
                  row_step=1, nthreads=0):
    """Chunked prefill of the attention layer (src/llm/qwen35.jl:292-318), ragged.

    qkv [B][T][2Hq+2Hk][D] bf16 bits; kc/vc [B][Hk][ctx][D] bf16 bits holding
    prior[b] cached tokens; q_len[b] chunk lengths. Returns (out [B][T][Hq][D],
    k_new [B][Hk][T][D], v_new [B][Hk][T][D]) in fp32; unevaluated rows are NaN.
    """
    qkv, kc, vc = _c(qkv, np.uint16), _c(kc, np.uint16), _c(vc, np.uint16)
    B, T, S, D = qkv.shape
    assert S == 2 * Hq + 2 * Hk
    ctx = kc.shape[2]
    out = np.full((B, T, Hq, D), np.nan, np.float32)
    kn = np.full((B, Hk, T, D), np.nan, np.float32)
    vn = np.full((B, Hk, T, D), np.nan, np.float32)
    lib().orc_gated_prefill(qkv, kc, vc, ctx, _c(prior, np.int32), _c(q_len, np.int32),
                            _c(qw, np.uint16), _c(kw, np.uint16), _c(cos_tab, np.float32),
                            _c(sin_tab, np.float32), B, T, Hq, Hk, D, cos_tab.shape[1], eps,
                            w_offset, out, kn, vn, int(row_step), int(nthreads))
    return out, kn, vn


def linear(x, W, *, nthreads=0):
    """y = W^T x in fp32 (src/linear.jl:40-57): x [..][K] bf16 bits (the reference's
    (K, N)), W [M][K] bf16 bits (the reference's K-major (K, M)) -> y [..][M]."""
    x = _c(x, np.uint16)
    W = _c(W, np.uint16)
    M, K = W.shape
    lead = x.shape[:-1]
    assert x.shape[-1] == K
    N = int(np.prod(lead)) if lead else 1
    y = np.empty(lead + (M,), np.float32)
    lib().orc_linear(x.reshape(N, K), W, y.reshape(N, M), M, N, K, int(nthreads))
    return y


def decode_layer(xn, Wqkv, Wo, kc, vc, positions, qw, kw, cos_tab, sin_tab, *, Hq, Hk, eps,
                 w_offset, nthreads=0):
    """decode!(h, ::AttnLayer, m, gen, xn) (src/llm/qwen35.jl:187-208) for one step:
    xn [B][Dm] bf16 bits -> h [B][Dm] fp32. The reference keeps qkv and the gated
    attention output in bf16 buffers (qwen35.jl:193, :205); they are rounded to bf16
    (RNE) here at those two points, everything else is fp32. Also returns the
    appended (k_new, v_new) rows."""
    B = xn.shape[0]
    D = kc.shape[-1]
    S = 2 * Hq + 2 * Hk
    qkv = f32_to_bf16(linear(xn, Wqkv, nthreads=nthreads)).reshape(B, S, D)
    o, kn, vn = gated_decode(qkv, kc, vc, positions, qw, kw, cos_tab, sin_tab, Hq=Hq, Hk=Hk,
                             eps=eps, w_offset=w_offset, nthreads=nthreads)
    h = linear(f32_to_bf16(o).reshape(B, Hq * D), Wo, nthreads=nthreads)
    return h, kn, vn


def prefill_layer(xn, Wqkv, Wo, kc, vc, prior, q_len, qw, kw, cos_tab, sin_tab, *, Hq, Hk, eps,
                  w_offset, row_step=1, nthreads=0):
    """forward(::AttnLayer, m, xn, T, B; offset) (src/llm/qwen35.jl:292-318), ragged:
    xn [B][T][Dm] bf16 bits -> h [B][T][Dm] fp32 (rows not evaluated are NaN). qkv
    and the gated attention output are rounded to bf16 as the reference stores
    them (qwen35.jl:296, :312-315)."""
    B, T = xn.shape[:2]
    D = kc.shape[-1]
    S = 2 * Hq + 2 * Hk
    qkv = f32_to_bf16(linear(xn, Wqkv, nthreads=nthreads)).reshape(B, T, S, D)
    o, kn, vn = gated_prefill(qkv, kc, vc, prior, q_len, qw, kw, cos_tab, sin_tab, Hq=Hq, Hk=Hk,
                              eps=eps, w_offset=w_offset, row_step=row_step, nthreads=nthreads)
    o = o.reshape(B, T, Hq * D)
    rows = ~np.isnan(o[..., 0])
    h = np.full((B, T, Wo.shape[0]), np.nan, np.float32)
    h[rows] = linear(f32_to_bf16(o[rows]), Wo, nthreads=nthreads)
    return h, kn, vn


def rms_norm(x, w, *, eps, offset, dx=None):
    """rms_norm! (src/kernels/rms_norm.jl:3-31), or fused_add_rms_norm!
    (src/kernels/residual_norm.jl:4-37) when dx is given: x, dx [N][M] bf16 bits
    (the reference's (M, N) columns), w [M]. Returns y [N][M] fp32, and with dx
    also x' = x + dx [N][M] fp32 (y is formed from bf16(x'), as the reference
    reloads the stored x')."""
    x = _c(x, np.uint16)
    N, M = x.shape
    y = np.empty((N, M), np.float32)
    xo = np.empty((N, M), np.float32) if dx is not None else None
    dxc = _c(dx, np.uint16) if dx is not None else None
    lib().orc_rms_norm(x, dxc.ctypes.data if dxc is not None else None, _c(w, np.uint16),
                       xo.ctypes.data if xo is not None else None, y, M, N, eps, offset)
    return (y, xo) if dx is not None else y


def silu_mul(gu):
    """mid = silu(gate) .* up (src/llm/qwen35.jl:234-243): gu [N][2I] bf16 bits ->
    mid [N][I] fp32."""
    gu = _c(gu, np.uint16)
    N, I2 = gu.shape
    mid = np.empty((N, I2 // 2), np.float32)
    lib().orc_silu_mul(gu, mid, I2 // 2, N)
    return mid


def lm_head_argmax(x, W, *, nthreads=0):
    """lm_head_argmax! (src/kernels/lm_head_topk.jl:27-101): x [B][K], W [N][K] bf16
    bits (the reference's (K, B) and K-major (K, N)). Returns (result [B] int32,
    1-based, ties to the smallest index; gap [B]: best minus second-best logit)."""
    x = _c(x, np.uint16)
    W = _c(W, np.uint16)
    B, K = x.shape
    N = W.shape[0]
    res = np.empty(B, np.int32)
    gap = np.empty(B, np.float32)
    lib().orc_lm_head_argmax(x, W, K, N, B, res, gap, nthreads or threads_env())
    return res, gap


def deltanet_decode_layer(xn, l, *, Dk, Dv, Hk, Hv, eps, nthreads=0):
    """decode!(h, l::DeltaNetLayer, m, gen, xn) (src/llm/qwen35.jl:210-232) for
    one step: xn [B][Dm] bf16 bits -> (h [B][Dm] fp32, new ring, new state).
    The reference's bf16 buffers (qz, ab, the conv output, O) are rounded to
    bf16 (RNE) at those points. l: dict with Wqz, Wab, Wout, conv_w, conv_b (or
    None), ring [B][K][n], A_log, dt_bias, gnorm_w, S [B][Hv][Dv][Dk]."""
    B = xn.shape[0]
    n = 2 * Hk * Dk + Hv * Dv
    qz = f32_to_bf16(linear(xn, l["Wqz"], nthreads=nthreads))
    ab = f32_to_bf16(linear(xn, l["Wab"], nthreads=nthreads))
    y, ring = conv1d_update(qz[:, :n], l["ring"], l["conv_w"], l.get("conv_b"), act=True)
    y = f32_to_bf16(y)
    hk = Hk * Dk
    o, S = fused_deltanet_decode(
        y[:, :hk].reshape(B, Hk, Dk), y[:, hk:2 * hk].reshape(B, Hk, Dk),
        y[:, 2 * hk:].reshape(B, Hv, Dv), ab[:, :Hv], ab[:, Hv:], qz[:, n:].reshape(B, Hv, Dv),
        l["A_log"], l["dt_bias"], l["gnorm_w"], l["S"], eps=eps)
    h = linear(f32_to_bf16(o).reshape(B, Hv * Dv), l["Wout"], nthreads=nthreads)
    return h, ring, S


def model_step(E, layers, norm_w, head, result, positions, cos_tab, sin_tab, *, Hq, Hk, eps,
               nthreads=0, linear_cfg=None):
    """step!(m, gen) (src/llm/qwen35.jl:245-273) for a stack of attention and
    DeltaNet layers (dicts with kind "linear_attention", see deltanet_decode_layer;
    linear_cfg = dict(Dk, Dv, Hk, Hv)), greedy. The reference's step buffers are
    bf16 (the residual x, xn, h, the MLP's gu and mid, qwen35.jl:235-250): every
    value is rounded to bf16 (RNE) where the reference stores it, everything
    else is fp32.

    E, head [vocab][Dm]; norm_w [Dm]; layers: dicts with norm1, norm2, Wqkv, Wo,
    qw, kw, kc, vc (caches [B][Hk][ctx][D]), Wgu [2I][Dm], Wd [Dm][I] (bf16 bits);
    result [B] 1-based tokens; positions [B]. Returns (next tokens [B] int32,
    logit gaps [B], final xn [B][Dm] fp32 of the bf16 values)."""
    r = np.clip(np.asarray(result, np.int64) - 1, 0, E.shape[0] - 1)
    x = _c(E[r], np.uint16)
    xn = f32_to_bf16(rms_norm(x, layers[0]["norm1"], eps=eps, offset=1.0))
    for i, l in enumerate(layers):
        if l.get("kind") == "linear_attention":
            h, _, _ = deltanet_decode_layer(xn, l, eps=eps, nthreads=nthreads, **linear_cfg)
        else:
            h, _, _ = decode_layer(xn, l["Wqkv"], l["Wo"], l["kc"], l["vc"], positions, l["qw"],
                                   l["kw"], cos_tab, sin_tab, Hq=Hq, Hk=Hk, eps=eps, w_offset=1.0,
                                   nthreads=nthreads)
        y, xo = rms_norm(x, l["norm2"], eps=eps, offset=1.0, dx=f32_to_bf16(h))
        x, xn = f32_to_bf16(xo), f32_to_bf16(y)
        gu = f32_to_bf16(linear(xn, l["Wgu"], nthreads=nthreads))
        h = linear(f32_to_bf16(silu_mul(gu)), l["Wd"], nthreads=nthreads)
        nw = norm_w if i == len(layers) - 1 else layers[i + 1]["norm1"]
        y, xo = rms_norm(x, nw, eps=eps, offset=1.0, dx=f32_to_bf16(h))
        x, xn = f32_to_bf16(xo), f32_to_bf16(y)
    res, gap = lm_head_argmax(xn, head, nthreads=nthreads)
    return res, gap, bf16_to_f32(xn)


def deltanet_prefill_layer(xn, l, *, Dk, Dv, Hk, Hv, eps, offset, nthreads=0):
    """forward(l::DeltaNetLayer, m, xn, T, B; offset) (src/llm/qwen35.jl:320-365):
    xn [B][T][Dm] bf16 bits -> (h [B][T][Dm] fp32, new ring, new state). qz, ab
    and the conv output are bf16 buffers in the reference (:322-323, :328), as
    is the gated norm's output fed to Wout (:363-364): rounded there. A suffix
    (offset > 0) takes its conv's left context from the ring (:333-344). l: as
    deltanet_decode_layer."""
    B, T, Dm = xn.shape
    n = 2 * Hk * Dk + Hv * Dv
    x2 = _c(xn, np.uint16).reshape(B * T, Dm)
    qz = f32_to_bf16(linear(x2, l["Wqz"], nthreads=nthreads)).reshape(B, T, -1)
    ab = f32_to_bf16(linear(x2, l["Wab"], nthreads=nthreads)).reshape(B, T, 2 * Hv)
    conv, ring = conv1d_sequence(np.ascontiguousarray(qz[..., :n]), l["conv_w"], l.get("conv_b"),
                                 s_in=l["ring"] if offset > 0 else None, act=True)
    p = deltanet_prep(f32_to_bf16(conv), ab, l["A_log"], l["dt_bias"], Dk=Dk, Dv=Dv, Hk=Hk, Hv=Hv)
    o, S = deltanet_sequence(p["q"], p["k"], p["v"], p["beta"], p["gate"], l["S"])
    y = gated_rms_norm(o, np.ascontiguousarray(qz[..., n:]), l["gnorm_w"], eps=eps)
    h = linear(f32_to_bf16(y).reshape(B * T, Hv * Dv), l["Wout"], nthreads=nthreads)
    return h.reshape(B, T, Dm), ring, S


def prefill_model(E, layers, norm_w, head, ids, offset, cos_tab, sin_tab, *, Hq, Hk, eps,
                  nthreads=0, linear_cfg=None):
    """prefill!(m, gen, ids; offset) (src/llm/qwen35.jl:369-395), greedy: ids [B][T]
    1-based tokens continuing `offset` resident ones. Layers as model_step: the
    attention layers' caches hold `offset` prior rows, the DeltaNet layers' ring
    and state carry the prefix. The residual x, xn, h, gu and mid are bf16 in
    the reference (:375-388): rounded there. Returns (next tokens [B], logit gaps
    [B], the last token's final xn [B][Dm] fp32, new states: per layer (K cache,
    V cache) or (ring, S))."""
    ids = np.asarray(ids, np.int64)
    B, T = ids.shape
    Dm = E.shape[1]
    x = _c(E[np.clip(ids - 1, 0, E.shape[0] - 1)], np.uint16).reshape(B * T, Dm)
    xn = f32_to_bf16(rms_norm(x, layers[0]["norm1"], eps=eps, offset=1.0))
    states = []
    for i, l in enumerate(layers):
        if l.get("kind") == "linear_attention":
            h, ring, S = deltanet_prefill_layer(xn.reshape(B, T, Dm), l, eps=eps, offset=offset,
                                                nthreads=nthreads, **linear_cfg)
            states.append((ring, S))
        else:
            prior = np.full(B, offset, np.int32)
            h, kn, vn = prefill_layer(xn.reshape(B, T, Dm), l["Wqkv"], l["Wo"], l["kc"], l["vc"],
                                      prior, np.full(B, T, np.int32), l["qw"], l["kw"], cos_tab,
                                      sin_tab, Hq=Hq, Hk=Hk, eps=eps, w_offset=1.0,
                                      nthreads=nthreads)
            kc, vc = _c(l["kc"], np.uint16).copy(), _c(l["vc"], np.uint16).copy()
            kc[:, :, offset:offset + T] = f32_to_bf16(kn)
            vc[:, :, offset:offset + T] = f32_to_bf16(vn)
            states.append((kc, vc))
        y, xo = rms_norm(x, l["norm2"], eps=eps, offset=1.0, dx=f32_to_bf16(h.reshape(B * T, Dm)))
        x, xn = f32_to_bf16(xo), f32_to_bf16(y)
        gu = f32_to_bf16(linear(xn, l["Wgu"], nthreads=nthreads))
        h = linear(f32_to_bf16(silu_mul(gu)), l["Wd"], nthreads=nthreads)
        nw = norm_w if i == len(layers) - 1 else layers[i + 1]["norm1"]
        y, xo = rms_norm(x, nw, eps=eps, offset=1.0, dx=f32_to_bf16(h))
        x, xn = f32_to_bf16(xo), f32_to_bf16(y)
    last = np.ascontiguousarray(xn.reshape(B, T, Dm)[:, T - 1])
    res, gap = lm_head_argmax(last, head, nthreads=nthreads)
    return res, gap, bf16_to_f32(last), states


# ---- linear-attention layer parts (oracle/deltanet.c) -----------------------

def _vp(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def conv1d_update(x, s, w, bias=None, *, act=True):
    """causal_conv1d! (src/kernels/causal_conv1d.jl:7-61), one step: x [B][D],
    ring s [B][K][D], w [K][D], bias [D] or None (bf16 bits). Returns (y [B][D]
    fp32, the shifted ring [B][K][D] bf16 bits)."""
    x, s, w = _c(x, np.uint16), _c(s, np.uint16), _c(w, np.uint16)
    bias = None if bias is None else _c(bias, np.uint16)
    B, K, D = s.shape
    y = np.empty((B, D), np.float32)
    so = np.empty_like(s)
    lib().orc_conv1d_update(x, s, so, w, _vp(bias), y, D, K, B, int(bool(act)))
    return y, so


def conv1d_sequence(x, w, bias=None, *, s_in=None, act=True):
    """causal_conv1d_sequence! (causal_conv1d.jl:73-149): x [B][T][D] -> (y
    [B][T][D] fp32, the seeded ring [B][K][D]); s_in (a prefix's ring) supplies
    the left context of a suffix (qwen35.jl:333-344), zeros when None."""
    x, w = _c(x, np.uint16), _c(w, np.uint16)
    bias = None if bias is None else _c(bias, np.uint16)
    s_in = None if s_in is None else _c(s_in, np.uint16)
    B, T, D = x.shape
    K = w.shape[0]
    y = np.empty((B, T, D), np.float32)
    so = np.empty((B, K, D), np.uint16)
    lib().orc_conv1d_sequence(x, w, _vp(bias), _vp(s_in), _vp(so), y, D, K, T, B,
                              int(bool(act)))
    return y, so


def deltanet_decode(q, k, v, beta, gate, s):
    """deltanet_recurrent_decode! (src/kernels/deltanet_recurrent.jl:15-95), fp32:
    q, k [B][Hk][Dk], v [B][Hv][Dv], beta, gate [B][Hv], s [B][Hv][Dv][Dk].
    Returns (o [B][Hv][Dv], new state)."""
    q, k, v, beta, gate, s = (_c(a, np.float32) for a in (q, k, v, beta, gate, s))
    B, Hk, Dk = q.shape
    Hv, Dv = v.shape[1], v.shape[2]
    o = np.empty((B, Hv, Dv), np.float32)
    so = np.empty_like(s)
    lib().orc_deltanet_decode(q, k, v, beta, gate, s, so, o, Dk, Dv, Hk, Hv, B)
    return o, so


def deltanet_sequence(q, k, v, beta, gate, s):
    """deltanet_sequence! (deltanet_recurrent.jl:109-198), fp32: q, k
    [B][Hk][T][Dk], v [B][Hv][T][Dv], beta, gate [B][T][Hv], s [B][Hv][Dv][Dk].
    Returns (o [B][Hv][T][Dv], final state)."""
    q, k, v, beta, gate, s = (_c(a, np.float32) for a in (q, k, v, beta, gate, s))
    B, Hk, T, Dk = q.shape
    Hv, Dv = v.shape[1], v.shape[3]
    o = np.empty((B, Hv, T, Dv), np.float32)
    so = np.empty_like(s)
    lib().orc_deltanet_sequence(q, k, v, beta, gate, s, so, o, Dk, Dv, T, Hk, Hv, B)
    return o, so


def fused_deltanet_decode(q, k, v, alpha, beta_raw, z, a_log, dt_bias, norm_w, s, *, eps):
    """fused_deltanet_decode! (src/kernels/deltanet_fused.jl:27-141): q, k
    [B][Hk][Dk], v, z [B][Hv][Dv], alpha, beta_raw [B][Hv], norm_w [Dv] bf16
    bits; a_log, dt_bias [Hv], s [B][Hv][Dv][Dk] fp32. Returns (o [B][Hv][Dv]
    fp32, new state)."""
    q, k, v, alpha, beta_raw, z, norm_w = (_c(a, np.uint16)
                                           for a in (q, k, v, alpha, beta_raw, z, norm_w))
    a_log, dt_bias, s = (_c(a, np.float32) for a in (a_log, dt_bias, s))
    B, Hk, Dk = q.shape
    Hv, Dv = v.shape[1], v.shape[2]
    o = np.empty((B, Hv, Dv), np.float32)
    so = np.empty_like(s)
    lib().orc_fused_deltanet_decode(q, k, v, alpha, beta_raw, z, a_log, dt_bias, norm_w, s, so,
                                    o, Dk, Dv, Hk, Hv, B, float(eps))
    return o, so


def deltanet_prep(cv, ab, a_log, dt_bias, *, Dk, Dv, Hk, Hv):
    """The prefill's inputs to deltanet_sequence! (src/llm/qwen35.jl:347-356):
    cv [B][T][2 Hk Dk + Hv Dv], ab [B][T][2 Hv] bf16 bits. Returns dict q, k
    [B][Hk][T][Dk], v [B][Hv][T][Dv], beta, gate [B][T][Hv] (fp32)."""
    cv, ab = _c(cv, np.uint16), _c(ab, np.uint16)
    a_log, dt_bias = _c(a_log, np.float32), _c(dt_bias, np.float32)
    B, T, _ = cv.shape
    out = dict(q=np.empty((B, Hk, T, Dk), np.float32), k=np.empty((B, Hk, T, Dk), np.float32),
               v=np.empty((B, Hv, T, Dv), np.float32), beta=np.empty((B, T, Hv), np.float32),
               gate=np.empty((B, T, Hv), np.float32))
    lib().orc_deltanet_prep(cv, ab, a_log, dt_bias, out["q"], out["k"], out["v"], out["beta"],
                            out["gate"], Dk, Dv, Hk, Hv, T, B)
    return out


def gated_rms_norm(o, z, norm_w, *, eps):
    """The prefill epilogue (qwen35.jl:360-364): o [B][Hv][T][Dv] fp32, z
    [B][T][Hv Dv] bf16 bits -> y [B][T][Hv][Dv] fp32 = o rstd norm_w silu(z)."""
    o = _c(o, np.float32)
    z, norm_w = _c(z, np.uint16), _c(norm_w, np.uint16)
    B, Hv, T, Dv = o.shape
    y = np.empty((B, T, Hv, Dv), np.float32)
    lib().orc_gated_rms_norm(o, z, z.shape[-1], norm_w, y, Dv, Hv, T, B, float(eps))
    return y


def threads_env() -> int:
    """OpenMP threads the oracle will use (OMP_NUM_THREADS or all cores)."""
    n = os.environ.get("OMP_NUM_THREADS")
    return int(n) if n else max_threads()
