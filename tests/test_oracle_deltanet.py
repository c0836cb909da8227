"""Pins of the CPU oracle's linear-attention parts (oracle/deltanet.c) — CPU only.

The reference holds no known-answer tests for these kernels either, so each
oracle function is checked against an independent formulation chosen so that a
plausible slip fails one of them (ring shifted the wrong way, kernel taps
reversed, bias or silu dropped, decay applied after the rank-1 update instead of
before, beta applied to the wrong term, the q/k head map h / (Hv/Hk) swapped for
h % Hk, q's 1/sqrt(Dk) dropped, rms instead of l2 norm, softplus / sigmoid
mixed up, the gated norm over the wrong axis):

  conv1d_sequence   numpy.convolve per channel (zero-padded, taps oldest
                    first); the seeded ring == the last K inputs; a suffix run
                    from the prefix's ring == the full run's matching rows
  conv1d_update     T chained steps == the sequence run, bit for bit, and the
                    final ring == the sequence's seed
  deltanet_decode   the delta rule's defining property (beta = 1, |k| = 1:
                    S'^T k = v after the step); beta = 0: S' = decay S and
                    o = S'^T q; the GQA head map on distinct qk heads
  deltanet_sequence the product form S_t = d_t (I - b_t k_t k_t^T) S_{t-1} +
                    b_t k_t v_t^T, o_t = S_t^T q_t in float64; T chained decode
                    steps == one sequence run
  fused decode      numpy l2 norms, expit / logaddexp gates, float64 delta step
                    and the gated RMSNorm, composed independently
  prep / gated norm numpy restatements of qwen35.jl:347-364; the fused decode
                    == prep + decode + gated norm on one token
"""
from __future__ import annotations

import numpy as np
from scipy.special import expit

import oracle
from oracle.rng import bf16_to_f32, f32_to_bf16, normal_bf16, normal_f32


def _f(a):
    return bf16_to_f32(a).astype(np.float64)


def _silu(x):
    return x * expit(x)


# ---------------------------------------------------------------- conv1d
def test_conv1d_sequence_is_numpy_convolve():
    B, T, D, K = 2, 9, 24, 4
    x = normal_bf16((B, T, D), 11)
    w = normal_bf16((K, D), 12, scale=0.5)
    bias = normal_bf16((D,), 13, scale=0.1)
    y, ring = oracle.conv1d_sequence(x, w, bias, act=True)
    y0, _ = oracle.conv1d_sequence(x, w, None, act=False)
    xf, wf, bf = _f(x), _f(w), _f(bias)
    for b in range(B):
        for d in range(D):
            # y[t] = sum_k w[k] x[t - K + 1 + k]: a full convolution with the taps
            # reversed (newest input meets w[K-1]), first T outputs
            ref = np.convolve(xf[b, :, d], wf[::-1, d])[:T]
            np.testing.assert_allclose(y0[b, :, d], ref, rtol=1e-5, atol=1e-5)
            np.testing.assert_allclose(y[b, :, d], _silu(ref + bf[d]), rtol=1e-5, atol=1e-5)
    # the seeded ring holds the last K raw inputs, newest in column K
    assert np.array_equal(ring, x[:, T - K:, :])


def test_conv1d_sequence_short_input_pads_the_ring_with_zeros():
    B, T, D, K = 1, 2, 8, 4
    x = normal_bf16((B, T, D), 21)
    w = normal_bf16((K, D), 22)
    _, ring = oracle.conv1d_sequence(x, w)
    assert not ring[:, :K - T].any()
    assert np.array_equal(ring[:, K - T:], x)


def test_conv1d_suffix_from_the_prefix_ring():
    B, T, D, K, P = 2, 11, 16, 4, 5
    x = normal_bf16((B, T, D), 31)
    w = normal_bf16((K, D), 32)
    bias = normal_bf16((D,), 33)
    y_full, ring_full = oracle.conv1d_sequence(x, w, bias)
    _, ring_p = oracle.conv1d_sequence(x[:, :P], w, bias)
    y_s, ring_s = oracle.conv1d_sequence(x[:, P:], w, bias, s_in=ring_p)
    assert np.array_equal(y_s, y_full[:, P:])
    assert np.array_equal(ring_s, ring_full)


def test_conv1d_update_chain_is_the_sequence():
    B, T, D, K = 3, 7, 40, 4
    x = normal_bf16((B, T, D), 41)
    w = normal_bf16((K, D), 42)
    bias = normal_bf16((D,), 43)
    y_seq, ring_seq = oracle.conv1d_sequence(x, w, bias)
    ring = np.zeros((B, K, D), np.uint16)
    for t in range(T):
        y, ring = oracle.conv1d_update(x[:, t], ring, w, bias)
        assert np.array_equal(y, y_seq[:, t])
    assert np.array_equal(ring, ring_seq)


# ---------------------------------------------------------------- delta rule
def _unit(v, axis=-1):
    return v / np.linalg.norm(v, axis=axis, keepdims=True)


def test_delta_rule_writes_v_under_unit_key():
    """beta = 1, |k| = 1: after the step the state maps k to v exactly (the
    delta rule replaces the value stored under k), whatever the decay."""
    B, Hk, Hv, Dk, Dv = 2, 2, 4, 32, 24
    rng = np.random.default_rng(5)
    q = rng.standard_normal((B, Hk, Dk)).astype(np.float32)
    k = _unit(rng.standard_normal((B, Hk, Dk))).astype(np.float32)
    v = rng.standard_normal((B, Hv, Dv)).astype(np.float32)
    beta = np.ones((B, Hv), np.float32)
    gate = rng.uniform(-2, 0, (B, Hv)).astype(np.float32)
    s = rng.standard_normal((B, Hv, Dv, Dk)).astype(np.float32)
    _, s1 = oracle.deltanet_decode(q, k, v, beta, gate, s)
    for b in range(B):
        for h in range(Hv):
            hk = h // (Hv // Hk)
            np.testing.assert_allclose(s1[b, h] @ k[b, hk], v[b, h], rtol=1e-4, atol=1e-4)


def test_delta_rule_beta_zero_is_pure_decay():
    B, Hk, Hv, Dk, Dv = 1, 1, 3, 16, 8
    rng = np.random.default_rng(6)
    q, k = (rng.standard_normal((B, Hk, Dk)).astype(np.float32) for _ in range(2))
    v = rng.standard_normal((B, Hv, Dv)).astype(np.float32)
    gate = np.array([[0.0, -0.5, -3.0]], np.float32)
    s = rng.standard_normal((B, Hv, Dv, Dk)).astype(np.float32)
    o, s1 = oracle.deltanet_decode(q, k, v, np.zeros((B, Hv), np.float32), gate, s)
    d = np.exp(gate.astype(np.float64))[..., None, None]
    np.testing.assert_allclose(s1, d * s, rtol=1e-6)
    np.testing.assert_allclose(o, np.einsum("bhcd,bd->bhc", s1, q[:, 0]), rtol=1e-5, atol=1e-6)


def _product_form(q, k, v, beta, gate, s):
    """float64: S_t = d_t (I - b_t k k^T) S_{t-1} + b_t k v^T with S (Dk, Dv);
    o_t = S_t^T q_t. q, k [B][Hk][T][Dk]; v [B][Hv][T][Dv]; s [B][Hv][Dv][Dk]."""
    B, Hk, T, Dk = q.shape
    Hv = v.shape[1]
    S = np.swapaxes(s.astype(np.float64), -1, -2).copy()  # [B][Hv][Dk][Dv]
    o = np.empty(v.shape, np.float64)
    for b in range(B):
        for h in range(Hv):
            hk = h // (Hv // Hk)
            for t in range(T):
                kt = k[b, hk, t].astype(np.float64)
                bt, dt = float(beta[b, t, h]), float(np.exp(np.float64(gate[b, t, h])))
                S[b, h] = dt * (np.eye(Dk) - bt * np.outer(kt, kt)) @ S[b, h] + bt * np.outer(
                    kt, v[b, h, t])
                o[b, h, t] = S[b, h].T @ q[b, hk, t]
    return o, np.swapaxes(S, -1, -2)


def test_deltanet_sequence_is_the_product_form():
    B, Hk, Hv, T, Dk, Dv = 2, 2, 4, 12, 16, 12
    rng = np.random.default_rng(7)
    q = (rng.standard_normal((B, Hk, T, Dk)) * 0.3).astype(np.float32)
    k = _unit(rng.standard_normal((B, Hk, T, Dk))).astype(np.float32)
    v = rng.standard_normal((B, Hv, T, Dv)).astype(np.float32)
    beta = rng.uniform(0, 1, (B, T, Hv)).astype(np.float32)
    gate = rng.uniform(-1, 0, (B, T, Hv)).astype(np.float32)
    s = rng.standard_normal((B, Hv, Dv, Dk)).astype(np.float32)
    o, s1 = oracle.deltanet_sequence(q, k, v, beta, gate, s)
    o_ref, s_ref = _product_form(q, k, v, beta, gate, s)
    np.testing.assert_allclose(o, o_ref, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(s1, s_ref, rtol=1e-4, atol=1e-4)


def test_deltanet_decode_chain_is_the_sequence():
    B, Hk, Hv, T, Dk, Dv = 1, 2, 6, 5, 8, 8
    rng = np.random.default_rng(8)
    q, k = (rng.standard_normal((B, Hk, T, Dk)).astype(np.float32) for _ in range(2))
    v = rng.standard_normal((B, Hv, T, Dv)).astype(np.float32)
    beta = rng.uniform(0, 1, (B, T, Hv)).astype(np.float32)
    gate = rng.uniform(-1, 0, (B, T, Hv)).astype(np.float32)
    s = rng.standard_normal((B, Hv, Dv, Dk)).astype(np.float32)
    o_seq, s_seq = oracle.deltanet_sequence(q, k, v, beta, gate, s)
    st = s
    for t in range(T):
        o, st = oracle.deltanet_decode(q[:, :, t], k[:, :, t], v[:, :, t], beta[:, t],
                                       gate[:, t], st)
        assert np.array_equal(o, o_seq[:, :, t])
    assert np.array_equal(st, s_seq)


def test_fused_decode_is_the_composition():
    """l2 norms (not rms), q's 1/sqrt(Dk), decay exp(-exp(A) softplus(a + dt)),
    beta sigmoid(b), the GQA map h // (Hv/Hk), then the gated RMSNorm over Dv
    with silu(z): restated in float64 numpy."""
    B, Hk, Hv, Dk, Dv, eps = 2, 2, 6, 32, 16, 1e-6
    q = normal_bf16((B, Hk, Dk), 51)
    k = normal_bf16((B, Hk, Dk), 52)
    v = normal_bf16((B, Hv, Dv), 53)
    z = normal_bf16((B, Hv, Dv), 54)
    alpha = normal_bf16((B, Hv), 55)
    beta_raw = normal_bf16((B, Hv), 56)
    norm_w = normal_bf16((Dv,), 57, scale=0.2, shift=1.0)
    a_log = normal_f32(Hv, 58, scale=0.5)
    dt_bias = normal_f32(Hv, 59, scale=0.5)
    s = normal_f32(B * Hv * Dv * Dk, 60, scale=0.1).reshape(B, Hv, Dv, Dk)
    o, s1 = oracle.fused_deltanet_decode(q, k, v, alpha, beta_raw, z, a_log, dt_bias, norm_w, s,
                                         eps=eps)
    qf, kf = _f(q), _f(k)
    qn = qf / np.sqrt((qf ** 2).sum(-1, keepdims=True) + 1e-6) / np.sqrt(Dk)
    kn = kf / np.sqrt((kf ** 2).sum(-1, keepdims=True) + 1e-6)
    decay = np.exp(-np.exp(a_log.astype(np.float64)) * np.logaddexp(0, _f(alpha) + dt_bias))
    beta = expit(_f(beta_raw))
    for b in range(B):
        for h in range(Hv):
            hk = h // (Hv // Hk)
            S = decay[b, h] * s[b, h].astype(np.float64)  # [Dv][Dk]
            delta = beta[b, h] * (_f(v)[b, h] - S @ kn[b, hk])
            S = S + np.outer(delta, kn[b, hk])
            out = S @ qn[b, hk]
            rstd = 1 / np.sqrt((out ** 2).mean() + eps)
            ref = out * rstd * _f(norm_w) * _silu(_f(z)[b, h])
            np.testing.assert_allclose(s1[b, h], S, rtol=2e-5, atol=2e-6)
            np.testing.assert_allclose(o[b, h], ref, rtol=2e-4, atol=2e-5)


def _prep_numpy(cv, ab, a_log, dt_bias, Dk, Dv, Hk, Hv):
    c = _f(cv)
    B, T, _ = c.shape
    q = c[..., :Hk * Dk].reshape(B, T, Hk, Dk)
    k = c[..., Hk * Dk:2 * Hk * Dk].reshape(B, T, Hk, Dk)
    v = c[..., 2 * Hk * Dk:].reshape(B, T, Hv, Dv)
    l2n = lambda y: y / np.sqrt((y ** 2).sum(-1, keepdims=True) + 1e-6)
    a = _f(ab)
    return dict(q=np.transpose(l2n(q) / np.sqrt(Dk), (0, 2, 1, 3)),
                k=np.transpose(l2n(k), (0, 2, 1, 3)), v=np.transpose(v, (0, 2, 1, 3)),
                beta=expit(a[..., Hv:]),
                gate=-np.exp(a_log.astype(np.float64)) * np.log1p(np.exp(a[..., :Hv] + dt_bias)))


def test_prep_and_gated_norm_are_the_reference_prefill_lines():
    B, T, Hk, Hv, Dk, Dv, eps = 2, 3, 2, 4, 16, 8, 1e-6
    n = 2 * Hk * Dk + Hv * Dv
    cv = normal_bf16((B, T, n), 61)
    ab = normal_bf16((B, T, 2 * Hv), 62)
    a_log = normal_f32(Hv, 63, scale=0.5)
    dt_bias = normal_f32(Hv, 64, scale=0.5)
    got = oracle.deltanet_prep(cv, ab, a_log, dt_bias, Dk=Dk, Dv=Dv, Hk=Hk, Hv=Hv)
    ref = _prep_numpy(cv, ab, a_log, dt_bias, Dk, Dv, Hk, Hv)
    for key in ("q", "k", "v", "beta", "gate"):
        np.testing.assert_allclose(got[key], ref[key], rtol=2e-6, atol=1e-7, err_msg=key)
    o = normal_f32(B * Hv * T * Dv, 65).reshape(B, Hv, T, Dv)
    z = normal_bf16((B, T, Hv * Dv), 66)
    norm_w = normal_bf16((Dv,), 67, scale=0.2, shift=1.0)
    y = oracle.gated_rms_norm(o, z, norm_w, eps=eps)
    of = np.transpose(o.astype(np.float64), (0, 2, 1, 3))  # [B][T][Hv][Dv]
    rstd = 1 / np.sqrt((of ** 2).mean(-1, keepdims=True) + eps)
    ref = of * rstd * _f(norm_w) * _silu(_f(z).reshape(B, T, Hv, Dv))
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-6)


def test_fused_decode_is_prep_decode_and_gated_norm():
    """The decode kernel (bf16 inputs, gates and norms inside) and the prefill's
    route (prep -> deltanet_sequence! -> gated norm) agree on one token."""
    B, Hk, Hv, Dk, Dv, eps = 2, 2, 4, 16, 16, 1e-6
    n = 2 * Hk * Dk + Hv * Dv
    cv = normal_bf16((B, 1, n), 71)
    ab = normal_bf16((B, 1, 2 * Hv), 72)
    z = normal_bf16((B, 1, Hv * Dv), 73)
    norm_w = normal_bf16((Dv,), 74, scale=0.2, shift=1.0)
    a_log = normal_f32(Hv, 75, scale=0.5)
    dt_bias = normal_f32(Hv, 76, scale=0.5)
    s = normal_f32(B * Hv * Dv * Dk, 77, scale=0.1).reshape(B, Hv, Dv, Dk)
    p = oracle.deltanet_prep(cv, ab, a_log, dt_bias, Dk=Dk, Dv=Dv, Hk=Hk, Hv=Hv)
    o_seq, s_seq = oracle.deltanet_sequence(p["q"], p["k"], p["v"], p["beta"], p["gate"], s)
    y = oracle.gated_rms_norm(o_seq, z, norm_w, eps=eps)
    c = cv[:, 0]
    o_f, s_f = oracle.fused_deltanet_decode(
        c[:, :Hk * Dk].reshape(B, Hk, Dk), c[:, Hk * Dk:2 * Hk * Dk].reshape(B, Hk, Dk),
        c[:, 2 * Hk * Dk:].reshape(B, Hv, Dv), ab[:, 0, :Hv], ab[:, 0, Hv:],
        z.reshape(B, Hv, Dv), a_log, dt_bias, norm_w, s, eps=eps)
    np.testing.assert_allclose(s_f, s_seq, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(o_f, y[:, 0], rtol=1e-4, atol=1e-5)


def test_bf16_rounding_of_conv_output_is_exact_ring_copy():
    """The ring holds raw bf16 inputs: a round trip through f32 is the identity."""
    x = normal_bf16((1, 6, 8), 81)
    w = normal_bf16((4, 8), 82)
    _, ring = oracle.conv1d_sequence(x, w)
    assert np.array_equal(f32_to_bf16(bf16_to_f32(ring)), ring)
