"""The rest of the decode step on the GPU vs the oracle: rms_norm! and
fused_add_rms_norm! (src/kernels/rms_norm.jl, residual_norm.jl), the MLP's
silu(gate) .* up (src/llm/qwen35.jl:234-243), the embedding gather (:251),
advance! (src/llm/generate.jl:82-88), lm_head_argmax! (src/kernels/
lm_head_topk.jl:109-147); then a whole step! of an attention-layer stack
(qwen35.jl:245-273) against the oracle composition, and captured generation
(generate.jl:147-196) against eager generation, token for token."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import (D, EPS, HALF, HK, HQ, S, THETA, TOL_MAX, TOL_MEAN, banner, dev_f32,
                      from_dev, i32, maxmean, to_dev)
from oracle.rng import bf16_to_f32, f32_to_bf16, normal_bf16

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N", [(2560, 32), (16384, 3), (24, 5)])
def test_rms_norm(vm, orc, M, N):
    banner(f"rms_norm M={M} N={N}")
    x = normal_bf16((N, M), 100 + M, scale=2.0)
    w = normal_bf16((M,), 101, scale=0.05)
    y = vm.rms_norm(to_dev(x), to_dev(w), eps=EPS, offset=1.0)["Y"]
    mx, mn = maxmean(dev_f32(y), orc.rms_norm(x, w, eps=EPS, offset=1.0))
    print(f"rms_norm {M}x{N}: max {mx:.3e} mean {mn:.3e}")
    assert mx <= TOL_MAX and mn <= TOL_MEAN


@pytest.mark.parametrize("inplace", [False, True])
def test_fused_add_rms_norm(vm, orc, inplace):
    """x' = x + dx stored (in place over x too, the decode step's use), y its norm."""
    banner(f"fused_add_rms_norm inplace={inplace}")
    M, N = 2560, 32
    x = normal_bf16((N, M), 110)
    dx = normal_bf16((N, M), 111, scale=0.5)
    w = normal_bf16((M,), 112, scale=0.05)
    X, dX = to_dev(x), to_dev(dx)
    Y = torch.empty_like(X)
    Xp = X if inplace else torch.empty_like(X)
    vm.fused_add_rms_norm_({"Y": Y, "Xp": Xp}, X, dX, to_dev(w), eps=EPS, offset=1.0)
    ry, rxo = orc.rms_norm(x, w, eps=EPS, offset=1.0, dx=dx)
    mx, mn = maxmean(dev_f32(Y), ry)
    # x' is one bf16 rounding of the exact fp32 sum
    assert np.array_equal(from_dev(Xp), f32_to_bf16(rxo))
    print(f"fused_add_rms_norm: y max {mx:.3e} mean {mn:.3e}")
    assert mx <= TOL_MAX and mn <= TOL_MEAN


def test_silu_mul(vm, orc):
    banner("silu_mul I=9216 N=32")
    I, N = 9216, 32
    gu = normal_bf16((N, 2 * I), 120, scale=2.0)
    mid = torch.empty((N, I), dtype=torch.bfloat16, device="cuda")
    vm.silu_mul_(mid, to_dev(gu))
    ref = orc.silu_mul(gu)
    got = dev_f32(mid)
    # values reach |g u| ~ 60 here: the bar is one bf16 ulp of the fp32 value
    # (2^-7 relative), i.e. one rounding of an fp32 evaluation
    err = np.abs(got.astype(np.float64) - ref) / (np.abs(ref) * 2.0 ** -7 + 1e-30)
    print(f"silu_mul: max error {err.max():.3f} ulp (|mid| max {np.abs(ref).max():.1f})")
    assert err.max() <= 1.0


def test_embed_gather(vm):
    """x[:, b] = E[:, ids[b]], 1-based, bit for bit; out-of-range ids clamp."""
    banner("embed vocab=1000 D=2560 B=6")
    E = normal_bf16((1000, 2560), 130)
    ids = np.array([1, 1000, 17, 500, 0, 1005], np.int32)
    x = torch.empty((6, 2560), dtype=torch.bfloat16, device="cuda")
    vm.embed_(x, to_dev(E), i32(ids))
    got = from_dev(x)
    want = E[np.clip(ids - 1, 0, 999)]
    assert np.array_equal(got, want)


def test_generation_advance(vm):
    """advance!: tokens_out[step, b] = result[b], step += 1, positions .+= 1; a
    step past max_new harvests nothing."""
    banner("generation advance B=3 max_new=2")
    gen = vm.Generation(3, 2)
    gen.positions.copy_(i32([5, 7, 9]))
    gen.result.copy_(i32([11, 12, 13]))
    gen.advance_()
    gen.result.copy_(i32([21, 22, 23]))
    gen.advance_()
    gen.result.copy_(i32([31, 32, 33]))
    gen.advance_()   # step 3 > max_new: no harvest
    torch.cuda.synchronize()
    assert gen.step.item() == 4
    assert gen.positions.cpu().tolist() == [8, 10, 12]
    assert gen.poll(1, 2).tolist() == [[11, 12, 13], [21, 22, 23]]


@pytest.mark.parametrize("N,B", [(20011, 1), (20011, 5), (4099, 32), (4099, 37)])
def test_lm_head_argmax(vm, orc, N, B):
    """GEMV + argmax against the oracle wherever the oracle's top-2 margin is not
    tiny (fp32 sums in another order); one column duplicated below the winner
    checks the smallest-index tie rule; N not a multiple of the tile, B across
    two batch tiles."""
    banner(f"lm_head_argmax K=2560 N={N} B={B}")
    K = 2560
    x = normal_bf16((B, K), 140 + B)
    W = normal_bf16((N, K), 141 + N, scale=0.05)
    res, gap = orc.lm_head_argmax(x, W)
    # a tie for sequence 0: its winner duplicated at a smaller index
    dup = max(0, res[0] - 1 - 7)
    W[dup] = W[res[0] - 1]
    Wd, Xd = to_dev(W), to_dev(x)
    got = vm.lm_head_argmax(Xd, Wd)["Result"].cpu().numpy()
    # fp32 sums in another order differ by ~1e-4 at these logit sizes (|l| < 20)
    ok = gap > 2e-3
    ok[0] = True
    want = res.copy()
    want[0] = dup + 1
    print(f"lm_head N={N} B={B}: margins min {gap.min():.3e}, compared {ok.sum()}/{B}")
    assert ok.sum() >= (B + 1) // 2
    assert np.array_equal(got[ok], want[ok]), (got, want, gap)


def _tiny_cfg(vm, B=4, Ctx=64, tied=True):
    a = vm.AttnConfig(D=512, Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=Ctx,
                      B=B)
    return vm.ModelConfig(attn=a, inter=1024, vocab=4099, n_layers=2, tied=tied)


def _host_layers(m):
    out = []
    for l in m.layers:
        out.append(dict(norm1=from_dev(l.norm1), norm2=from_dev(l.norm2), Wqkv=from_dev(l.Wqkv),
                        Wo=from_dev(l.Wo), qw=from_dev(l.qw), kw=from_dev(l.kw),
                        kc=from_dev(l.K_cache), vc=from_dev(l.V_cache), Wgu=from_dev(l.Wgu),
                        Wd=from_dev(l.Wd)))
    return out


def test_decode_step_vs_oracle(vm, orc):
    """One step! of a 2-layer stack (hidden 512, MLP 1024, vocab 4099, B = 4)
    over random caches, against the oracle's composition with the reference's
    bf16 buffers: the final normed hidden state within the bf16 bar, the greedy
    tokens equal wherever the oracle's top-2 margin is not tiny."""
    banner("decode step 2 layers B=4")
    cfg = _tiny_cfg(vm, tied=False)  # an untied head: the tokens depend on every layer
    m = vm.random_model(cfg, seed=3)
    for i, l in enumerate(m.layers):
        vm.fill_normal_(l.K_cache, 150 + i)
        vm.fill_normal_(l.V_cache, 160 + i)
    gen = vm.Generation(cfg.B, 4)
    pos = np.array([5, 33, 64, 17], np.int32)
    tok = np.array([1, 4099, 77, 2048], np.int32)
    gen.positions.copy_(i32(pos))
    gen.result.copy_(i32(tok))
    layers = _host_layers(m)   # before the step appends its rows
    vm.step_(m, gen)
    torch.cuda.synchronize()
    c, s = orc.rope_tables(HALF, cfg.attn.Ctx, THETA)
    res, gap, xn = orc.model_step(from_dev(m.E), layers, from_dev(m.norm_w), from_dev(m.head), tok,
                                  pos, c, s, Hq=HQ, Hk=HK, eps=EPS)
    mx, mn = maxmean(dev_f32(m.xn), xn)
    got = gen.result.cpu().numpy()
    ok = gap > 0.05
    rel = mn / np.abs(xn).mean()
    print(f"step: xn max {mx:.3e} mean {mn:.3e} ({rel:.2%} of mean |xn|; |xn| max "
          f"{np.abs(xn).max():.2f}); tokens {got.tolist()} oracle {res.tolist()} margins "
          f"{np.round(gap, 3).tolist()}")
    # a chain of bf16 buffers (x, xn, h, gu, mid, qkv, O per layer) each rounded in
    # both evaluations, with sums in different orders: about half an ulp on average
    assert mx <= 0.1 and rel <= 1e-2
    assert ok.sum() >= cfg.B - 1 and np.array_equal(got[ok], res[ok])


def test_identity_model_step(vm):
    """Every projection zero, tied head: the next token is the input token."""
    banner("identity model step")
    cfg = _tiny_cfg(vm)
    m = vm.random_model(cfg, seed=4)
    for l in m.layers:
        for t in (l.Wqkv, l.Wo, l.Wgu, l.Wd, l.norm1, l.norm2):
            t.zero_()
    m.norm_w.zero_()
    gen = vm.Generation(cfg.B, 2)
    gen.positions.copy_(i32([3, 4, 5, 6]))
    tok = [1, 4099, 2, 3000]
    gen.result.copy_(i32(tok))
    vm.step_(m, gen)
    assert gen.result.cpu().tolist() == tok


def test_generate_captured_matches_eager(vm):
    """generate_captured! == generate! token for token (generate.jl:132-196): prefill
    of a 24-token prompt, then 12 tokens, 3 of them eager warm-up steps and the
    rest hipGraph replays of (step!; advance!); the session's graph is reused by
    a second captured run."""
    banner("generate captured vs eager B=4 T=24 n=12")
    cfg = _tiny_cfg(vm, tied=False)  # varied tokens (a tied head mostly repeats its input)
    m = vm.random_model(cfg, seed=5)
    ids = torch.as_tensor(np.random.default_rng(6).integers(1, cfg.vocab + 1, size=(cfg.B, 24)),
                          dtype=torch.int32).cuda()
    gen = vm.Generation(cfg.B, 16)
    eager, t_e = vm.generate_(m, gen, ids, max_new_tokens=12, poll_every=5)
    sess = vm.CaptureSession()
    cap, t_c = vm.generate_captured_(m, gen, ids, max_new_tokens=12, warmup=3, session=sess)
    cap2, _ = vm.generate_captured_(m, gen, ids, max_new_tokens=12, warmup=3, session=sess)
    sess.close()
    print(f"eager {eager.T.tolist()}\ncaptured {cap.T.tolist()}")
    print(f"timing eager {t_e}, captured {t_c}")
    assert eager.shape == (12, cfg.B)
    assert np.array_equal(eager, cap) and np.array_equal(eager, cap2)
    assert gen.positions.cpu().tolist() == [24 + 1 + 12] * cfg.B


def test_captured_session_survives_a_longer_prompt(vm):
    """A session reused for a longer prompt after its graph was captured: the
    eager prefill's projection workspace grows in between (forced here, as a
    longer prompt's GEMM plans may need), and the replays still match eager
    generation token for token -- the captured step holds only the decode
    workspace, which is sized before capture and then fixed."""
    banner("captured session reused with a longer prompt")
    cfg = _tiny_cfg(vm, tied=False)
    m = vm.random_model(cfg, seed=15)
    rng = np.random.default_rng(16)
    short = torch.as_tensor(rng.integers(1, cfg.vocab + 1, size=(cfg.B, 8)), dtype=torch.int32).cuda()
    long_ = torch.as_tensor(rng.integers(1, cfg.vocab + 1, size=(cfg.B, 40)), dtype=torch.int32).cuda()
    gen = vm.Generation(cfg.B, 16)
    sess = vm.CaptureSession()
    vm.generate_captured_(m, gen, short, max_new_tokens=8, warmup=2, session=sess)
    assert sess.exec is not None
    dec = m.attn.dec_space.data_ptr()
    eager_ws = m.attn.linear_workspace().numel()
    m.attn.linear_workspace(eager_ws + (64 << 20))  # the eager workspace is replaced
    cap, _ = vm.generate_captured_(m, gen, long_, max_new_tokens=12, warmup=2, session=sess)
    eager, _ = vm.generate_(m, gen, long_, max_new_tokens=12)
    sess.close()
    print(f"eager {eager.T.tolist()}\ncaptured {cap.T.tolist()}")
    assert m.attn.dec_space.data_ptr() == dec
    assert np.array_equal(eager, cap)
    # the frozen decode workspace refuses to grow rather than free what the graph holds
    with pytest.raises(vm.ArgumentError):
        m.attn.decode_workspace(m.attn.dec_space.numel() + 1)


# ---------------------------------------------------------------- mixed stacks
def _mixed_cfg(vm, B=3, Ctx=64, tied=False, n_layers=4):
    """Qwen3.5's layer pattern (every 4th layer full attention) at a small width:
    hidden 512, DeltaNet Dk = Dv = 128 with Hk = 2, Hv = 4 (1024 conv channels)."""
    a = vm.AttnConfig(D=512, Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=Ctx,
                      B=B)
    return vm.ModelConfig(attn=a, inter=1024, vocab=4099, n_layers=n_layers, tied=tied,
                          linear=vm.DeltaNetConfig(Dk=128, Dv=128, Hk=2, Hv=4, convK=4),
                          interval=4)


def _host_mixed_layers(vm, m):
    out = []
    for l in m.layers:
        common = dict(norm1=from_dev(l.norm1), norm2=from_dev(l.norm2), Wgu=from_dev(l.Wgu),
                      Wd=from_dev(l.Wd))
        if isinstance(l, vm.DeltaNetLayer):
            common.update(kind="linear_attention", Wqz=from_dev(l.Wqz), Wab=from_dev(l.Wab),
                          Wout=from_dev(l.Wout), conv_w=from_dev(l.conv_w), conv_b=None,
                          ring=from_dev(l.conv_state), A_log=l.A_log.cpu().numpy(),
                          dt_bias=l.dt_bias.cpu().numpy(), gnorm_w=from_dev(l.gnorm_w),
                          S=l.S.cpu().numpy())
        else:
            common.update(Wqkv=from_dev(l.Wqkv), Wo=from_dev(l.Wo), qw=from_dev(l.qw),
                          kw=from_dev(l.kw), kc=from_dev(l.K_cache), vc=from_dev(l.V_cache))
        out.append(common)
    return out


def test_decode_step_mixed_vs_oracle(vm, orc):
    """One step! of 3 DeltaNet layers + 1 attention layer (B = 3) from random
    states, rings and caches, against the oracle's composition: the final normed
    hidden state within the bf16 bar, the greedy tokens where margins allow, and
    each DeltaNet state and ring as the oracle leaves them."""
    banner("decode step mixed 3 DeltaNet + 1 attention B=3")
    cfg = _mixed_cfg(vm)
    m = vm.random_model(cfg, seed=7)
    assert cfg.layer_types == ("linear_attention",) * 3 + ("full_attention",)
    for i, l in enumerate(m.layers):
        if isinstance(l, vm.DeltaNetLayer):
            l.S.copy_(torch.randn(l.S.shape, generator=torch.Generator().manual_seed(i)) * 0.05)
            vm.fill_normal_(l.conv_state, 170 + i)
        else:
            vm.fill_normal_(l.K_cache, 150 + i)
            vm.fill_normal_(l.V_cache, 160 + i)
    gen = vm.Generation(cfg.B, 4)
    pos = np.array([5, 33, 64], np.int32)
    tok = np.array([1, 4099, 77], np.int32)
    gen.positions.copy_(i32(pos))
    gen.result.copy_(i32(tok))
    layers = _host_mixed_layers(vm, m)
    vm.step_(m, gen)
    torch.cuda.synchronize()
    c, s = orc.rope_tables(HALF, cfg.attn.Ctx, THETA)
    lc = cfg.linear
    res, gap, xn = orc.model_step(from_dev(m.E), layers, from_dev(m.norm_w), from_dev(m.head), tok,
                                  pos, c, s, Hq=HQ, Hk=HK, eps=EPS,
                                  linear_cfg=dict(Dk=lc.Dk, Dv=lc.Dv, Hk=lc.Hk, Hv=lc.Hv))
    mx, mn = maxmean(dev_f32(m.xn), xn)
    got = gen.result.cpu().numpy()
    ok = gap > 0.05
    rel = mn / np.abs(xn).mean()
    print(f"mixed step: xn max {mx:.3e} mean {mn:.3e} ({rel:.2%}); tokens {got.tolist()} "
          f"oracle {res.tolist()} margins {np.round(gap, 3).tolist()}")
    assert mx <= 0.1 and rel <= 1e-2
    assert ok.sum() >= cfg.B - 1 and np.array_equal(got[ok], res[ok])
    # the first DeltaNet layer's state and ring after the step, from the same xn
    l0, h0 = m.layers[0], layers[0]
    xn0 = orc.f32_to_bf16(orc.rms_norm(from_dev(m.E)[tok - 1], h0["norm1"], eps=EPS, offset=1.0))
    _, ring1, S1 = orc.deltanet_decode_layer(xn0, h0, eps=EPS, Dk=lc.Dk, Dv=lc.Dv, Hk=lc.Hk,
                                             Hv=lc.Hv)
    ring_got = from_dev(l0.conv_state)
    assert np.array_equal(ring_got[:, :-1], h0["ring"][:, 1:])   # shifted exactly
    new_col, want = bf16_to_f32(ring_got[:, -1]), bf16_to_f32(ring1[:, -1])
    assert np.all(np.abs(new_col - want) <= 2.0 ** -7 * np.abs(want) + 1e-6)  # the projection
    np.testing.assert_allclose(l0.S.cpu().numpy(), S1, rtol=1e-3, atol=1e-4)


def test_generate_captured_matches_eager_mixed(vm):
    """generate_captured! == generate! token for token on the mixed stack, the
    recurrent state reset before each run (reset!, qwen35.jl:175-185); without
    the reset the second run continues the first's state and differs."""
    banner("generate captured vs eager, mixed stack B=3")
    cfg = _mixed_cfg(vm)
    m = vm.random_model(cfg, seed=8)
    ids = torch.as_tensor(np.random.default_rng(9).integers(1, cfg.vocab + 1, size=(cfg.B, 20)),
                          dtype=torch.int32).cuda()
    gen = vm.Generation(cfg.B, 16)
    m.reset_()
    eager, _ = vm.generate_(m, gen, ids, max_new_tokens=10, poll_every=4)
    m.reset_()
    sess = vm.CaptureSession()
    cap, _ = vm.generate_captured_(m, gen, ids, max_new_tokens=10, warmup=3, session=sess)
    carried, _ = vm.generate_captured_(m, gen, ids, max_new_tokens=10, warmup=3, session=sess)
    sess.close()
    print(f"eager {eager.T.tolist()}\ncaptured {cap.T.tolist()}\ncarried {carried.T.tolist()}")
    assert np.array_equal(eager, cap)
    assert not np.array_equal(eager, carried)


def test_prefix_prefill_with_restore_matches_full(vm):
    """prefill!(prefix); snapshot; ...; restore!; prefill!(suffix; offset) leaves
    the DeltaNet states, rings, attention cache rows and next tokens of one
    whole prefill (the reference's prefix caching, qwen35.jl:397-427, and the
    suffix conv path, :333-344, whose left context is the restored ring). The
    two runs differ only by rounding: the projections' GEMMs see different row
    counts, and the chunked recurrence splits at another token."""
    banner("prefix prefill + restore vs full prefill, mixed stack B=3")
    cfg = _mixed_cfg(vm)
    m = vm.random_model(cfg, seed=10)
    ids = torch.as_tensor(np.random.default_rng(11).integers(1, cfg.vocab + 1, size=(cfg.B, 21)),
                          dtype=torch.int32).cuda()
    gen = vm.Generation(cfg.B, 2)
    attn = [l for l in m.layers if not isinstance(l, vm.DeltaNetLayer)]
    m.reset_()
    vm.prefill_(m, gen, ids)
    full = [(l.S.clone(), l.conv_state.clone()) for l in m.dn_layers]
    full_kv = [(l.K_cache[:, :, :21].clone(), l.V_cache[:, :, :21].clone()) for l in attn]
    res_full = gen.result.clone()
    xn_full = m.xn.float().clone()
    for l in attn:   # the split run must write every row itself
        l.K_cache.zero_()
        l.V_cache.zero_()
    m.reset_()
    vm.prefill_(m, gen, ids[:, :13].contiguous())
    snap = m.snapshot()
    m.reset_()                      # state lost (another request ran) ...
    m.restore_(snap)                # ... and restored from the snapshot
    vm.prefill_(m, gen, ids[:, 13:].contiguous(), offset=13)
    torch.cuda.synchronize()
    for i, ((S_f, r_f), l) in enumerate(zip(full, m.dn_layers)):
        s_err = float((l.S - S_f).abs().max() / S_f.abs().max())
        r_err = float(np.abs(dev_f32(l.conv_state) - dev_f32(r_f)).max() / np.abs(dev_f32(r_f)).max())
        print(f"DeltaNet layer {i}: S max err / max {s_err:.2e}, ring {r_err:.2e}")
        assert s_err <= 2e-2 and r_err <= 2e-2
    for i, ((K_f, V_f), l) in enumerate(zip(full_kv, attn)):
        k_err = float((l.K_cache[:, :, :21].float() - K_f.float()).abs().max())
        v_err = float((l.V_cache[:, :, :21].float() - V_f.float()).abs().max())
        print(f"attention layer {i}: cache rows 1..21 max err K {k_err:.2e}, V {v_err:.2e}")
        assert k_err <= 5e-2 and v_err <= 5e-2
    x_err = float((m.xn.float() - xn_full).abs().max() / xn_full.abs().max())
    logits = xn_full @ m.head.float().t()
    top2 = torch.topk(logits, 2, dim=1).values
    margin = (top2[:, 0] - top2[:, 1]).cpu().numpy()
    got, want = gen.result.cpu().numpy(), res_full.cpu().numpy()
    print(f"final hidden max err / max {x_err:.2e}; tokens full {want.tolist()} split "
          f"{got.tolist()} margins {np.round(margin, 3).tolist()}")
    assert x_err <= 2e-2
    ok = margin > 0.05
    assert ok.sum() >= cfg.B - 1 and np.array_equal(got[ok], want[ok])
    assert gen.positions.cpu().tolist() == [22] * cfg.B


def _lin_cfg(cfg):
    lc = cfg.linear
    return dict(Dk=lc.Dk, Dv=lc.Dv, Hk=lc.Hk, Hv=lc.Hv)


def _check_prefill(vm, m, gen, res, gap, xn, states, what):
    """GPU prefill_ results against orc.prefill_model's: the last token's final
    xn, the tokens where the oracle's margin allows, each DeltaNet state and
    ring, each attention layer's cache rows."""
    mx, mn = maxmean(dev_f32(m.xn), xn)
    rel = mn / np.abs(xn).mean()
    got = gen.result.cpu().numpy()
    ok = gap > 0.05
    print(f"{what}: xn max {mx:.3e} mean {mn:.3e} ({rel:.2%}); tokens {got.tolist()} oracle "
          f"{res.tolist()} margins {np.round(gap, 3).tolist()}")
    assert mx <= 0.1 and rel <= 1e-2
    assert ok.sum() >= len(got) - 1 and np.array_equal(got[ok], res[ok])
    for i, (l, st) in enumerate(zip(m.layers, states)):
        if isinstance(l, vm.DeltaNetLayer):
            ring_o, S_o = st
            s_err = float(np.abs(l.S.cpu().numpy() - S_o).max() / np.abs(S_o).max())
            r_err = float(np.abs(dev_f32(l.conv_state) - bf16_to_f32(ring_o)).max() /
                          np.abs(bf16_to_f32(ring_o)).max())
            print(f"  layer {i} DeltaNet: S max err / max {s_err:.2e}, ring {r_err:.2e}")
            assert s_err <= 1e-2 and r_err <= 1e-2
        else:
            kc_o, vc_o = st
            k_err = float(np.abs(dev_f32(l.K_cache) - bf16_to_f32(kc_o)).max())
            v_err = float(np.abs(dev_f32(l.V_cache) - bf16_to_f32(vc_o)).max())
            print(f"  layer {i} attention: cache max err K {k_err:.2e} V {v_err:.2e}")
            assert k_err <= 5e-2 and v_err <= 5e-2


def test_prefill_mixed_vs_oracle(vm, orc):
    """prefill! (qwen35.jl:369-395) of the mixed stack (3 DeltaNet + 1 attention,
    B = 3) from a reset state over 21 tokens, against orc.prefill_model; then a
    13-token prefix and an 8-token suffix (offset 13, the suffix conv's left
    context from the ring) against the oracle run the same way."""
    banner("prefill mixed 3 DeltaNet + 1 attention B=3 T=21, and 13 + 8")
    cfg = _mixed_cfg(vm)
    m = vm.random_model(cfg, seed=21)
    ids = np.random.default_rng(22).integers(1, cfg.vocab + 1, size=(cfg.B, 21)).astype(np.int32)
    c, s = orc.rope_tables(HALF, cfg.attn.Ctx, THETA)
    kw = dict(Hq=HQ, Hk=HK, eps=EPS, linear_cfg=_lin_cfg(cfg))
    E, nw, head = from_dev(m.E), from_dev(m.norm_w), from_dev(m.head)
    gen = vm.Generation(cfg.B, 2)
    m.reset_()
    for l in m.layers:
        if not isinstance(l, vm.DeltaNetLayer):
            l.K_cache.zero_()
            l.V_cache.zero_()
    layers0 = _host_mixed_layers(vm, m)     # reset DeltaNet states, zero caches
    vm.prefill_(m, gen, torch.from_numpy(ids).cuda())
    torch.cuda.synchronize()
    res, gap, xn, states = orc.prefill_model(E, layers0, nw, head, ids, 0, c, s, **kw)
    _check_prefill(vm, m, gen, res, gap, xn, states, "prefill T=21")
    # prefix + suffix, on both sides
    m.reset_()
    vm.prefill_(m, gen, torch.from_numpy(ids[:, :13]).cuda())
    vm.prefill_(m, gen, torch.from_numpy(ids[:, 13:]).cuda(), offset=13)
    torch.cuda.synchronize()
    _, _, _, st13 = orc.prefill_model(E, layers0, nw, head, ids[:, :13], 0, c, s, **kw)
    cont = [dict(l) for l in layers0]
    for l, st in zip(cont, st13):
        if l.get("kind") == "linear_attention":
            l["ring"], l["S"] = st
        else:
            l["kc"], l["vc"] = st
    res2, gap2, xn2, states2 = orc.prefill_model(E, cont, nw, head, ids[:, 13:], 13, c, s, **kw)
    _check_prefill(vm, m, gen, res2, gap2, xn2, states2, "prefill 13 + 8")
    assert gen.positions.cpu().tolist() == [22] * cfg.B


def test_decode_step_qwen35_4b_shape_vs_oracle(vm, orc):
    """One step! of the Qwen3.5-4B-shaped model the bench reports (32 layers,
    24 Gated DeltaNet + 8 gated attention, hidden 2560, MLP 9216, vocab 151936,
    tied head, random weights; B = 32 at ragged positions, random DeltaNet states
    and rings), against orc.model_step on four of the sequences: the tokens where
    the margin allows, and the final normed hidden state within twice the
    distance one extra bf16 rounding of the input moves the oracle's own."""
    banner("decode step Qwen3.5-4B shape B=32, 4 sequences vs oracle")
    B, Ctx = 32, 2048
    a = vm.AttnConfig(D=2560, Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=Ctx,
                      B=B)
    cfg = vm.ModelConfig(attn=a, inter=9216, vocab=151936, n_layers=32, tied=True, interval=4)
    m = vm.random_model(cfg, seed=23)
    g = torch.Generator(device="cuda").manual_seed(24)
    for i, l in enumerate(m.layers):
        if isinstance(l, vm.DeltaNetLayer):
            l.S.copy_(torch.randn(l.S.shape, generator=g, device="cuda") * 0.05)
            vm.fill_normal_(l.conv_state, 240 + i)
        else:
            vm.fill_normal_(l.K_cache, 250 + i)
            vm.fill_normal_(l.V_cache, 260 + i)
    rng = np.random.default_rng(25)
    pos = rng.integers(256, Ctx + 1, size=B).astype(np.int32)
    tok = rng.integers(1, cfg.vocab + 1, size=B).astype(np.int32)
    sample = np.array([0, 9, 20, 31])
    pos[sample[0]] = Ctx
    gen = vm.Generation(B, 2)
    gen.positions.copy_(i32(pos))
    gen.result.copy_(i32(tok))
    # the sampled sequences' states before the step, and the weights
    layers = []
    for l in m.layers:
        d = dict(norm1=from_dev(l.norm1), norm2=from_dev(l.norm2), Wgu=from_dev(l.Wgu),
                 Wd=from_dev(l.Wd))
        if isinstance(l, vm.DeltaNetLayer):
            d.update(kind="linear_attention", Wqz=from_dev(l.Wqz), Wab=from_dev(l.Wab),
                     Wout=from_dev(l.Wout), conv_w=from_dev(l.conv_w), conv_b=None,
                     ring=from_dev(l.conv_state[sample]), A_log=l.A_log.cpu().numpy(),
                     dt_bias=l.dt_bias.cpu().numpy(), gnorm_w=from_dev(l.gnorm_w),
                     S=l.S[sample].cpu().numpy())
        else:
            d.update(Wqkv=from_dev(l.Wqkv), Wo=from_dev(l.Wo), qw=from_dev(l.qw), kw=from_dev(l.kw),
                     kc=from_dev(l.K_cache[sample]), vc=from_dev(l.V_cache[sample]))
        layers.append(d)
    vm.step_(m, gen)
    torch.cuda.synchronize()
    c, s = orc.rope_tables(HALF, Ctx, THETA)
    res, gap, xn = orc.model_step(from_dev(m.E), layers, from_dev(m.norm_w), from_dev(m.head),
                                  tok[sample], pos[sample], c, s, Hq=HQ, Hk=HK, eps=EPS,
                                  linear_cfg=_lin_cfg(cfg))
    mx, mn = maxmean(dev_f32(m.xn)[sample], xn)
    got = gen.result.cpu().numpy()[sample]
    ok = gap > 0.05
    # the model's own sensitivity: the oracle again with every input embedding
    # element moved by one bf16 ulp (a random sign), i.e. one different rounding
    # of the step's first buffer
    E = from_dev(m.E)
    rows = tok[sample] - 1
    flip = np.random.default_rng(26).choice(np.array([-1, 1], np.int32), size=(len(sample), E.shape[1]))
    Ep = E.copy()
    Ep[rows] = (E[rows].astype(np.int32) + flip).astype(np.uint16)
    _, _, xn_p = orc.model_step(Ep, layers, from_dev(m.norm_w), from_dev(m.head), tok[sample],
                                pos[sample], c, s, Hq=HQ, Hk=HK, eps=EPS, linear_cfg=_lin_cfg(cfg))
    pmx, pmn = maxmean(xn_p, xn)
    print(f"4B-shape step, sequences {sample.tolist()}: xn vs oracle max {mx:.3e} mean {mn:.3e} "
          f"({mn / np.abs(xn).mean():.2%}); oracle vs its 1-ulp-input twin max {pmx:.3e} mean "
          f"{pmn:.3e}; tokens {got.tolist()} oracle {res.tolist()} margins {np.round(gap, 3).tolist()}")
    # a 32-layer random-weight stack amplifies a one-ulp change of its input to a
    # few % of |xn|: the GPU step may differ from the oracle by no more than twice
    # what that single extra rounding does (measured: 0.8x mean, 1.1x max)
    assert mn <= 2.0 * pmn and mx <= 2.0 * pmx
    assert ok.sum() >= len(sample) - 1 and np.array_equal(got[ok], res[ok])


def test_identity_mixed_model_step(vm):
    """Every projection zero on the mixed stack: the next token is the input."""
    banner("identity mixed model step")
    cfg = _mixed_cfg(vm, tied=True)
    m = vm.random_model(cfg, seed=12)
    for l in m.layers:
        ts = (l.W_in, l.Wout) if isinstance(l, vm.DeltaNetLayer) else (l.Wqkv, l.Wo)
        for t in ts + (l.Wgu, l.Wd, l.norm1, l.norm2):
            t.zero_()
    m.norm_w.zero_()
    gen = vm.Generation(cfg.B, 2)
    gen.positions.copy_(i32([3, 4, 5]))
    tok = [1, 4099, 2]
    gen.result.copy_(i32(tok))
    vm.step_(m, gen)
    assert gen.result.cpu().tolist() == tok


@pytest.mark.parametrize("D_,N,K", [(2560, 32, 4096), (2560, 3, 9216), (2560, 16, 64),
                                   (2560, 64, 4096), (1024, 25, 1024)])
def test_linear_add_rms_norm_is_the_two_calls(vm, D_, N, K):
    """linear! + fused_add_rms_norm! in one call (the split GEMV's slices summed
    by the norm; one slice; the GEMM library's path at N = 64) is bit-identical
    to the two calls, residual updated in place."""
    banner(f"linear_add_rms_norm D={D_} N={N} K={K}")
    a = to_dev(normal_bf16((N, K), 990 + K))
    W = to_dev(normal_bf16((D_, K), 991 + D_, scale=K ** -0.5))
    x0 = to_dev(normal_bf16((N, D_), 992))
    nw = to_dev(normal_bf16((D_,), 993, scale=0.05))
    h = vm.linear(a, W)["y"]
    x_ref = x0.clone()
    y_ref = torch.empty_like(x0)
    vm.fused_add_rms_norm_({"Y": y_ref, "Xp": x_ref}, x_ref, h, nw, eps=EPS, offset=1.0)
    x = x0.clone()
    y = torch.empty_like(x0)
    print(f"workspace {vm.linear_add_rms_norm_workspace_bytes(a, W)} B")
    vm.linear_add_rms_norm_({"Y": y, "X": x}, a, W, nw, eps=EPS, offset=1.0)
    torch.cuda.synchronize()
    assert torch.equal(x.view(torch.int16), x_ref.view(torch.int16))
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))


def test_linear_add_rms_norm_misaligned_input(vm):
    """An input view off the GEMV's alignment takes the GEMM library's path."""
    banner("linear_add_rms_norm misaligned input")
    D_, N, K = 2560, 4, 512
    a_full = to_dev(normal_bf16((N, K + 8), 994))
    a = a_full[:, 4:K + 4]
    W = to_dev(normal_bf16((D_, K), 995, scale=K ** -0.5))
    x0 = to_dev(normal_bf16((N, D_), 996))
    nw = to_dev(normal_bf16((D_,), 997, scale=0.05))
    h = vm.linear(a, W)["y"]
    x_ref, y_ref = x0.clone(), torch.empty_like(x0)
    vm.fused_add_rms_norm_({"Y": y_ref, "Xp": x_ref}, x_ref, h, nw, eps=EPS, offset=1.0)
    x, y = x0.clone(), torch.empty_like(x0)
    vm.linear_add_rms_norm_({"Y": y, "X": x}, a, W, nw, eps=EPS, offset=1.0)
    torch.cuda.synchronize()
    assert torch.equal(x.view(torch.int16), x_ref.view(torch.int16))
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))
