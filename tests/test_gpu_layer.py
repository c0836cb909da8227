"""The projections around the block and whole attention layers on the GPU vs the
oracle: linear! (hipBLASLt, src/linear.jl:40-57) alone for the decode GEMV and
prefill GEMM shapes, decode!(h, ::AttnLayer, m, gen, xn) (qwen35.jl:187-208) at
BASELINE config 1 and forward(::AttnLayer, m, xn, T, B) (qwen35.jl:292-318) at
config 2, hidden state to hidden state, and the whole decode layer step captured
in a hipGraph and replayed with the position advancing (replays == eager)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import (D, EPS, HALF, HK, HQ, S, THETA, TOL_MAX, TOL_MEAN, banner, dev_f32,
                      from_dev, i32, maxmean, to_dev)
from oracle.rng import bf16_to_f32, f32_to_bf16, normal_bf16

pytestmark = pytest.mark.gpu

DM = 2560  # hidden size of the layer (the Qwen3.5 small-model width)


@pytest.mark.parametrize("M,N,K", [(S * D, 1, DM), (S * D, 32, DM), (DM, 4096, HQ * D),
                                   (520, 300, 136)])
def test_linear_operator(vm, orc, M, N, K):
    """y = W^T x for the qkv GEMV (N = 1, 32), the Wo GEMM of a 4096-token
    prefill and an odd shape; checked on every 8th column of y (N > 64)."""
    banner(f"linear M={M} N={N} K={K}")
    x = normal_bf16((N, K), 700 + N)
    W = normal_bf16((M, K), 800 + M, scale=K ** -0.5)
    y = vm.linear(to_dev(x), to_dev(W))["y"]
    torch.cuda.synchronize()
    rows = slice(None, None, 8) if N > 64 else slice(None)
    ref = orc.linear(x[rows], W)
    mx, mn = maxmean(dev_f32(y)[rows], ref)
    print(f"linear {M}x{N}x{K}: max {mx:.3e} mean {mn:.3e}")
    assert mx <= TOL_MAX and mn <= TOL_MEAN


NARROW = [(S * D, 1, DM), (S * D, 16, DM), (DM, 16, HQ * D), (DM, 1, HQ * D),
          (2 * 9216, 16, DM), (DM, 16, 9216), (100, 7, 64), (4, 1, 64), (36, 16, 640),
          (2 * 9216, 3, DM), (DM, 32, HQ * D), (DM, 32, 9216), (4096, 25, 1024)]


def _narrow_bar(x, W, ref):
    """Per-element bar of a narrow product with fp32 accumulation: the bf16
    rounding of the output (half an ulp, 2^-9 |y|, taken as one ulp) plus fp32
    reassociation, bounded by 2^-20 sum_k |x_k w_k|."""
    xa = np.abs(bf16_to_f32(x).astype(np.float64))
    wa = np.abs(bf16_to_f32(W).astype(np.float64))
    return 2.0 ** -8 * np.abs(ref) + 2.0 ** -20 * (xa.reshape(-1, xa.shape[-1]) @ wa.T).reshape(
        ref.shape)


def _offset_view(t, off, ld):
    """t (rows, cols) copied into a buffer as rows of `ld` elements starting `off`
    elements in: a view with column stride ld and a data pointer off * 2 bytes
    past an aligned one."""
    rows, cols = t.shape
    buf = torch.full((off + rows * ld,), 3.0, dtype=torch.bfloat16, device="cuda")
    v = buf[off:].view(rows, ld)[:, :cols]
    v.copy_(t)
    return v, buf


# (M, N, K, x offset / stride, W offset / stride, y offset / stride)
GENERAL = [(37, 5, 29, (0, 31), (0, 29), (0, 37)),         # odd strides everywhere
           (520, 300, 136, (0, 136), (1, 136), (0, 520)),  # W 2 bytes off alignment
           (197, 70, 1000, (1, 1000), (0, 1000), (3, 197)),
           (10, 3, 1, (0, 1), (0, 1), (0, 10)),             # K = 1
           (2560, 257, 2048, (0, 2048), (0, 2048), (1, 2560)),
           (64, 64, 64, (0, 72), (0, 65), (0, 64))]


@pytest.mark.parametrize("M,N,K,xs,ws,ys", GENERAL)
def test_linear_general_kernel(vm, orc, M, N, K, xs, ws, ys):
    """Views the GEMM library is not given (column strides that are not
    multiples of 8, data pointers off 16-byte alignment) run on the library's
    general bf16 MFMA kernel, the role of the reference's mul! fallback
    (linear.jl:59-61, :67): every element within one bf16 ulp (plus fp32
    reassociation) of the fp32 oracle, elements outside the view untouched,
    and no workspace needed."""
    banner(f"linear general M={M} N={N} K={K} x{xs} W{ws} y{ys}")
    x = normal_bf16((N, K), 730 + N + K)
    W = normal_bf16((M, K), 830 + M, scale=K ** -0.5)
    xv, _ = _offset_view(to_dev(x), *xs)
    Wv, _ = _offset_view(to_dev(W), *ws)
    yv, flat = _offset_view(torch.full((N, M), 3.0, dtype=torch.bfloat16, device="cuda"), *ys)
    if ys[1] % 8 or xs[1] % 8 or ws[1] % 8:
        assert vm.linear_workspace_bytes(xv, Wv, yv) == 0
    vm.linear_({"y": yv}, xv, Wv, workspace=torch.empty(16, dtype=torch.uint8, device="cuda"))
    torch.cuda.synchronize()
    rows = slice(None, None, 8) if N > 64 else slice(None)
    ref = orc.linear(x[rows], W).astype(np.float64)
    bar = _narrow_bar(x[rows], W, ref)
    got = dev_f32(yv)[rows].astype(np.float64)
    worst = float(np.max(np.abs(got - ref) / bar))
    print(f"linear general {M}x{N}x{K}: worst |err|/bar {worst:.3f}")
    assert worst <= 1.0
    # the padding around the view keeps its fill (3.0), and so do the elements before it
    off, ld = ys
    pad = flat[off:off + N * ld].view(N, ld)[:, M:]
    assert bool((pad == 3.0).all())
    if off:
        assert bool((flat[:off] == 3.0).all())


@pytest.mark.parametrize("M,N,K", NARROW)
def test_linear_narrow(vm, orc, M, N, K):
    """The decode projections (N <= 16, or N <= 32 with M <= 4096) run on the library's split-K
    MFMA kernel: every element within one bf16 ulp (plus fp32 reassociation)
    of the fp32 oracle, the result bitwise the same on a second call (the
    slices add in a fixed order), and strided x / y columns honoured."""
    banner(f"linear narrow M={M} N={N} K={K}")
    x = normal_bf16((N, K), 710 + N + K)
    W = normal_bf16((M, K), 810 + M, scale=K ** -0.5)
    xd, Wd = to_dev(x), to_dev(W)
    print(f"workspace {vm.linear_workspace_bytes(xd, Wd)} B")
    y1 = vm.linear(xd, Wd)["y"]
    y2 = vm.linear(xd, Wd)["y"]
    # x and y as columns of wider buffers (column strides K + 64, M + 8)
    xw = torch.zeros((N, K + 64), dtype=torch.bfloat16, device="cuda")
    xw[:, :K] = xd
    yw = torch.full((N, M + 8), 7.0, dtype=torch.bfloat16, device="cuda")
    vm.linear_({"y": yw[:, :M]}, xw[:, :K], Wd)
    torch.cuda.synchronize()
    ref = orc.linear(x, W).astype(np.float64)
    bar = _narrow_bar(x, W, ref)
    got = dev_f32(y1).astype(np.float64)
    worst = float(np.max(np.abs(got - ref) / bar))
    print(f"linear narrow {M}x{N}x{K}: worst |err|/bar {worst:.3f}")
    assert worst <= 1.0
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    assert torch.equal(yw[:, :M].view(torch.int16), y1.view(torch.int16))
    assert bool((yw[:, M:] == 7.0).all())


def test_linear_narrow_split_workspace(vm):
    """A split GEMV keeps its K slices' fp32 partials in the workspace: a
    workspace full of garbage, one shared by problems in turn, and a captured
    graph replayed with other problems run eagerly between the replays all give
    the fresh-workspace results, bit for bit."""
    banner("linear narrow split workspace")
    probs = [(DM, 32, 9216), (DM, 16, HQ * D), (DM, 3, HQ * D), (4096, 25, 1024)]
    xs, Ws, refs = [], [], []
    for i, (M, N, K) in enumerate(probs):
        x = to_dev(normal_bf16((N, K), 740 + i))
        W = to_dev(normal_bf16((M, K), 840 + i, scale=K ** -0.5))
        need = vm.linear_workspace_bytes(x, W)
        print(f"M={M} N={N} K={K}: workspace {need} B")
        assert need > 0, "expected a split problem"
        y = vm.linear(x, W, workspace=torch.zeros(need, dtype=torch.uint8, device="cuda"))["y"]
        xs.append(x)
        Ws.append(W)
        refs.append(y)
    nmax = max(vm.linear_workspace_bytes(x, W) for x, W in zip(xs, Ws))
    ws = torch.randint(0, 256, (nmax,), dtype=torch.uint8, device="cuda")  # garbage
    ys = [torch.empty_like(r) for r in refs]
    for _ in range(2):
        for x, W, y, r in zip(xs, Ws, ys, refs):
            vm.linear_({"y": y}, x, W, workspace=ws)
            torch.cuda.synchronize()
            assert torch.equal(y.view(torch.int16), r.view(torch.int16))
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            vm.linear_({"y": ys[0]}, xs[0], Ws[0], workspace=ws)
    torch.cuda.synchronize()
    for k in range(4):
        ys[0].zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(ys[0].view(torch.int16), refs[0].view(torch.int16)), f"replay {k}"
        vm.linear_({"y": ys[1 + k % 3]}, xs[1 + k % 3], Ws[1 + k % 3], workspace=ws)  # between
        torch.cuda.synchronize()
        assert torch.equal(ys[1 + k % 3].view(torch.int16), refs[1 + k % 3].view(torch.int16))
    del g


def test_linear_narrow_misaligned_view(vm, orc):
    """A view off the kernel's 16-byte alignment takes the GEMM library's
    path for the same problem: same results to the parity bar."""
    banner("linear narrow misaligned view")
    M, N, K = 256, 4, 512
    x = normal_bf16((N, K + 8), 733)
    W = normal_bf16((M, K), 834, scale=K ** -0.5)
    xd = to_dev(x)[:, 4:K + 4]  # 8-byte offset, column stride K + 8
    y = vm.linear(xd, to_dev(W))["y"]
    torch.cuda.synchronize()
    ref = orc.linear(np.ascontiguousarray(x[:, 4:K + 4]), W).astype(np.float64)
    mx, mn = maxmean(dev_f32(y), ref)
    print(f"linear misaligned: max {mx:.3e} mean {mn:.3e}")
    assert mx <= TOL_MAX and mn <= TOL_MEAN


def _silu_mul_bar(orc, x, W, I):
    """The oracle's mid (orc.linear's fp32 gate-up rounded to bf16, as the
    reference stores gu, then orc.silu_mul, rounded) and a per-element bar:
    mid's own bf16 rounding (2^-7 |mid|, one ulp taken generously) plus what
    one ulp and the fp32 reassociation of gate and up (2^-7 |g| + 2^-20
    sum_k |x_k w_k|) move it by through d mid / d g = u silu'(g) and
    d mid / d u = silu(g)."""
    gu = f32_to_bf16(orc.linear(x, W))
    ref = bf16_to_f32(f32_to_bf16(orc.silu_mul(gu))).astype(np.float64)
    g = bf16_to_f32(gu[:, :I]).astype(np.float64)
    u = bf16_to_f32(gu[:, I:]).astype(np.float64)
    sg = 1.0 / (1.0 + np.exp(-g))
    silu = g * sg
    xa = np.abs(bf16_to_f32(x).astype(np.float64))
    wa = np.abs(bf16_to_f32(W).astype(np.float64))
    ra = xa @ wa.T
    dg = 2.0 ** -7 * np.abs(g) + 2.0 ** -20 * ra[:, :I]
    du = 2.0 ** -7 * np.abs(u) + 2.0 ** -20 * ra[:, I:]
    dsilu = sg * (1.0 + g * (1.0 - sg))
    bar = 2.0 ** -7 * np.abs(ref) + np.abs(u * dsilu) * dg + np.abs(silu) * du + 1e-30
    return ref, bar


@pytest.mark.parametrize("I,N,K", [(9216, 32, 2560), (9216, 1, 2560), (1000, 20, 640),
                                   (1024, 7, 512), (512, 40, 256)])
def test_linear_silu_mul(vm, orc, I, N, K):
    """linear! + silu .* mul in one call (the MLP's first half, qwen35.jl:234-243):
    at N <= 32 the stream-K GEMV's fp32 partials summed by the silu kernel (I =
    9216: the decode step's shape; 1000: row groups past the end of W), at N =
    40 linear! + silu .* mul. Every element within the bar of the propagated
    bf16 roundings of gate and up; a second call bitwise equal; a strided mid
    honoured."""
    banner(f"linear_silu_mul I={I} N={N} K={K}")
    x = normal_bf16((N, K), 900 + N + K)
    W = normal_bf16((2 * I, K), 910 + I, scale=K ** -0.5)
    xd, Wd = to_dev(x), to_dev(W)
    ws = torch.empty(vm.linear_silu_mul_workspace_bytes(xd, Wd), dtype=torch.uint8, device="cuda")
    m1 = torch.empty((N, I), dtype=torch.bfloat16, device="cuda")
    m2 = torch.empty_like(m1)
    vm.linear_silu_mul_(m1, xd, Wd, workspace=ws)
    vm.linear_silu_mul_(m2, xd, Wd, workspace=ws)
    mw = torch.full((N, I + 16), 3.0, dtype=torch.bfloat16, device="cuda")
    vm.linear_silu_mul_(mw[:, :I], xd, Wd, workspace=ws)
    torch.cuda.synchronize()
    ref, bar = _silu_mul_bar(orc, x, W, I)
    got = dev_f32(m1).astype(np.float64)
    worst = float(np.max(np.abs(got - ref) / bar))
    print(f"linear_silu_mul {I}x{N}x{K}: worst |err|/bar {worst:.3f}, "
          f"mean |err| {np.abs(got - ref).mean():.2e} (|mid| mean {np.abs(ref).mean():.2e})")
    assert worst <= 1.0
    assert torch.equal(m1.view(torch.int16), m2.view(torch.int16))
    assert torch.equal(mw[:, :I].view(torch.int16), m1.view(torch.int16))
    assert bool((mw[:, I:] == 3.0).all())


def test_linear_silu_mul_misaligned_input(vm, orc):
    """x one element off 16-byte alignment: the call takes linear! + silu .* mul
    (within the same bar)."""
    banner("linear_silu_mul misaligned x")
    I, N, K = 1024, 8, 512
    x = normal_bf16((N, K), 930)
    W = normal_bf16((2 * I, K), 931, scale=K ** -0.5)
    xb = torch.zeros((N * (K + 8) + 1,), dtype=torch.bfloat16, device="cuda")
    xv = xb[1:1 + N * (K + 8)].view(N, K + 8)[:, :K]
    xv.copy_(to_dev(x))
    Wd = to_dev(W)
    mid = torch.empty((N, I), dtype=torch.bfloat16, device="cuda")
    vm.linear_silu_mul_(mid, xv, Wd)
    torch.cuda.synchronize()
    ref, bar = _silu_mul_bar(orc, x, W, I)
    worst = float(np.max(np.abs(dev_f32(mid).astype(np.float64) - ref) / bar))
    print(f"misaligned: worst |err|/bar {worst:.3f}")
    assert worst <= 1.0


def test_linear_first_call_captured_then_tuned(vm, orc):
    """vm_linear keeps the header's contract on the first call of a new problem:
    it builds the plan with the heuristic's first algorithm (host work only), so
    that call can sit inside a capture (which any device allocation on the
    capturing thread would fail). vm_linear_tune is the separate load-time call
    that times the candidates; once tuned, the pick stays the same for later
    calls, eager or captured. Problems of this test's shapes occur nowhere else,
    so their plans are new here."""
    banner("linear: first call under capture, then tuned")
    lib = vm._lib
    for M, N, K in ((1000, 48, 768), (1016, 40, 832)):
        x = normal_bf16((N, K), 740 + N, scale=1.0)
        W = normal_bf16((M, K), 741 + N, scale=K ** -0.5)
        xd, Wd = to_dev(x), to_dev(W)
        y = torch.empty((N, M), dtype=torch.bfloat16, device="cuda")
        ws = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")  # the plan's cap
        prob = (M, N, K, K, K, M)
        ref = orc.linear(x, W).astype(np.float64)

        def run():
            lib.call("vm_linear", vm.ops._p(y), M, vm.ops._p(xd), K, vm.ops._p(Wd), K, M, N, K,
                     vm.ops._p(ws), ws.numel(), vm.ops._stream())

        def check(what):
            torch.cuda.synchronize()
            mx, mn = maxmean(dev_f32(y), ref)
            print(f"linear {M}x{N}x{K} {what}: max {mx:.3e} mean {mn:.3e}, plan state "
                  f"{lib.load().vm_linear_plan_state(*prob)}")
            assert mx <= TOL_MAX and mn <= TOL_MEAN

        assert lib.load().vm_linear_plan_state(*prob) == -2  # no plan yet
        if M == 1000:
            # the very first call is captured: the plan is built untuned
            sess = vm.CaptureSession().capture(run)
            assert lib.load().vm_linear_plan_state(*prob) == -1
            y.zero_()
            sess.launch()
            check("first call captured, replayed")
            sess.close()
            lib.call("vm_linear_tune", *prob)
        else:
            lib.call("vm_linear_tune", *prob)  # tuned before any call
        pick = lib.load().vm_linear_plan_state(*prob)
        assert pick >= 0
        y.zero_()
        run()
        check("eager after tuning")
        sess = vm.CaptureSession().capture(run)
        y.zero_()
        sess.launch()
        check("captured after tuning")
        sess.close()
        lib.call("vm_linear_tune", *prob)  # a second tune keeps the plan
        assert lib.load().vm_linear_plan_state(*prob) == pick


def _layer(vm, cfg, seed):
    qw = normal_bf16((D,), seed + 1, scale=0.05)
    kw = normal_bf16((D,), seed + 2, scale=0.05)
    Wqkv = normal_bf16((S * D, DM), seed + 6, scale=DM ** -0.5)
    Wo = normal_bf16((DM, HQ * D), seed + 7, scale=(HQ * D) ** -0.5)
    return qw, kw, Wqkv, Wo


def test_decode_layer_config1(vm, orc):
    """BASELINE config 1 through the whole layer: xn -> qkv GEMV -> gated decode
    -> Wo GEMV -> h, against the oracle; the appended cache row too."""
    banner("decode layer config1 B=1 ctx=512 pos=512")
    B, ctx, pos = 1, 512, 512
    cfg = vm.AttnConfig(D=DM, Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=ctx,
                        B=B)
    qw, kw, Wqkv, Wo = _layer(vm, cfg, 1000)
    kc, vc = normal_bf16((B, HK, ctx, D), 1003), normal_bf16((B, HK, ctx, D), 1004)
    xn = normal_bf16((B, DM), 1005)
    m = vm.AttnModel(cfg)
    layer = vm.AttnLayer(qw=to_dev(qw), kw=to_dev(kw), K_cache=to_dev(kc), V_cache=to_dev(vc),
                         Wqkv=to_dev(Wqkv), Wo=to_dev(Wo))
    gen = vm.Generation(B)
    gen.positions.fill_(pos)
    h = torch.empty((B, DM), dtype=torch.bfloat16, device="cuda")
    vm.decode_(h, layer, m, gen, to_dev(xn))
    torch.cuda.synchronize()
    c, s = orc.rope_tables(HALF, ctx, THETA)
    ref, kn, _ = orc.decode_layer(xn, Wqkv, Wo, kc, vc, np.array([pos], np.int32), qw, kw, c, s,
                                  Hq=HQ, Hk=HK, eps=EPS, w_offset=1.0)
    mx, mn = maxmean(dev_f32(h), ref)
    kmx, _ = maxmean(bf16_to_f32(from_dev(layer.K_cache)[0, :, pos - 1]), kn[0])
    print(f"decode layer: h max {mx:.3e} mean {mn:.3e} (|h| max {np.abs(ref).max():.3f}); "
          f"K max {kmx:.3e}")
    assert mx <= TOL_MAX and mn <= TOL_MEAN and kmx <= TOL_MAX


def test_prefill_layer_config2(vm, orc):
    """BASELINE config 2 through the whole layer: xn -> qkv GEMM -> gated prefill
    -> Wo GEMM -> h, T = 4096; every 16th row against the oracle."""
    banner("prefill layer config2 T=4096")
    B, T = 1, 4096
    cfg = vm.AttnConfig(D=DM, Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=T,
                        B=B)
    qw, kw, Wqkv, Wo = _layer(vm, cfg, 2000)
    xn = normal_bf16((B, T, DM), 2005)
    m = vm.AttnModel(cfg)
    layer = vm.attn_layer(cfg, to_dev(qw), to_dev(kw), Wqkv=to_dev(Wqkv), Wo=to_dev(Wo))
    h = vm.forward(layer, m, to_dev(xn), T, B)
    torch.cuda.synchronize()
    zero = np.zeros((B, HK, T, D), np.uint16)
    c, s = orc.rope_tables(HALF, T, THETA)
    ref, kn, _ = orc.prefill_layer(xn, Wqkv, Wo, zero, zero, np.zeros(B, np.int32),
                                   np.full(B, T, np.int32), qw, kw, c, s, Hq=HQ, Hk=HK, eps=EPS,
                                   w_offset=1.0, row_step=16)
    got = dev_f32(h)
    fin = ~np.isnan(ref)
    mx, mn = maxmean(got[fin], ref[fin])
    # the appended rows against the oracle's K norm + RoPE of the GPU's own qkv
    # (the projection is deterministic: the same plan gives the same bits); the
    # oracle's own bf16 qkv differs from it by summation-order roundings
    qkv_gpu = from_dev(vm.linear(to_dev(xn).reshape(T, DM), to_dev(Wqkv))["y"])
    _, kn, _ = orc.gated_prefill(qkv_gpu.reshape(B, T, S, D), zero, zero, np.zeros(B, np.int32),
                                 np.full(B, T, np.int32), qw, kw, c, s, Hq=HQ, Hk=HK, eps=EPS,
                                 w_offset=1.0, row_step=T)
    kmx, kmn = maxmean(bf16_to_f32(from_dev(layer.K_cache)[0]).reshape(HK, T, D), kn[0])
    print(f"prefill layer: h max {mx:.3e} mean {mn:.3e} (|h| max {np.nanmax(np.abs(ref)):.3f}); "
          f"K max {kmx:.3e} mean {kmn:.3e}")
    assert mx <= TOL_MAX and mn <= TOL_MEAN and kmx <= TOL_MAX and kmn <= TOL_MEAN


def test_decode_layer_graph_replay(vm, orc):
    """The whole layer step (qkv GEMV, gated attention, Wo GEMV, clock advance)
    captured once in a hipGraph; 16 replays equal 16 eager steps bit for bit,
    hidden states and cache rows (generate.jl:136-137, 185-191)."""
    banner("decode layer graph replay B=4 ctx=2048")
    B, ctx, n = 4, 2048, 16
    p0 = np.array([1500, 7, 2000, 640], np.int32)
    cfg = vm.AttnConfig(D=DM, Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=ctx,
                        B=B)
    qw, kw, Wqkv, Wo = _layer(vm, cfg, 3000)
    K0 = to_dev(normal_bf16((B, HK, ctx, D), 3003))
    V0 = to_dev(normal_bf16((B, HK, ctx, D), 3004))
    xn = to_dev(normal_bf16((B, DM), 3005))
    m = vm.AttnModel(cfg)
    layer = vm.AttnLayer(qw=to_dev(qw), kw=to_dev(kw), K_cache=K0.clone(), V_cache=V0.clone(),
                         Wqkv=to_dev(Wqkv), Wo=to_dev(Wo))
    h = torch.empty((B, DM), dtype=torch.bfloat16, device="cuda")
    gen = vm.Generation(B)
    gen.positions.copy_(i32(p0))
    eager = []
    for _ in range(n):
        vm.decode_(h, layer, m, gen, xn, advance=True)
        eager.append(h.clone())
    torch.cuda.synchronize()
    K_e, V_e = layer.K_cache.clone(), layer.V_cache.clone()
    layer.K_cache.copy_(K0)
    layer.V_cache.copy_(V0)
    gen.positions.copy_(i32(p0))
    torch.cuda.synchronize()
    sess = vm.CaptureSession().capture(lambda: vm.decode_(h, layer, m, gen, xn, advance=True), models=(m,))
    replay = []
    for _ in range(n):
        sess.launch()
        replay.append(h.clone())
    torch.cuda.synchronize()
    sess.close()
    assert np.array_equal(gen.positions.cpu().numpy(), p0 + n)
    for a, b in zip(eager, replay):
        assert torch.equal(a, b)
    assert torch.equal(K_e, layer.K_cache) and torch.equal(V_e, layer.V_cache)
    assert torch.isfinite(replay[-1].float()).all()
