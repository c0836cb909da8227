"""Benchmark of the gated full-attention path on one MI355X.

Headline (BASELINE.json ``metric``, configs[1]): causal gated-attention prefill,
B=1, T=4096, 16 q / 4 kv heads, head_dim 256, 64-dim partial RoPE (theta 1e7).
One step = vm_gated_attn_prefill over one synthetic packed projection: one
kernel for the K/V norm+RoPE cache append and the V -> V^T workspace staging,
then the flash-attention kernel with the q norm+RoPE prologue and sigmoid-gate
epilogue. ``value`` = algorithmic TFLOP/s =
4*D*Hq*sum_{i=1..T} i / step time (QK^T + PV over unmasked pairs only).

Also reported (same JSON line, key "decode"): BASELINE configs 3 (B=32 batched
decode, lengths ~U{1024..32768}) and 4 (B=1 at 131072 tokens, one step captured
in a hipGraph and replayed 256 times on a dedicated stream with the position
advancing on the device; under the HIP runtime's default graph launch path, and
again in a child process with DEBUG_CLR_GRAPH_PACKET_CAPTURE=0 as
"config4.packet_capture_off")
in HBM GB/s of K/V actually attended (4096 B per token) + 32 KiB per sequence,
and config 1 (B=1 at 512 tokens, launch-latency-bound) as time per step.
Key "prefill_config2_online_max": the config-2 prefill with one K-norm weight
of 4 (kw[0] = 4), whose logit bound passes the static shift's 64 so the kernel
takes its online-max softmax; "decode.config3_running_max" likewise for config 3.
Key "prefill_config5": BASELINE config 5 (B=4 ragged chunks after 8-32 K
priors) in algorithmic TFLOP/s, step and attention kernel, and the step with the
layer's V^T workspace kept between chunks (staging the chunk only). Key "decode_step": the
whole captured decode step of a Qwen3.5-4B-shaped model (24 Gated DeltaNet + 8
gated-attention layers, MLPs, lm head; B = 32), and the lm-head GEMV + argmax
alone. Key "prefill_model": prefill! of that model at B = 1 over 4096 prompt
tokens, eager (tokens/s, TFLOP/s of its projections and attention). Key "deltanet": the DeltaNet layer kernels alone (fused decode step and
conv step against the HBM roofline, the prefill recurrence in tokens/s). Key "layer": whole
attention layers, hidden state to hidden state (the qkv and Wo projections on
hipBLASLt around the block) at the config-2 prefill and config-3 decode shapes.

``roofline`` is for the dominant kernel (the prefill attention kernel): its
launches, and only its, are bracketed by hipEvents on the launch stream inside
the timed region (libvallmo_attn's vm_profile_*); the other kernels are timed
in separate untimed passes. Before the timed steps, after --warmup steps, a
clock-settle phase runs untimed steps until successive block means of the
attention kernel agree within 1% (``settle_ms`` in the JSON line).
``cpu_baseline`` times the C fp32 oracle (oracle/, test infrastructure) on this
host's cores for every config (key "configs"), with the CPU model and core count.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-decode]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

# Graph replays (config 4) run under the HIP runtime's default settings. The
# runtime's DEBUG_CLR_GRAPH_PACKET_CAPTURE=0 (its plain dispatch path for graph
# kernels) saves ~3 us per replay on this ROCm image; config 4 is measured that
# way too, in a child process started before this one touches the GPU (the
# variable is read when HIP initialises), and both figures are reported.
PACKET_CAPTURE_VAR = "DEBUG_CLR_GRAPH_PACKET_CAPTURE"

HQ, HK, D, HALF, THETA, EPS = 16, 4, 256, 32, 1.0e7, 1.0e-6
S = 2 * HQ + 2 * HK
PEAK_BF16_TFLOPS = 2516.6   # 256 CU x 2.4 GHz x 4096 FLOP/clk (dense bf16 MFMA)
PEAK_HBM_GBS = 8000.0


def prefill_flops(T: int, prior: int = 0) -> float:
    """4*D*Hq*sum over unmasked (q,k) pairs: row t sees prior + t + 1 keys."""
    return 4.0 * D * HQ * (T * prior + T * (T + 1) / 2)


def profiled_traffic(name="prefill_fused_kernel_config2.md"):
    """HBM bytes per launch of the prefill kernel from the committed rocprofv3
    FETCH_SIZE/WRITE_SIZE summary (counters cannot be read from inside this
    process); None when the summary is absent."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def settle_clocks(vm, torch, step, block=20, tol=0.01, min_s=0.25, max_s=5.0):
    """Untimed steps until the GPU clocks have settled: blocks of `block` steps
    are run with the attention kernel on its own events, until the last three
    block means agree within `tol` (after at least min_s, at most max_s). A cold
    GPU runs its first tens of milliseconds at lower clocks (the first 20 prefill
    launches average ~169 us against ~140 us settled); --warmup alone counts
    steps, not time, so this phase keeps the timed steps off that ramp."""
    lib = vm._lib
    means = []
    t0 = time.perf_counter()
    n = 0
    while True:
        lib.profile_select(lib.VM_K_PREFILL)
        lib.profile_enable(True)
        for _ in range(block):
            step()
        torch.cuda.synchronize()
        k, ms = lib.profile_read(lib.VM_K_PREFILL)
        lib.profile_enable(False)
        lib.profile_select()
        n += block
        means.append(ms / max(k, 1))
        el = time.perf_counter() - t0
        if el >= max_s:
            break
        if el >= min_s and len(means) >= 3:
            last = means[-3:]
            if max(last) / min(last) - 1.0 < tol:
                break
    return {"settle_ms": round(1e3 * (time.perf_counter() - t0), 1), "settle_steps": n,
            "block_means_us": [round(1e3 * m, 2) for m in means[:3]] + ["..."] +
                              [round(1e3 * m, 2) for m in means[-3:]]
            if len(means) > 6 else [round(1e3 * m, 2) for m in means]}


def _big_kw0(kw, kw0):
    """kw[0] = kw0 (bf16): with (w + 1) weights, max|kw + 1| = kw0 + 1 lifts the
    static logit bound past 64 (log2 units), so the kernels take their exact
    online-max softmax (prefill and decode alike: a running row max, rescaled
    lazily)."""
    if kw0 is not None:
        kw[0] = float(kw0)


def bench_prefill(vm, torch, steps, warmup, T=4096, seed=2, settle=True, kw0=None):
    B, ctx = 1, T
    cfg = vm.AttnConfig(Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=ctx, B=B)
    qw = torch.empty(D, dtype=torch.bfloat16, device="cuda")
    kw = torch.empty_like(qw)
    vm.fill_normal_(qw, seed * 100 + 1, scale=0.05)
    vm.fill_normal_(kw, seed * 100 + 2, scale=0.05)
    _big_kw0(kw, kw0)
    qkv = torch.empty((B, T, S, D), dtype=torch.bfloat16, device="cuda")
    vm.fill_normal_(qkv, seed * 100 + 3)
    m = vm.AttnModel(cfg)
    layer = vm.attn_layer(cfg, qw, kw)
    out = torch.empty((B, T, HQ * D), dtype=torch.bfloat16, device="cuda")
    prior = torch.zeros((B,), dtype=torch.int32, device="cuda")

    def step():
        vm.gated_attn_prefill(layer, m, qkv, T, B, prior=prior, out=out)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    lib = vm._lib
    settle = settle_clocks(vm, torch, step) if settle else {"settle_ms": 0.0, "settle_steps": 0}
    # timed region: the whole steps, no events inside (each per-dispatch event
    # pair costs the step a few microseconds)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # the same steps again with HIP events around each dispatch of the
    # attention kernel (the roofline's launch time)
    lib.profile_select(lib.VM_K_PREFILL)
    lib.profile_enable(True)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    n_attn, ms_attn = lib.profile_read(lib.VM_K_PREFILL)
    lib.profile_enable(False)
    assert n_attn == steps
    # untimed: the append + V^T staging kernel on its own events
    lib.profile_select(lib.VM_K_ROWS)
    lib.profile_enable(True)
    n_side = min(steps, 20)
    for _ in range(n_side):
        step()
    torch.cuda.synchronize()
    n_rows, ms_rows = lib.profile_read(lib.VM_K_ROWS)
    lib.profile_enable(False)
    lib.profile_select()
    assert n_rows == n_side
    flops = prefill_flops(T)
    return {
        "settle": settle,
        "ms_per_step": 1e3 * wall / steps,
        "tflops": flops / (wall / steps) / 1e12,
        "attn_kernel_ms": ms_attn / n_attn,
        "append_vt_kernel_ms": ms_rows / n_rows,
        "flops": flops,
    }


def bench_prefill5(vm, torch, steps, warmup, seed=5):
    """Config 5: B=4 ragged chunks (a seeded permutation of {512, 1024, 2048, 2048})
    after prior caches ~U{8192..32768} (the same draws as the config-5 GPU test)."""
    rng = np.random.default_rng(seed)
    qlen = rng.permutation(np.array([512, 1024, 2048, 2048], np.int32)).astype(np.int32)
    prior = rng.integers(8192, 32769, size=4).astype(np.int32)
    B, T = 4, int(qlen.max())
    ctx = int((prior + qlen).max())
    cfg = vm.AttnConfig(Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=ctx, B=B)
    qw = torch.empty(D, dtype=torch.bfloat16, device="cuda")
    kw = torch.empty_like(qw)
    vm.fill_normal_(qw, seed * 100 + 1, scale=0.05)
    vm.fill_normal_(kw, seed * 100 + 2, scale=0.05)
    layer = vm.attn_layer(cfg, qw, kw)
    vm.fill_normal_(layer.K_cache, seed * 100 + 3)
    vm.fill_normal_(layer.V_cache, seed * 100 + 4)
    qkv = torch.empty((B, T, S, D), dtype=torch.bfloat16, device="cuda")
    vm.fill_normal_(qkv, seed * 100 + 5)
    m = vm.AttnModel(cfg)
    out = torch.empty((B, T, HQ * D), dtype=torch.bfloat16, device="cuda")
    pr = torch.from_numpy(prior).cuda()
    ql = torch.from_numpy(qlen).cuda()

    def step():   # appends the same chunk columns each time: same work per step
        vm.gated_attn_prefill(layer, m, qkv, T, B, prior=pr, q_lengths=ql, out=out)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    lib = vm._lib
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # the attention kernel's per-dispatch events, over the same steps again
    lib.profile_select(lib.VM_K_PREFILL)
    lib.profile_enable(True)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    n_attn, ms_attn = lib.profile_read(lib.VM_K_PREFILL)
    lib.profile_enable(False)
    lib.profile_select()
    assert n_attn == steps
    # the same chunk with the layer's V^T workspace kept (StagedV, as a chunk-by-
    # chunk prefill runs): after the first call, a call stages the chunk's rows only
    staged = vm.StagedV(cfg, B)
    vm.gated_attn_prefill(layer, m, qkv, T, B, prior=pr, q_lengths=ql, out=out, staged=staged)
    for _ in range(warmup):
        vm.gated_attn_prefill(layer, m, qkv, T, B, prior=pr, q_lengths=ql, out=out, staged=staged)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        vm.gated_attn_prefill(layer, m, qkv, T, B, prior=pr, q_lengths=ql, out=out, staged=staged)
    torch.cuda.synchronize()
    wall_staged = time.perf_counter() - t0
    del staged
    c, p = qlen.astype(np.float64), prior.astype(np.float64)
    flops = float(4 * D * HQ * np.sum(c * p + c * (c + 1) / 2))
    kms = ms_attn / n_attn
    return {
        "config": f"config5: ragged chunked prefill B=4 chunks={qlen.tolist()} "
                  f"priors={prior.tolist()} (seed {seed})",
        "flop_per_step": flops,
        "ms_per_step": 1e3 * wall / steps,
        "tflops": flops / (wall / steps) / 1e12,
        "ms_per_step_staged": 1e3 * wall_staged / steps,
        "tflops_staged": flops / (wall_staged / steps) / 1e12,
        "attn_kernel_ms": kms,
        "attn_kernel_tflops": flops / (kms * 1e-3) / 1e12,
        "frac_of_bf16_peak": flops / (kms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
    }


def bench_decode1(vm, torch, steps, warmup, seed=1):
    """Config 1: B=1, attended length 512 (prior 511 tokens + the new one)."""
    B, ctx, L = 1, 512, 512
    cfg = vm.AttnConfig(Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=ctx, B=B)
    qw = torch.empty(D, dtype=torch.bfloat16, device="cuda")
    kw = torch.empty_like(qw)
    vm.fill_normal_(qw, seed * 100 + 1, scale=0.05)
    vm.fill_normal_(kw, seed * 100 + 2, scale=0.05)
    layer = vm.attn_layer(cfg, qw, kw)
    vm.fill_normal_(layer.K_cache, seed * 100 + 3)
    vm.fill_normal_(layer.V_cache, seed * 100 + 4)
    qkv = torch.empty((B, S, D), dtype=torch.bfloat16, device="cuda")
    vm.fill_normal_(qkv, seed * 100 + 5)
    m = vm.AttnModel(cfg)
    gen = vm.Generation(B)
    gen.positions.fill_(L)
    O = torch.empty((B, HQ, D), dtype=torch.bfloat16, device="cuda")
    for _ in range(warmup):
        vm.gated_attn_decode_(O, layer, m, gen, qkv)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        vm.gated_attn_decode_(O, layer, m, gen, qkv)   # same position each step: same bytes
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    nbytes = decode_bytes([L])
    return {
        "config": "config1: decode B=1 at attended length 512 (launch-latency-bound parity config)",
        "bytes_per_step": nbytes,
        "us_per_step": 1e6 * wall / steps,
        "gbs": nbytes / (wall / steps) / 1e9,
    }


def decode_bytes(lengths):
    return float(np.sum(np.asarray(lengths, np.float64)) * 4096.0 + 32768.0 * len(lengths))


def bench_decode3(vm, torch, steps, warmup, seed=3, kw0=None):
    B, ctx = 32, 32768
    rng = np.random.default_rng(seed)
    lengths = rng.integers(1024, 32769, size=B).astype(np.int32)
    cfg = vm.AttnConfig(Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=ctx, B=B)
    qw = torch.empty(D, dtype=torch.bfloat16, device="cuda")
    kw = torch.empty_like(qw)
    vm.fill_normal_(qw, 301, scale=0.05)
    vm.fill_normal_(kw, 302, scale=0.05)
    _big_kw0(kw, kw0)
    layer = vm.attn_layer(cfg, qw, kw)
    vm.fill_normal_(layer.K_cache, 303)
    vm.fill_normal_(layer.V_cache, 304)
    qkv = torch.empty((B, S, D), dtype=torch.bfloat16, device="cuda")
    vm.fill_normal_(qkv, 305)
    m = vm.AttnModel(cfg)
    gen = vm.Generation(B)
    pos = torch.from_numpy(lengths).cuda()
    O = torch.empty((B, HQ, D), dtype=torch.bfloat16, device="cuda")
    for _ in range(warmup):
        gen.positions.copy_(pos)
        vm.gated_attn_decode_(O, layer, m, gen, qkv)
    torch.cuda.synchronize()
    gen.positions.copy_(pos)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        vm.gated_attn_decode_(O, layer, m, gen, qkv)   # same position each step: same bytes
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # untimed: both kernels on their own hipEvents
    lib = vm._lib
    lib.profile_enable(True)
    for _ in range(min(steps, 20)):
        vm.gated_attn_decode_(O, layer, m, gen, qkv)
    torch.cuda.synchronize()
    n_s, ms_s = lib.profile_read(lib.VM_K_DECODE_SPLIT)
    n_c, ms_c = lib.profile_read(lib.VM_K_DECODE_COMBINE)
    lib.profile_enable(False)
    nbytes = decode_bytes(lengths)
    step_s = wall / steps
    return {
        "config": "config3: batched decode B=32, lengths~U{1024..32768} (seed 3), capacity 32768",
        "bytes_per_step": nbytes,
        "ms_per_step": 1e3 * step_s,
        "gbs": nbytes / step_s / 1e9,
        "split_kernel_ms": ms_s / n_s,
        "split_kernel_gbs": nbytes / (ms_s / n_s * 1e-3) / 1e9,
        "combine_kernel_ms": ms_c / n_c,
    }


def bench_decode4(vm, torch, replays=256, seed=4):
    B, p0 = 1, 131072
    ctx = p0 + replays
    cfg = vm.AttnConfig(Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=ctx, B=B)
    qw = torch.empty(D, dtype=torch.bfloat16, device="cuda")
    kw = torch.empty_like(qw)
    vm.fill_normal_(qw, 401, scale=0.05)
    vm.fill_normal_(kw, 402, scale=0.05)
    layer = vm.attn_layer(cfg, qw, kw)
    vm.fill_normal_(layer.K_cache, 403)
    vm.fill_normal_(layer.V_cache, 404)
    qkv = torch.empty((B, S, D), dtype=torch.bfloat16, device="cuda")
    vm.fill_normal_(qkv, 405)
    m = vm.AttnModel(cfg)
    gen = vm.Generation(B)
    O = torch.empty((B, HQ, D), dtype=torch.bfloat16, device="cuda")
    # eager warmup + split-kernel timing at the first position
    gen.positions.fill_(p0)
    for _ in range(3):
        vm.gated_attn_decode_(O, layer, m, gen, qkv)
    torch.cuda.synchronize()
    lib = vm._lib
    lib.profile_enable(True)
    for _ in range(10):
        vm.gated_attn_decode_(O, layer, m, gen, qkv)
    torch.cuda.synchronize()
    n_s, ms_s = lib.profile_read(lib.VM_K_DECODE_SPLIT)
    lib.profile_enable(False)
    gen.positions.fill_(p0)
    torch.cuda.synchronize()
    sess = vm.CaptureSession().capture(lambda: vm.gated_attn_decode_(O, layer, m, gen, qkv, advance=True))
    # replays on a stream of their own, as a serving loop runs them (the
    # reference's generate loop replays on its task's stream): launches on the
    # legacy default stream measure ~4 us more per replay (implicit
    # synchronisation with the other streams)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(replays):
            sess.launch()
        stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop)
    assert gen.positions.item() == p0 + replays
    sess.close()
    lengths = np.arange(p0, p0 + replays)
    nbytes = decode_bytes(lengths) / replays
    return {
        "config": "config4: long-context decode B=1, 131072..131327 tokens, 256 hipGraph replays",
        "launch": "hipGraphLaunch on a dedicated non-default stream",
        "runtime_env": {"DEBUG_CLR_GRAPH_PACKET_CAPTURE":
                        os.environ.get("DEBUG_CLR_GRAPH_PACKET_CAPTURE", "(runtime default)")},
        "bytes_per_replay": nbytes,
        "ms_per_replay": ms / replays,
        "gbs": nbytes / (ms / replays * 1e-3) / 1e9,
        "split_kernel_ms": ms_s / n_s,
        "split_kernel_gbs": (p0 * 4096.0 + 32768) / (ms_s / n_s * 1e-3) / 1e9,
    }


DM = 2560   # hidden size of the layer benchmarks (the Qwen3.5 small-model width)


def _event_ms(torch, fn, reps):
    """Mean ms of fn() over reps launches on torch's current stream (events)."""
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def _graph_ms(torch, fn, n=20, reps=5):
    """Median ms of one fn() call: n calls captured in a graph on a side stream,
    replayed reps times (kernel time without the host's per-call dispatch)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        fn()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=side):
            for _ in range(n):
                fn()
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ts = []
    for _ in range(reps):
        a.record()
        g.replay()
        b.record()
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b) / n)
    del g
    return float(np.median(ts))


def _cold_gemv_ms(vm, torch, W, x, y, ws, total_bytes=1.2e9):
    """ms per y = W^T x with W streamed from HBM: the graph rotates over copies
    of W (total > the last-level cache), one call per copy."""
    nc = max(2, int(total_bytes // (W.numel() * 2)) + 1)
    Ws = [W.clone() for _ in range(nc)]
    calls = [(lambda Wc=Wc: vm.linear_({"y": y}, x, Wc, workspace=ws)) for Wc in Ws]
    t = _graph_ms(torch, lambda: [f() for f in calls], n=1) / nc
    del Ws
    return t


def bench_layer(vm, torch, reps=20):
    """Whole attention layers, hidden state to hidden state (qkv projection,
    gated attention, Wo projection): the config-2 prefill layer (T = 4096) and the
    config-3-shaped decode layer (B = 32), with the projections (hipBLASLt) timed
    alone against their rooflines: GEMM FLOP / bf16 peak, GEMV weight bytes / HBM."""
    res = {}
    S_ = 2 * HQ + 2 * HK
    # ---- prefill layer, config 2
    T, B = 4096, 1
    cfg = vm.AttnConfig(D=DM, Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=T, B=B)
    qw = torch.empty(D, dtype=torch.bfloat16, device="cuda")
    kw = torch.empty_like(qw)
    vm.fill_normal_(qw, 2001, scale=0.05)
    vm.fill_normal_(kw, 2002, scale=0.05)
    Wqkv = torch.empty((S_ * D, DM), dtype=torch.bfloat16, device="cuda")
    Wo = torch.empty((DM, HQ * D), dtype=torch.bfloat16, device="cuda")
    vm.fill_normal_(Wqkv, 2006, scale=DM ** -0.5)
    vm.fill_normal_(Wo, 2007, scale=(HQ * D) ** -0.5)
    xn = torch.empty((B, T, DM), dtype=torch.bfloat16, device="cuda")
    vm.fill_normal_(xn, 2005)
    m = vm.AttnModel(cfg)
    layer = vm.attn_layer(cfg, qw, kw, Wqkv=Wqkv, Wo=Wo)
    fwd = lambda: vm.forward(layer, m, xn, T, B)
    for _ in range(5):
        fwd()
    torch.cuda.synchronize()
    t_layer = _event_ms(torch, fwd, reps)
    x2 = xn.view(T, DM)
    qkv = torch.empty((T, S_ * D), dtype=torch.bfloat16, device="cuda")
    o = torch.empty((T, HQ * D), dtype=torch.bfloat16, device="cuda")
    h = torch.empty((T, DM), dtype=torch.bfloat16, device="cuda")
    ws = m.linear_workspace()
    t_qkv = _event_ms(torch, lambda: vm.linear_({"y": qkv}, x2, Wqkv, workspace=ws), reps)
    t_wo = _event_ms(torch, lambda: vm.linear_({"y": h}, o, Wo, workspace=ws), reps)
    f_qkv, f_wo = 2.0 * T * DM * S_ * D, 2.0 * T * HQ * D * DM
    f_attn = prefill_flops(T)
    res["prefill_config2"] = {
        "ms_per_layer": t_layer,
        "tflops_layer": (f_qkv + f_wo + f_attn) / (t_layer * 1e-3) / 1e12,
        "qkv_gemm_ms": t_qkv, "qkv_gemm_tflops": f_qkv / (t_qkv * 1e-3) / 1e12,
        "qkv_gemm_frac_of_bf16_peak": f_qkv / (t_qkv * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
        "wo_gemm_ms": t_wo, "wo_gemm_tflops": f_wo / (t_wo * 1e-3) / 1e12,
        "wo_gemm_frac_of_bf16_peak": f_wo / (t_wo * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
        "shape": f"hidden {DM}, T {T}: qkv {T}x{DM} -> {S_ * D}, Wo {T}x{HQ * D} -> {DM}",
    }
    del layer, m, qkv, o, h, xn, x2
    # ---- decode layer, config-3 shape (B = 32, lengths ~U{1024..32768})
    B, ctx = 32, 32768
    lengths = np.random.default_rng(3).integers(1024, 32769, size=B).astype(np.int32)
    cfg = vm.AttnConfig(D=DM, Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=ctx, B=B)
    m = vm.AttnModel(cfg)
    layer = vm.attn_layer(cfg, qw, kw, Wqkv=Wqkv, Wo=Wo)
    vm.fill_normal_(layer.K_cache, 303)
    vm.fill_normal_(layer.V_cache, 304)
    xd = torch.empty((B, DM), dtype=torch.bfloat16, device="cuda")
    vm.fill_normal_(xd, 3005)
    hd = torch.empty_like(xd)
    gen = vm.Generation(B)
    gen.positions.copy_(torch.from_numpy(lengths).cuda())
    step = lambda: vm.decode_(hd, layer, m, gen, xd)
    for _ in range(3):
        step()
    torch.cuda.synchronize()
    t_step = _event_ms(torch, step, reps)
    qkv_d, O_d = m.decode_buffers()
    ws = m.decode_workspace()
    # the GEMVs alone, timed from graph replays (a host loop of these ~10 us
    # launches measures Python's dispatch, not the kernels) that rotate over
    # copies of the weight totalling > 1 GB, so each call streams it from HBM as
    # in a decode step (one copy re-read would sit in the 256 MB last-level cache)
    t_gv1 = _cold_gemv_ms(vm, torch, Wqkv, xd, qkv_d.view(B, -1), ws)
    t_gv2 = _cold_gemv_ms(vm, torch, Wo, O_d.view(B, -1), hd, ws)
    b_qkv = 2.0 * (S_ * D * DM + B * DM + B * S_ * D)
    b_wo = 2.0 * (DM * HQ * D + B * HQ * D + B * DM)
    res["decode_config3"] = {
        "ms_per_layer_step": t_step,
        "kv_gbs_in_layer_step": decode_bytes(lengths) / (t_step * 1e-3) / 1e9,
        "qkv_gemv_ms": t_gv1, "qkv_gemv_gbs": b_qkv / (t_gv1 * 1e-3) / 1e9,
        "qkv_gemv_frac_of_hbm_peak": b_qkv / (t_gv1 * 1e-3) / 1e9 / PEAK_HBM_GBS,
        "wo_gemv_ms": t_gv2, "wo_gemv_gbs": b_wo / (t_gv2 * 1e-3) / 1e9,
        "wo_gemv_frac_of_hbm_peak": b_wo / (t_gv2 * 1e-3) / 1e9 / PEAK_HBM_GBS,
        "shape": f"hidden {DM}, B {B}: qkv {B}x{DM} -> {S_ * D}, Wo {B}x{HQ * D} -> {DM}",
    }
    return res


def bench_step(vm, torch, replays=40, seed=9):
    """The whole decode step (step!, qwen35.jl:245-273) of a Qwen3.5-4B-shaped
    model: 32 layers in its pattern (every 4th gated full attention, the rest
    Gated DeltaNet: Dk = Dv = 128, 16 qk / 32 value heads, conv 4), hidden 2560,
    MLP 9216, vocab 151936 (tied head), random weights; B = 32 with the attention
    layers at ragged attended lengths ~U{1024..8128}: (step!; advance!) captured
    once and replayed on a dedicated stream. HBM bytes per step: every weight once
    (projections, MLPs, conv, head), the attended K/V, the DeltaNet states read
    and written (fp32) and their conv rings. Also the lm head alone (GEMV +
    argmax) at B = 1 and 32."""
    B, Ctx, L = 32, 8192, 32
    a = vm.AttnConfig(D=DM, Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=Ctx, B=B)
    cfg = vm.ModelConfig(attn=a, inter=9216, vocab=151936, n_layers=L, tied=True, interval=4)
    m = vm.random_model(cfg, seed=seed)
    attn = [l for l in m.layers if not isinstance(l, vm.DeltaNetLayer)]
    for i, l in enumerate(attn):
        vm.fill_normal_(l.K_cache, 9000 + i)
        vm.fill_normal_(l.V_cache, 9100 + i)
    rng = np.random.default_rng(seed)
    pos0 = rng.integers(1024, Ctx - replays - 8, size=B).astype(np.int32)
    gen = vm.Generation(B, replays + 16)
    gen.positions.copy_(torch.as_tensor(pos0).cuda())
    gen.result.copy_(torch.as_tensor(rng.integers(1, cfg.vocab + 1, size=B).astype(np.int32)).cuda())
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):   # warm-up: plans, workspace
            vm.step_(m, gen)
            gen.advance_()
        sess = vm.CaptureSession().capture(lambda: (vm.step_(m, gen), gen.advance_()), models=(m.attn,))
        for _ in range(3):
            sess.launch()
        p_start = gen.positions.clone()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(replays):
            sess.launch()
        e1.record()
    torch.cuda.synchronize()
    sess.close()
    ms = e0.elapsed_time(e1) / replays
    p_start = p_start.cpu().numpy().astype(np.float64)
    La = len(attn)
    kv = float(np.sum(p_start + (replays - 1) / 2.0)) * HK * D * 2 * 2 * La  # attended K + V
    w_bytes = float(m.head.numel() * 2)
    for l in m.layers:
        ts = ((l.W_in, l.Wout, l.conv_w) if isinstance(l, vm.DeltaNetLayer)
              else (l.Wqkv, l.Wo))
        w_bytes += sum(t.numel() * 2 for t in ts + (l.Wgu, l.Wd))
    dn_state = float(sum(2 * l.S.numel() * 4 + 2 * l.conv_state.numel() * 2
                         for l in m.dn_layers))
    nbytes = w_bytes + kv + dn_state
    res = {
        "config": f"Qwen3.5-4B shape: {L} layers ({L - La} Gated DeltaNet + {La} gated attention, "
                  f"full_attention_interval 4), hidden {DM}, MLP {cfg.inter}, vocab {cfg.vocab} "
                  f"(tied head), random weights, B={B}, attended lengths U{{1024..8128}} (seed "
                  f"{seed}), (step!; advance!) captured, {replays} replays on a dedicated stream",
        "ms_per_step": ms,
        "tokens_per_s": B / (ms * 1e-3),
        "bytes_per_step": nbytes,
        "weight_bytes": w_bytes,
        "kv_bytes": kv,
        "deltanet_state_bytes": dn_state,
        "gbs": nbytes / (ms * 1e-3) / 1e9,
        "frac_of_hbm_peak": nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
    }
    # the lm head alone
    lib = vm._lib
    for b in (1, B):
        x = m.xn[:b]
        out = torch.empty((b,), dtype=torch.int32, device="cuda")
        sc = torch.empty(max(vm.lm_head_argmax_scratch_bytes(x, m.head), 16), dtype=torch.uint8,
                         device="cuda")
        for _ in range(3):
            vm.lm_head_argmax_({"Result": out}, x, m.head, scratch=sc)
        lib.profile_select(lib.VM_K_LM_HEAD)
        lib.profile_enable(True)
        for _ in range(20):
            vm.lm_head_argmax_({"Result": out}, x, m.head, scratch=sc)
        torch.cuda.synchronize()
        n, t = lib.profile_read(lib.VM_K_LM_HEAD)
        lib.profile_enable(False)
        lib.profile_select()
        hb = m.head.numel() * 2.0
        res[f"lm_head_B{b}"] = {"us": 1e3 * t / n, "gbs": hb / (t / n * 1e-3) / 1e9,
                                "frac_of_hbm_peak": hb / (t / n * 1e-3) / 1e9 / PEAK_HBM_GBS}
    del m
    torch.cuda.empty_cache()
    return res


def bench_prefill_model(vm, torch, T=4096, runs=5, seed=13):
    """prefill!(m, gen, ids) (qwen35.jl:369-395) of the same Qwen3.5-4B-shaped
    model as bench_step at B = 1 over T = 4096 prompt tokens, eager, from a reset
    state: embedding, 24 Gated DeltaNet layers (projection, sequence conv, prep,
    chunked recurrence, gated norm, out projection), 8 gated-attention layers
    (projection, K/V append + fused attention, Wo), the MLPs and norms, and the
    lm head for the last token. Events bracket each whole prefill. FLOP: every
    projection weight twice per token, plus the causal attention's 4 D Hq sum i
    per attention layer (the DeltaNet recurrence and the norms not counted)."""
    B, L = 1, 32
    a = vm.AttnConfig(D=DM, Hq=HQ, Hkv=HK, Dh=D, rot_half=HALF, theta=THETA, eps=EPS, Ctx=T, B=B)
    cfg = vm.ModelConfig(attn=a, inter=9216, vocab=151936, n_layers=L, tied=True, interval=4)
    m = vm.random_model(cfg, seed=seed)
    gen = vm.Generation(B, 16)
    rng = np.random.default_rng(seed)
    ids = torch.as_tensor(rng.integers(1, cfg.vocab + 1, size=(B, T)).astype(np.int32)).cuda()
    for _ in range(2):
        m.reset_()
        vm.prefill_(m, gen, ids)
    torch.cuda.synchronize()
    ms = []
    for _ in range(runs):
        m.reset_()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        vm.prefill_(m, gen, ids)
        e1.record()
        torch.cuda.synchronize()
        ms.append(e0.elapsed_time(e1))
    w = 0
    for l in m.layers:
        ts = ((l.W_in, l.Wout) if isinstance(l, vm.DeltaNetLayer) else (l.Wqkv, l.Wo))
        w += sum(t.numel() for t in ts + (l.Wgu, l.Wd))
    n_attn = sum(1 for l in m.layers if not isinstance(l, vm.DeltaNetLayer))
    flops = 2.0 * w * T * B + n_attn * prefill_flops(T)
    t = float(np.median(ms))
    del m
    torch.cuda.empty_cache()
    return {
        "config": f"Qwen3.5-4B shape: {L} layers ({L - n_attn} Gated DeltaNet + {n_attn} gated "
                  f"attention), hidden {DM}, MLP {cfg.inter}, vocab {cfg.vocab} (tied head), random "
                  f"weights, B={B}, T={T} prompt tokens from a reset state, eager, median of {runs}",
        "ms": t,
        "tokens_per_s": B * T / (t * 1e-3),
        "flops": flops,
        "tflops": flops / (t * 1e-3) / 1e12,
    }


def _profiled_us(vm, torch, kernel, fn, n=20):
    """Mean us per launch of one kernel class (events around its launches)."""
    lib = vm._lib
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    lib.profile_select(kernel)
    lib.profile_enable(True)
    for _ in range(n):
        fn()
    torch.cuda.synchronize()
    cnt, t = lib.profile_read(kernel)
    lib.profile_enable(False)
    lib.profile_select()
    return 1e3 * t / cnt


def bench_deltanet(vm, torch, seed=11):
    """The Gated DeltaNet layer kernels alone at the Qwen3.5-4B shape (Dk = Dv =
    128, Hk = 16, Hv = 32, 8192 conv channels, conv 4), against the HBM roofline:
    the fused decode step (its bytes: the fp32 state read and written, q / k / v /
    z / gates read, O written) at B = 1 and 32; the decode conv step at B = 32
    (ring read and written, input, weight, output); the prefill's recurrence
    (deltanet_sequence!) over T = 4096 at B = 1 (latency-bound: reported as
    tokens/s), with its prep, conv and gated-norm kernels."""
    Dk = Dv = 128
    Hk, Hv, K = 16, 32, 4
    n = 2 * Hk * Dk + Hv * Dv
    res = {}
    f32 = dict(dtype=torch.float32, device="cuda")
    for B in (1, 32):
        qz = _dev_normal(vm, torch, (B, n + Hv * Dv), seed + B)
        ab = _dev_normal(vm, torch, (B, 2 * Hv), seed + 100 + B)
        S = torch.randn((B, Hv, Dv, Dk), **f32) * 0.05
        a_log = torch.randn((Hv,), **f32) * 0.5
        dt = torch.randn((Hv,), **f32) * 0.5
        gw = _dev_normal(vm, torch, (Dv,), seed + 7)
        O = torch.empty((B, Hv, Dv), dtype=torch.bfloat16, device="cuda")
        hk = Hk * Dk
        q = qz[:, :hk].unflatten(-1, (Hk, Dk))
        k = qz[:, hk:2 * hk].unflatten(-1, (Hk, Dk))
        v = qz[:, 2 * hk:n].unflatten(-1, (Hv, Dv))
        z = qz[:, n:].unflatten(-1, (Hv, Dv))
        fn = lambda: vm.fused_deltanet_decode_({"O": O, "Sp": S}, q, k, v, ab[:, :Hv],
                                               ab[:, Hv:], z, a_log, dt, gw, S, eps=EPS)
        us = _profiled_us(vm, torch, vm._lib.VM_K_DELTANET, fn)
        nbytes = B * Hv * (2.0 * Dk * Dv * 4 + 3 * Dv * 2 + 4) + B * 2 * hk * 2
        res[f"fused_decode_B{B}"] = {"us": us, "bytes": nbytes,
                                     "gbs": nbytes / (us * 1e-6) / 1e9,
                                     "frac_of_hbm_peak": nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS}
    B = 32
    x = _dev_normal(vm, torch, (B, n), seed + 200)
    ring = _dev_normal(vm, torch, (B, K, n), seed + 201)
    w = _dev_normal(vm, torch, (K, n), seed + 202, scale=0.5)
    y = torch.empty((B, n), dtype=torch.bfloat16, device="cuda")
    us = _profiled_us(vm, torch, vm._lib.VM_K_CONV,
                      lambda: vm.causal_conv1d_({"Y": y, "Sp": ring}, x, ring, w, None,
                                                sigma="silu"))
    nbytes = 2.0 * (B * n * (1 + (K - 1) + K + 1) + K * n)
    res["conv_decode_B32"] = {"us": us, "bytes": nbytes, "gbs": nbytes / (us * 1e-6) / 1e9,
                              "frac_of_hbm_peak": nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS}
    # prefill pieces, B = 1, T = 4096
    B, T = 1, 4096
    X = _dev_normal(vm, torch, (B, T, n), seed + 300)
    Y = torch.empty_like(X)
    Sp = torch.zeros((B, K, n), dtype=torch.bfloat16, device="cuda")
    us_conv = _profiled_us(vm, torch, vm._lib.VM_K_CONV,
                           lambda: vm.causal_conv1d_sequence_({"Y": Y}, X, w, None, sigma="silu",
                                                              Sp=Sp), n=5)
    ab = _dev_normal(vm, torch, (B, T, 2 * Hv), seed + 301)
    p = {"Q": torch.empty((B, Hk, T, Dk), **f32), "K": torch.empty((B, Hk, T, Dk), **f32),
         "V": torch.empty((B, Hv, T, Dv), **f32), "Beta": torch.empty((B, T, Hv), **f32),
         "Gate": torch.empty((B, T, Hv), **f32)}
    a_log = torch.randn((Hv,), **f32) * 0.5
    dt = torch.randn((Hv,), **f32) * 0.5
    us_prep = _profiled_us(vm, torch, vm._lib.VM_K_ROWS,
                           lambda: vm.deltanet_prefill_prep_(p, Y, ab, a_log, dt, Dk=Dk, Dv=Dv,
                                                             Hk=Hk, Hv=Hv), n=5)
    # the layer's form: the conv and the prep in one pass (the conv output not written)
    us_cp = _profiled_us(vm, torch, vm._lib.VM_K_CONV,
                         lambda: vm.deltanet_conv_prep_(p, X, w, ab, a_log, dt, Dk=Dk, Dv=Dv,
                                                        Hk=Hk, Hv=Hv, Sp=Sp), n=5)
    S = torch.zeros((B, Hv, Dv, Dk), **f32)
    o = torch.empty((B, Hv, T, Dv), **f32)
    us_seq = _profiled_us(vm, torch, vm._lib.VM_K_DELTANET,
                          lambda: vm.deltanet_sequence_({"O": o, "Sp": S}, p["Q"], p["K"], p["V"],
                                                        p["Beta"], p["Gate"], S), n=3)
    ws = torch.empty(vm.deltanet_sequence_workspace_bytes(T, Hv, B), dtype=torch.uint8,
                     device="cuda")
    us_chk = _profiled_us(vm, torch, vm._lib.VM_K_DELTANET,
                          lambda: vm.deltanet_sequence_chunked_({"O": o, "Sp": S}, p["Q"], p["K"],
                                                                p["V"], p["Beta"], p["Gate"], S,
                                                                workspace=ws), n=5)
    z = _dev_normal(vm, torch, (B, T, Hv, Dv), seed + 302)
    gw = _dev_normal(vm, torch, (Dv,), seed + 303, 0.2)
    yb = torch.empty((B, T, Hv, Dv), dtype=torch.bfloat16, device="cuda")
    us_gn = _profiled_us(vm, torch, vm._lib.VM_K_ROWS,
                         lambda: vm.gated_rms_norm_(yb, o, z, gw, eps=EPS), n=5)
    # the layer's form: the chunked recurrence with the gated norm in its output kernel
    us_chk_gn = _profiled_us(vm, torch, vm._lib.VM_K_DELTANET,
                             lambda: vm.deltanet_sequence_chunked_gated_norm_(
                                 {"Y": yb, "Sp": S}, z, gw, p["Q"], p["K"], p["V"], p["Beta"],
                                 p["Gate"], S, eps=EPS, workspace=ws), n=5)
    # prep: conv rows read (bf16), fp32 q, k, v written, ab read, gates written;
    # gated norm: fp32 o and bf16 z read, bf16 y written
    prep_bytes = 2.0 * T * n + 4.0 * T * n + 2.0 * T * 2 * Hv + 8.0 * T * Hv
    # conv + prep: projection rows read (bf16), fp32 q, k, v written, ab, gates, ring
    cp_bytes = 2.0 * T * n + 4.0 * T * n + 2.0 * T * 2 * Hv + 8.0 * T * Hv + 2.0 * 2 * K * n
    gn_bytes = (4.0 + 2.0 + 2.0) * T * Hv * Dv
    res["prefill_B1_T4096"] = {
        "conv_sequence_us": us_conv,
        "conv_sequence_gbs": 2.0 * (2 * T * n + K * n) / (us_conv * 1e-6) / 1e9,
        "sequence_ms": us_seq * 1e-3,
        "sequence_tokens_per_s": T / (us_seq * 1e-6),
        "sequence_us_per_token": us_seq / T,
        "chunked_ms": us_chk * 1e-3,
        "chunked_tokens_per_s": T / (us_chk * 1e-6),
        "chunked_gated_norm_ms": us_chk_gn * 1e-3,
        "prep_us": us_prep,
        "prep_gbs": prep_bytes / (us_prep * 1e-6) / 1e9,
        "conv_prep_us": us_cp,
        "conv_prep_gbs": cp_bytes / (us_cp * 1e-6) / 1e9,
        "gated_norm_us": us_gn,
        "gated_norm_gbs": gn_bytes / (us_gn * 1e-6) / 1e9,
    }
    return res


def cpu_info():
    """CPU model, sockets x physical cores per socket, and logical CPUs of this host."""
    import subprocess
    info = {"cpu_model": None, "physical_cores": None, "logical_cpus": os.cpu_count()}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = {}
        for line in out.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                kv[k.strip()] = v.strip()
        info["cpu_model"] = kv.get("Model name")
        cps, sock = kv.get("Core(s) per socket"), kv.get("Socket(s)")
        if cps and sock and cps.isdigit() and sock.isdigit():
            info["physical_cores"] = int(cps) * int(sock)
    except (OSError, subprocess.SubprocessError):
        pass
    return info


def _median_time(fn, min_runs, max_runs, budget_s):
    """Median wall time of fn() over at least min_runs runs (at most max_runs, or
    fewer once budget_s is spent after min_runs)."""
    times = []
    while True:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if len(times) >= max_runs or (len(times) >= min_runs and sum(times) > budget_s):
            break
    return float(np.median(times)), len(times)


def _dev_normal(vm, torch, shape, seed, scale=1.0):
    t = torch.empty(shape, dtype=torch.bfloat16, device="cuda")
    vm.fill_normal_(t, seed, scale=scale)
    return t


def cpu_baseline(vm, torch):
    """The fp32 C oracle (oracle/, test infrastructure) timed on this host's cores
    for every BASELINE config, on the same seeded inputs as the GPU legs (generated
    on the device by the same generator and copied to host memory):
      config 1, 3: one decode step (median of repeated steps);
      config 4: 8 consecutive decode steps at 131072.. (per-step median);
      config 2, 5: the whole prefill problem, median of 3 runs (7 for config 2).
    Decode figures are GB/s of the same algorithmic bytes as the GPU legs, prefill
    figures TFLOP/s of the same algorithmic FLOP."""
    import oracle
    threads = oracle.threads_env()
    res = {}

    def hb(t):
        return t.view(torch.int16).cpu().numpy().view(np.uint16)

    # ---- config 2: the headline (whole problem)
    T = 4096
    qkv = hb(_dev_normal(vm, torch, (1, T, S, D), 203))
    qw, kw = hb(_dev_normal(vm, torch, (D,), 201, 0.05)), hb(_dev_normal(vm, torch, (D,), 202, 0.05))
    zero = np.zeros((1, HK, T, D), np.uint16)
    c, s = oracle.rope_tables(HALF, T, THETA)
    one = np.zeros(1, np.int32)
    dt, n = _median_time(lambda: oracle.gated_prefill(
        qkv, zero, zero, one, np.full(1, T, np.int32), qw, kw, c, s, Hq=HQ, Hk=HK, eps=EPS,
        w_offset=1.0, nthreads=threads), 3, 7, 12.0)
    fl = prefill_flops(T)
    res["config2"] = {"tflops": fl / dt / 1e12, "s_per_step": dt, "runs": n,
                      "sample": f"the whole config2 problem ({fl / 1e9:.1f} GFLOP)"}
    del qkv, zero

    # ---- config 1: B=1 at 512 (bench_decode1's draws)
    ctx, L = 512, 512
    qw1, kw1 = hb(_dev_normal(vm, torch, (D,), 101, 0.05)), hb(_dev_normal(vm, torch, (D,), 102, 0.05))
    kc, vc = hb(_dev_normal(vm, torch, (1, HK, ctx, D), 103)), hb(_dev_normal(vm, torch, (1, HK, ctx, D), 104))
    q1 = hb(_dev_normal(vm, torch, (1, S, D), 105))
    c, s = oracle.rope_tables(HALF, ctx, THETA)
    dt, n = _median_time(lambda: oracle.gated_decode(
        q1, kc, vc, np.array([L], np.int32), qw1, kw1, c, s, Hq=HQ, Hk=HK, eps=EPS, w_offset=1.0,
        nthreads=threads), 20, 2000, 1.0)
    nb = decode_bytes([L])
    res["config1"] = {"gbs": nb / dt / 1e9, "us_per_step": 1e6 * dt, "runs": n,
                      "sample": "one decode step, B=1 at attended length 512"}

    # ---- config 3: B=32 ragged (bench_decode3's draws), one whole step
    B, ctx = 32, 32768
    lengths = np.random.default_rng(3).integers(1024, 32769, size=B).astype(np.int32)
    qw3, kw3 = hb(_dev_normal(vm, torch, (D,), 301, 0.05)), hb(_dev_normal(vm, torch, (D,), 302, 0.05))
    kc = hb(_dev_normal(vm, torch, (B, HK, ctx, D), 303))
    vc = hb(_dev_normal(vm, torch, (B, HK, ctx, D), 304))
    q3 = hb(_dev_normal(vm, torch, (B, S, D), 305))
    torch.cuda.empty_cache()
    c, s = oracle.rope_tables(HALF, ctx, THETA)
    dt, n = _median_time(lambda: oracle.gated_decode(
        q3, kc, vc, lengths, qw3, kw3, c, s, Hq=HQ, Hk=HK, eps=EPS, w_offset=1.0,
        nthreads=threads), 3, 5, 8.0)
    nb = decode_bytes(lengths)
    res["config3"] = {"gbs": nb / dt / 1e9, "ms_per_step": 1e3 * dt, "runs": n,
                      "sample": f"one whole decode step, B=32, sum of lengths {int(lengths.sum())}"}
    del kc, vc

    # ---- config 4: B=1 at 131072.. (bench_decode4's draws), 8 consecutive steps
    p0, ctx = 131072, 131072 + 256
    qw4, kw4 = hb(_dev_normal(vm, torch, (D,), 401, 0.05)), hb(_dev_normal(vm, torch, (D,), 402, 0.05))
    kc = hb(_dev_normal(vm, torch, (1, HK, ctx, D), 403))
    vc = hb(_dev_normal(vm, torch, (1, HK, ctx, D), 404))
    q4 = hb(_dev_normal(vm, torch, (1, S, D), 405))
    torch.cuda.empty_cache()
    c, s = oracle.rope_tables(HALF, ctx, THETA)
    times = []
    for i in range(8):
        t0 = time.perf_counter()
        oracle.gated_decode(q4, kc, vc, np.array([p0 + i], np.int32), qw4, kw4, c, s, Hq=HQ,
                            Hk=HK, eps=EPS, w_offset=1.0, nthreads=threads)
        times.append(time.perf_counter() - t0)
    dt = float(np.median(times))
    nb = decode_bytes([p0 + 4])
    res["config4"] = {"gbs": nb / dt / 1e9, "ms_per_step": 1e3 * dt, "runs": 8,
                      "sample": "8 consecutive decode steps at attended lengths 131072..131079 "
                                "(median per step)"}
    del kc, vc

    # ---- config 5: ragged chunked prefill (bench_prefill5's draws), whole problem
    seed = 5
    rng = np.random.default_rng(seed)
    qlen = rng.permutation(np.array([512, 1024, 2048, 2048], np.int32)).astype(np.int32)
    prior = rng.integers(8192, 32769, size=4).astype(np.int32)
    B, T = 4, int(qlen.max())
    ctx = int((prior + qlen).max())
    qw5, kw5 = hb(_dev_normal(vm, torch, (D,), seed * 100 + 1, 0.05)), hb(_dev_normal(vm, torch, (D,), seed * 100 + 2, 0.05))
    kc = hb(_dev_normal(vm, torch, (B, HK, ctx, D), seed * 100 + 3))
    vc = hb(_dev_normal(vm, torch, (B, HK, ctx, D), seed * 100 + 4))
    q5 = hb(_dev_normal(vm, torch, (B, T, S, D), seed * 100 + 5))
    torch.cuda.empty_cache()
    c, s = oracle.rope_tables(HALF, ctx, THETA)
    dt, n = _median_time(lambda: oracle.gated_prefill(
        q5, kc, vc, prior, qlen, qw5, kw5, c, s, Hq=HQ, Hk=HK, eps=EPS, w_offset=1.0,
        nthreads=threads), 3, 3, 30.0)
    cc, pp = qlen.astype(np.float64), prior.astype(np.float64)
    fl = float(4 * D * HQ * np.sum(cc * pp + cc * (cc + 1) / 2))
    res["config5"] = {"tflops": fl / dt / 1e12, "s_per_step": dt, "runs": n,
                      "sample": f"the whole config5 problem ({fl / 1e12:.2f} TFLOP)"}
    del kc, vc

    # ---- the Wo projection of the config-2 layer (fp32 GEMM, 4096 x 4096 -> 2560)
    o = hb(_dev_normal(vm, torch, (4096, HQ * D), 2010))
    Wo = hb(_dev_normal(vm, torch, (DM, HQ * D), 2007, (HQ * D) ** -0.5))
    dt, n = _median_time(lambda: oracle.linear(o, Wo, nthreads=threads), 3, 3, 10.0)
    fl = 2.0 * 4096 * HQ * D * DM
    res["layer_wo_gemm"] = {"tflops": fl / dt / 1e12, "s_per_step": dt, "runs": n,
                            "sample": f"the config-2 layer's Wo projection ({fl / 1e9:.1f} GFLOP)"}

    # ---- the DeltaNet kernels (Qwen3.5-4B shape): the fused decode step at B = 32
    # (the oracle is one thread per call: cores 1 for this entry) and the prefill
    # recurrence over a 512-token sample at B = 1 (OpenMP over the 32 value heads)
    Dk = Dv = 128
    Hk, Hv, B = 16, 32, 32
    rng = np.random.default_rng(21)
    qz = hb(_dev_normal(vm, torch, (B, 2 * Hk * Dk + 2 * Hv * Dv), 2101))
    ab = hb(_dev_normal(vm, torch, (B, 2 * Hv), 2102))
    n = 2 * Hk * Dk + Hv * Dv
    S0 = (rng.standard_normal((B, Hv, Dv, Dk)) * 0.05).astype(np.float32)
    a_log = rng.standard_normal(Hv).astype(np.float32) * 0.5
    dtb = rng.standard_normal(Hv).astype(np.float32) * 0.5
    gw = hb(_dev_normal(vm, torch, (Dv,), 2103))
    hk = Hk * Dk
    args = (qz[:, :hk].reshape(B, Hk, Dk), qz[:, hk:2 * hk].reshape(B, Hk, Dk),
            qz[:, 2 * hk:n].reshape(B, Hv, Dv), ab[:, :Hv], ab[:, Hv:],
            qz[:, n:].reshape(B, Hv, Dv), a_log, dtb, gw, S0)
    dt, nr = _median_time(lambda: oracle.fused_deltanet_decode(*args, eps=EPS), 3, 7, 5.0)
    nb = B * Hv * (2.0 * Dk * Dv * 4 + 3 * Dv * 2 + 4) + B * 2 * hk * 2
    res["deltanet_decode_B32"] = {"gbs": nb / dt / 1e9, "us_per_step": 1e6 * dt, "runs": nr,
                                  "cores": 1,
                                  "sample": "one fused DeltaNet decode step, B=32, Hv=32, "
                                            "Dk=Dv=128 (single-threaded oracle)"}
    T = 512
    cv = hb(_dev_normal(vm, torch, (1, T, n), 2104))
    abT = hb(_dev_normal(vm, torch, (1, T, 2 * Hv), 2105))
    p = oracle.deltanet_prep(cv, abT, a_log, dtb, Dk=Dk, Dv=Dv, Hk=Hk, Hv=Hv)
    Sz = np.zeros((1, Hv, Dv, Dk), np.float32)
    dt, nr = _median_time(lambda: oracle.deltanet_sequence(p["q"], p["k"], p["v"], p["beta"],
                                                           p["gate"], Sz), 1, 3, 10.0)
    res["deltanet_sequence_B1"] = {"tokens_per_s": T / dt, "us_per_token": 1e6 * dt / T,
                                   "runs": nr,
                                   "sample": f"the prefill recurrence over {T} tokens, B=1 "
                                             f"({threads} OpenMP threads over value heads)"}

    info = cpu_info()
    c2 = res["config2"]
    return {"value": c2["tflops"], "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"{c2['sample']}: median of {c2['runs']} runs = {c2['s_per_step']:.3f} s with "
                      f"{threads} OpenMP threads of the fp32 C oracle; every config in 'configs'",
            "cpu_model": info["cpu_model"], "physical_cores": info["physical_cores"],
            "logical_cpus": info["logical_cpus"], "threads": threads, "configs": res}


def config4_packet_capture_off():
    """Config 4 measured in a child process whose HIP runtime dispatches graph
    kernels without packet capture (its figures, or None if the child failed)."""
    import subprocess
    env = dict(os.environ)
    env[PACKET_CAPTURE_VAR] = "0"
    log(f"[bench] decode config4 with {PACKET_CAPTURE_VAR}=0 (child process)")
    try:
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--config4-only"], env=env,
                           stdout=subprocess.PIPE, timeout=600, check=False, text=True)
    except subprocess.TimeoutExpired:
        log("[bench] config-4 child timed out")
        return None
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
    if r.returncode != 0 or not lines:
        log(f"[bench] config-4 child failed (exit {r.returncode})")
        return None
    return json.loads(lines[-1])["config4"]


def bench_operators(vm, torch, reps=20, seed=15):
    """The operators at head shapes other than Qwen3.5's: attention! on the MFMA
    kernel at D = 128 and 64 and on the generic kernel at Dk != Dv, and the
    generic decode_attention! and fused_deltanet_decode! (seeded N(0,1)
    inputs, one event pair around `reps` launches each)."""
    import numpy as np
    g = torch.Generator(device="cuda").manual_seed(seed)

    def rnd(*shape):
        return torch.randn(*shape, device="cuda", generator=g).to(torch.bfloat16)

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    res = {}
    B, H, Hk, L = 1, 16, 4, 4096
    for Dk, Dv, path in ((128, 128, "mfma"), (64, 64, "mfma"), (128, 64, "generic")):
        Q, K, V = rnd(B, H, L, Dk), rnd(B, Hk, L, Dk), rnd(B, Hk, L, Dv)
        O = torch.empty(B, H, L, Dv, dtype=torch.bfloat16, device="cuda")
        ms = timed(lambda: vm.attention_({"O": O}, Q, K, V, causal=True))
        fl = 2 * (Dk + Dv) * H * L * (L + 1) / 2
        res[f"attention_causal_T4096_Dk{Dk}_Dv{Dv}"] = {
            "kernel": path, "us": 1e3 * ms, "tflops": fl / (ms * 1e-3) / 1e12,
            "frac_of_bf16_peak": fl / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS}
    rng = np.random.default_rng(seed)
    B, H, Hk, D, ctx = 32, 16, 4, 128, 32768
    lens = torch.from_numpy(rng.integers(1024, ctx + 1, B).astype(np.int32)).cuda()
    Q, K, V = rnd(B, H, D), rnd(B, Hk, ctx, D), rnd(B, Hk, ctx, D)
    O = torch.empty(B, H, D, dtype=torch.bfloat16, device="cuda")
    sc = torch.empty(vm.decode_scratch_bytes(Q, K, V), dtype=torch.uint8, device="cuda")
    ms = timed(lambda: vm.decode_attention_({"O": O}, Q, K, V, lengths=lens, scratch=sc))
    nb = int(lens.sum()) * Hk * D * 2 * 2
    res["decode_attention_B32_D128"] = {"kernel": "generic", "us": 1e3 * ms,
                                        "gbs": nb / (ms * 1e-3) / 1e9,
                                        "frac_of_hbm_peak": nb / (ms * 1e-3) / 1e9 / 8000.0}
    del K, V
    B, Hk, Hv, Dd = 32, 16, 32, 64
    q, k, v, z = rnd(B, Hk, Dd), rnd(B, Hk, Dd), rnd(B, Hv, Dd), rnd(B, Hv, Dd)
    ab = rnd(B, 2 * Hv)
    zero = torch.zeros(Hv, device="cuda")
    S = torch.randn(B, Hv, Dd, Dd, device="cuda", generator=g) * 0.05
    nw = rnd(Dd)
    ms = timed(lambda: vm.fused_deltanet_decode(q, k, v, ab[:, :Hv], ab[:, Hv:], z, zero, zero,
                                                nw, S, Sp=S))
    nb = B * Hv * Dd * Dd * 4 * 2
    res["fused_deltanet_decode_B32_D64"] = {"kernel": "generic", "us": 1e3 * ms,
                                            "gbs": nb / (ms * 1e-3) / 1e9,
                                            "frac_of_hbm_peak": nb / (ms * 1e-3) / 1e9 / 8000.0}
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # untimed steps before the timed ones: --warmup steps, then a time-sized
    # clock-settle phase (settle_clocks) whose length the JSON line reports
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-config5", action="store_true", help="skip the config-5 prefill leg")
    ap.add_argument("--no-layer", action="store_true", help="skip the whole-layer leg")
    ap.add_argument("--no-step", action="store_true", help="skip the whole-decode-step leg")
    ap.add_argument("--no-deltanet", action="store_true", help="skip the DeltaNet kernel leg")
    ap.add_argument("--no-operators", action="store_true",
                    help="skip the leg of the operators at other head shapes")
    ap.add_argument("--no-model-prefill", action="store_true",
                    help="skip the whole-model prefill leg")
    ap.add_argument("--no-settle", action="store_true",
                    help="skip the clock-settle phase (counter-collection runs)")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--calib-copy", action="store_true",
                    help="first run one 1 GiB device-to-device copy (a known-traffic kernel "
                         "for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--config4-only", action="store_true",
                    help="run only the config-4 replay leg (twice, the first as warm-up) and "
                         "print its figures as one JSON line")
    ap.add_argument("--no-config4-env", action="store_true",
                    help="skip the config-4 measurement with the runtime's packet capture off")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the multi-GPU sharding is a design note, not a measured path", file=sys.stderr)
        sys.exit(2)

    d4_env = None
    if not args.config4_only and not args.no_decode and not args.no_config4_env:
        # before this process touches the GPU: a child with the variable set
        d4_env = config4_packet_capture_off()

    import torch
    import __graft_entry__
    vm = __graft_entry__.load_package()
    torch.cuda.set_device(0)
    if args.config4_only:
        bench_decode4(vm, torch)
        print(json.dumps({"config4": bench_decode4(vm, torch)}), flush=True)
        return
    if args.calib_copy:
        src = torch.ones(1 << 29, dtype=torch.int16, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log("[bench] calibration copy: 1 GiB read + 1 GiB written")
        del src, dst

    pf = None
    if not args.no_prefill:
        log("[bench] prefill config2 T=4096")
        pf = bench_prefill(vm, torch, args.steps, args.warmup, settle=not args.no_settle)
        log(f"[bench] settle: {pf['settle']}")
        log(f"[bench] prefill: {pf['ms_per_step']:.3f} ms/step, {pf['tflops']:.1f} TFLOP/s, "
            f"attn kernel {pf['attn_kernel_ms'] * 1e3:.1f} us (per-dispatch events), "
            f"K/V append + V^T staging {pf['append_vt_kernel_ms']:.4f} ms")
    pf_shift = None
    if not args.no_prefill:
        # the exact-softmax path the kernel takes when the norm weights allow
        # logits past the static bound: one K-norm weight of 4 (kw[0] = 4)
        log("[bench] prefill config2 with kw[0] = 4 (online-max softmax)")
        r = bench_prefill(vm, torch, max(20, args.steps // 5), 5, settle=False, kw0=4.0)
        pf_shift = {"kw0": 4.0, "softmax": "online row max, moved lazily (by > 8 in log2 units), "
                                           "O and l rescaled when it moves",
                    "ms_per_step": r["ms_per_step"], "tflops": r["tflops"],
                    "attn_kernel_ms": r["attn_kernel_ms"],
                    "attn_kernel_tflops": r["flops"] / (r["attn_kernel_ms"] * 1e-3) / 1e12,
                    "attn_kernel_frac_of_bf16_peak":
                        r["flops"] / (r["attn_kernel_ms"] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                    "vs_static_kernel": r["attn_kernel_ms"] / pf["attn_kernel_ms"] if pf else None}
        log(f"[bench] prefill kw[0]=4: attn kernel {r['attn_kernel_ms'] * 1e3:.1f} us = "
            f"{pf_shift['attn_kernel_tflops']:.0f} TFLOP/s ({pf_shift['vs_static_kernel']:.2f}x the "
            f"static path)")
    pf5 = None
    if not args.no_prefill and not args.no_config5:
        log("[bench] prefill config5 (ragged chunked, B=4)")
        pf5 = bench_prefill5(vm, torch, max(10, args.steps // 15), max(3, args.warmup // 30))
        log(f"[bench] prefill5: {pf5['ms_per_step']:.3f} ms/step, {pf5['tflops']:.1f} TFLOP/s, "
            f"attn kernel {pf5['attn_kernel_ms']:.3f} ms = {pf5['attn_kernel_tflops']:.1f} TFLOP/s; "
            f"V^T kept between chunks: {pf5['ms_per_step_staged']:.3f} ms/step")
    decode = None
    if not args.no_decode:
        log("[bench] decode config3 B=32")
        d3 = bench_decode3(vm, torch, max(10, args.steps // 2), 3)
        log(f"[bench] decode3: {d3['ms_per_step']:.3f} ms/step {d3['gbs']:.0f} GB/s "
            f"(split kernel {d3['split_kernel_gbs']:.0f} GB/s)")
        log("[bench] decode config3 with kw[0] = 4 (running-max softmax)")
        d3s = bench_decode3(vm, torch, max(10, args.steps // 2), 3, kw0=4.0)
        d3s["kw0"] = 4.0
        d3s["softmax"] = "running max, rescaled lazily (only when it grows by > 8 in log2 units)"
        log(f"[bench] decode3 kw[0]=4: {d3s['ms_per_step']:.3f} ms/step {d3s['gbs']:.0f} GB/s")
        log("[bench] decode config4 B=1 131072, 256 graph replays")
        d4 = bench_decode4(vm, torch)
        log(f"[bench] decode4: {d4['ms_per_replay'] * 1e3:.1f} us/replay {d4['gbs']:.0f} GB/s "
            f"(split kernel {d4['split_kernel_gbs']:.0f} GB/s)")
        if d4_env is not None:
            d4_env["frac_of_hbm_peak"] = d4_env["gbs"] / PEAK_HBM_GBS
            d4["packet_capture_off"] = d4_env
            log(f"[bench] decode4 with {PACKET_CAPTURE_VAR}=0 (child process): "
                f"{d4_env['ms_per_replay'] * 1e3:.1f} us/replay {d4_env['gbs']:.0f} GB/s")
        log("[bench] decode config1 B=1 at 512")
        d1 = bench_decode1(vm, torch, max(20, args.steps // 3), 10)
        log(f"[bench] decode1: {d1['us_per_step']:.1f} us/step")
        for d in (d3, d3s, d4, d1):
            d["frac_of_hbm_peak"] = d["gbs"] / PEAK_HBM_GBS
        decode = {"config3": d3, "config3_running_max": d3s, "config4": d4, "config1": d1,
                  "peak_GBs": PEAK_HBM_GBS}
    layer = None
    if not args.no_layer:
        log("[bench] layers (projections + attention), hidden 2560")
        layer = bench_layer(vm, torch)
        lp, ld = layer["prefill_config2"], layer["decode_config3"]
        log(f"[bench] prefill layer: {lp['ms_per_layer']:.3f} ms, qkv GEMM {lp['qkv_gemm_tflops']:.0f} "
            f"TFLOP/s, Wo GEMM {lp['wo_gemm_tflops']:.0f} TFLOP/s")
        log(f"[bench] decode layer B=32: {ld['ms_per_layer_step']:.3f} ms, qkv GEMV "
            f"{ld['qkv_gemv_gbs']:.0f} GB/s, Wo GEMV {ld['wo_gemv_gbs']:.0f} GB/s")
    ops_other = None
    if not args.no_operators:
        log("[bench] operators at other head shapes (D = 128 / 64, Dk != Dv)")
        ops_other = bench_operators(vm, torch)
        for k, v in ops_other.items():
            fig = f"{v['tflops']:.1f} TFLOP/s" if "tflops" in v else f"{v['gbs']:.0f} GB/s"
            log(f"[bench] {k} ({v['kernel']}): {v['us']:.1f} us = {fig}")
    dnet = None
    if not args.no_deltanet:
        log("[bench] Gated DeltaNet kernels (Qwen3.5-4B shape)")
        dnet = bench_deltanet(vm, torch)
        f1, f32_, cv = dnet["fused_decode_B1"], dnet["fused_decode_B32"], dnet["conv_decode_B32"]
        pp = dnet["prefill_B1_T4096"]
        log(f"[bench] deltanet: fused decode B=1 {f1['us']:.1f} us, B=32 {f32_['us']:.1f} us = "
            f"{f32_['gbs']:.0f} GB/s; conv decode B=32 {cv['us']:.1f} us = {cv['gbs']:.0f} GB/s; "
            f"prefill T=4096: conv {pp['conv_sequence_us']:.1f} us, recurrence "
            f"{pp['sequence_ms']:.2f} ms sequential ({pp['sequence_us_per_token']:.2f} us/token), "
            f"{pp['chunked_ms']:.3f} ms chunked ({pp['chunked_gated_norm_ms']:.3f} ms with the gated "
            f"norm fused, the layer's form); prep {pp['prep_us']:.1f} us = {pp['prep_gbs']:.0f} "
            f"GB/s, conv + prep in one pass {pp['conv_prep_us']:.1f} us = "
            f"{pp['conv_prep_gbs']:.0f} GB/s (the layer's form), gated norm "
            f"{pp['gated_norm_us']:.1f} us = {pp['gated_norm_gbs']:.0f} GB/s")
    step = None
    if not args.no_step:
        log("[bench] whole decode step, Qwen3.5-4B shape (24 DeltaNet + 8 attention), B=32")
        step = bench_step(vm, torch)
        log(f"[bench] step: {step['ms_per_step']:.3f} ms/step, {step['tokens_per_s']:.0f} tok/s, "
            f"{step['gbs']:.0f} GB/s; lm head alone B=1 {step['lm_head_B1']['gbs']:.0f} GB/s, "
            f"B=32 {step['lm_head_B32']['gbs']:.0f} GB/s")
    pmodel = None
    if not args.no_model_prefill:
        log("[bench] whole-model prefill, Qwen3.5-4B shape, B=1 T=4096")
        pmodel = bench_prefill_model(vm, torch)
        log(f"[bench] model prefill: {pmodel['ms']:.2f} ms = {pmodel['tokens_per_s']:.0f} tokens/s, "
            f"{pmodel['tflops']:.0f} TFLOP/s (projections + attention)")
    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline (oracle), configs 1-5")
        cpu = cpu_baseline(vm, torch)
        for k, v in sorted(cpu["configs"].items()):
            fig = (f"{v['tflops']:.4f} TFLOP/s" if "tflops" in v else
                   f"{v['gbs']:.1f} GB/s" if "gbs" in v else f"{v['tokens_per_s']:.0f} tokens/s")
            log(f"[bench] cpu {k}: {fig} ({v['sample']}, {v['runs']} runs)")

    if pf is None:
        print(json.dumps({"decode": decode, "layer": layer, "decode_step": step, "deltanet": dnet,
                          "operators_other_shapes": ops_other,
                          "prefill_model": pmodel, "cpu_baseline": cpu}), flush=True)
        return
    achieved = pf["flops"] / (pf["attn_kernel_ms"] * 1e-3) / 1e12
    line = {
        "metric": "prefill attn TFLOP/s + decode HBM GB/s (% of MI355X peak) vs host-CPU baseline",
        "value": round(pf["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(pf["ms_per_step"], 4),
        "settle_ms": pf["settle"]["settle_ms"],
        "settle_steps": pf["settle"]["settle_steps"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 q/k/v/gate, norm weights 1+N(0,0.05))",
        "config": {"workload": "config2: causal gated-attention prefill B=1 T=4096 Hq=16 Hkv=4 "
                               "D=256 rope64 theta=1e7 (K/V append + fused attention)",
                   "global_batch": 1, "seq_len": 4096, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": profiled_traffic(), "kernel": "prefill_fused_kernel<CAUSAL>",
                     "kernel_ms": round(pf["attn_kernel_ms"], 5),
                     "timing": "kernel_ms: mean of the HIP events recorded around each "
                               "dispatch of the attention kernel in the timed steps, on its "
                               "launch stream",
                     "flop_per_launch": pf["flops"]},
        "cpu_baseline": cpu,
        "prefill_config2_online_max": pf_shift,
        "prefill_config5": pf5,
        "decode": decode,
        "layer": layer,
        "decode_step": step,
        "prefill_model": pmodel,
        "deltanet": dnet,
        "operators_other_shapes": ops_other,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
