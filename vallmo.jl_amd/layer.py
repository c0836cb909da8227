"""Attention-layer verbs and the decode clock — src/llm/qwen35.jl and generate.jl.

The reference's layer verbs run hidden state -> hidden state: the qkv
projection, the gated attention block, the Wo projection (linear!, hipBLASLt
here as cuBLASLt there):

    decode_(h, l, m, gen, xn)            decode!(h, l::AttnLayer, m, gen, xn),
                                         qwen35.jl:187-208
    forward(l, m, xn, T, B; offset)      forward(l::AttnLayer, m, xn, T, B; offset),
                                         qwen35.jl:292-318

and their attention parts, from the packed projection ``qkv`` to the Wo input,
are the fused gated-attention kernels:

    gated_attn_decode_(O, l, m, gen, qkv)        qwen35.jl:195-205
    gated_attn_prefill(l, m, qkv, T, B; offset)  qwen35.jl:293-317 (returns the
                                                 (Dh*Hq, T*B) Wo input)

Packed projection slots per token (qwen35.jl:189-192): [q1 g1 q2 g2 .. qHq gHq |
k1..kHkv | v1..vHkv], each Dh wide. The KV cache layout (Dh, Ctx, Hkv, B) of
qwen35.jl:138-139 is kept: it is the on-device format shared by prefill and decode.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import ops
from ._lib import ArgumentError, BoundsError, DimensionMismatch, call
from .sizes import sizes


@dataclass(frozen=True)
class AttnConfig:
    """The attention facts of a Qwen3.5 text config (qwen35.jl:82-96); D is the
    hidden size (the projections' other side)."""
    D: int = 2560
    Hq: int = 16
    Hkv: int = 4
    Dh: int = 256
    rot_half: int = 32          # head_dim * partial_rotary_factor / 2
    theta: float = 1.0e7
    eps: float = 1.0e-6
    Ctx: int = 4096
    B: int = 1


@dataclass
class AttnLayer:
    """qwen35.jl:129-142: norm weights, the layer's own KV cache, and the two
    projections (K-major, the checkpoint's orientation; None for callers of the
    attention part only)."""
    qw: torch.Tensor            # (Dh,) bf16, applied as (w + 1)
    kw: torch.Tensor            # (Dh,) bf16
    K_cache: torch.Tensor       # (Dh, Ctx, Hkv, B) -> torch (B, Hkv, Ctx, Dh) bf16
    V_cache: torch.Tensor
    Wqkv: torch.Tensor | None = None   # (D, Dh*(2Hq+2Hkv)) -> torch (Dh*(2Hq+2Hkv), D)
    Wo: torch.Tensor | None = None     # (Dh*Hq, D) -> torch (D, Dh*Hq)
    # the decoder-layer parts around the block (qwen35.jl:133-141): the two
    # RMSNorm weights (applied as w + 1) and the MLP (mlp_parts, qwen35.jl:124-127)
    norm1: torch.Tensor | None = None  # (D,)
    norm2: torch.Tensor | None = None  # (D,)
    Wgu: torch.Tensor | None = None    # (D, 2I) [gate | up] -> torch (2I, D)
    Wd: torch.Tensor | None = None     # (I, D) -> torch (D, I)


def attn_layer(cfg: AttnConfig, qw: torch.Tensor, kw: torch.Tensor, Wqkv=None,
               Wo=None) -> AttnLayer:
    """Allocate a layer with zeroed caches (qwen35.jl:138-139)."""
    shape = (cfg.B, cfg.Hkv, cfg.Ctx, cfg.Dh)
    return AttnLayer(qw=qw, kw=kw,
                     K_cache=torch.zeros(shape, dtype=torch.bfloat16, device="cuda"),
                     V_cache=torch.zeros(shape, dtype=torch.bfloat16, device="cuda"),
                     Wqkv=Wqkv, Wo=Wo)


class AttnModel:
    """The model-level state the attention verbs read: cfg, RoPE tables and the
    decode space (the reference's Arena, qwen35.jl:110), allocated once so a
    captured step replays the same addresses: the split-KV scratch, the decode
    projections' workspace, and the decode step's qkv and attention-output
    buffers (the layer frame's temporaries, qwen35.jl:193). Prefill and forward
    use a workspace of their own that grows freely: a graph never records it."""


    def __init__(self, cfg: AttnConfig, *, n_splits: int = 0):
        self.cfg = cfg
        self.rope = ops.rope_tables(cfg)
        self.n_splits = int(n_splits)
        nbytes = int(ops._lib.load().vm_decode_scratch_bytes(
            cfg.B, cfg.Hq, cfg.Hkv, cfg.Dh, cfg.Ctx, self.n_splits))
        self.space = torch.empty(max(nbytes, 16), dtype=torch.uint8, device="cuda")
        self.prefill_space = None
        self.lin_space = None
        self.dec_space = None
        self.dec_frozen = False   # set once a graph may have recorded dec_space
        self.qkv = None
        self.attn_out = None

    def linear_workspace(self, need: int = 0) -> torch.Tensor:
        """The eager (prefill, forward) projections' workspace, grown to `need`
        bytes. Never passed to a captured step: growing it replaces the tensor."""
        if self.lin_space is None or self.lin_space.numel() < need:
            self.lin_space = torch.empty(max(need, 256), dtype=torch.uint8, device="cuda")
        return self.lin_space

    def decode_workspace(self, need: int = 0) -> torch.Tensor:
        """The decode step's projections' workspace: sized by the first (eager)
        calls, then fixed, because a captured step replays its address. Once
        ``dec_frozen`` is set (a graph may hold the buffer) a larger need raises
        instead of replacing it; so does one inside a stream capture."""
        if self.dec_space is None or self.dec_space.numel() < need:
            if self.dec_frozen or torch.cuda.is_current_stream_capturing():
                have = 0 if self.dec_space is None else self.dec_space.numel()
                raise ArgumentError(
                    f"the decode workspace holds {have} bytes and a captured step may use it; "
                    f"this call needs {need}: size it eagerly before capturing")
            self.dec_space = torch.empty(max(need, 256), dtype=torch.uint8, device="cuda")
        return self.dec_space

    def decode_buffers(self):
        """(qkv (B, 2Hq+2Hkv, Dh), O (B, Hq, Dh)) bf16, allocated on first use."""
        if self.qkv is None:
            c = self.cfg
            self.qkv = torch.empty((c.B, 2 * c.Hq + 2 * c.Hkv, c.Dh), dtype=torch.bfloat16,
                                   device="cuda")
            self.attn_out = torch.empty((c.B, c.Hq, c.Dh), dtype=torch.bfloat16, device="cuda")
        return self.qkv, self.attn_out

    def prefill_workspace(self, B: int, ctx: int) -> torch.Tensor:
        """The prefill workspace (V staged transposed), grown on demand and kept,
        so repeated prefills reuse one buffer."""
        need = int(ops._lib.load().vm_prefill_scratch_bytes(B, self.cfg.Hkv, self.cfg.Dh, ctx))
        if self.prefill_space is None or self.prefill_space.numel() < need:
            self.prefill_space = torch.empty(max(need, 256), dtype=torch.uint8, device="cuda")
        return self.prefill_space


class StagedV:
    """One attention layer's V^T workspace kept between the chunks of a chunk-by-
    chunk prefill (vm_gated_attn_prefill_staged): ``vt`` holds the V^T tiles of
    the first ``rows[b]`` cache rows of each sequence, so a chunk stages only its
    own rows (and rows appended since, e.g. by decode steps) instead of the
    whole prior. ``reset_(b)`` (all sequences when b is None) forgets what is
    held: call it for a new sequence in slot b and after writing V cache rows
    below ``rows[b]`` by any other means. It belongs to one layer: used with
    another layer's cache, it forgets everything first."""

    def __init__(self, cfg: AttnConfig, B: int, ctx: int | None = None):
        ctx = cfg.Ctx if ctx is None else int(ctx)
        need = int(ops._lib.load().vm_prefill_scratch_bytes(B, cfg.Hkv, cfg.Dh, ctx))
        self.B, self.ctx = B, ctx
        self.vt = torch.empty(max(need, 256), dtype=torch.uint8, device="cuda")
        # [0, B): rows held per sequence; [B, 2B): the library's arrival counters
        self.state = torch.zeros(2 * B, dtype=torch.int32, device="cuda")
        self.rows = self.state[:B]
        self.cache = None  # data_ptr of the V cache whose rows vt holds

    def reset_(self, b: int | None = None):
        if b is None:
            self.rows.zero_()
        else:
            self.rows[b] = 0
        return self


class Generation:
    """The engine's device state (generate.jl:54-72). positions[b]: the 1-based
    column of the current token = rope column = cache column = attended length
    (the clock); step: the next 1-based row of tokens_out to write; result: the
    last generated token per sequence (1-based); tokens_out: the harvested
    tokens, (max_new, B) column-major (torch (B, max_new)); col_offsets[b] =
    b * max_new. All on the device, so a captured step needs no host writes."""

    def __init__(self, B: int, max_new: int = 1):
        if B < 0 or max_new < 0:
            raise ArgumentError(f"Generation(B = {B}, max_new = {max_new})")
        dev = "cuda"
        self.B, self.max_new = B, max_new
        self.positions = torch.zeros((B,), dtype=torch.int32, device=dev)
        self.step = torch.ones((1,), dtype=torch.int32, device=dev)
        self.result = torch.ones((B,), dtype=torch.int32, device=dev)
        self.tokens_out = torch.zeros((B, max_new), dtype=torch.int32, device=dev)
        self.col_offsets = torch.arange(B, dtype=torch.int32, device=dev) * max_new

    def reset_(self):
        """reset!(gen) (generate.jl:74-78): step = 1, tokens_out = 0."""
        self.step.fill_(1)
        self.tokens_out.zero_()
        return self

    def advance_(self):
        """advance!(gen) (generate.jl:82-88), one kernel: tokens_out[step, :] =
        result (when step <= max_new), step += 1, positions .+= 1."""
        if self.max_new == 0:
            call("vm_advance_positions", ops._p(self.positions), self.B, ops._stream())
            self.step.add_(1)
            return self
        call("vm_generation_advance", ops._p(self.tokens_out), ops._p(self.col_offsets),
             ops._p(self.step), ops._p(self.positions), ops._p(self.result), self.B,
             self.max_new, ops._stream())
        return self

    def poll(self, lo: int, hi: int):
        """Rows lo..hi (1-based) of tokens_out on the host, (hi - lo + 1, B)
        (generate.jl:92): one device-to-host copy."""
        return self.tokens_out[:, lo - 1:hi].t().contiguous().cpu().numpy()


def _qkv_views(qkv, cfg):
    """q, gate, k, v views of a packed (B, 2Hq+2Hkv, Dh) projection (qwen35.jl:195-198)."""
    q = qkv[:, 0:2 * cfg.Hq:2, :]
    g = qkv[:, 1:2 * cfg.Hq:2, :]
    k = qkv[:, 2 * cfg.Hq:2 * cfg.Hq + cfg.Hkv, :]
    v = qkv[:, 2 * cfg.Hq + cfg.Hkv:, :]
    return q, g, k, v


def gated_attn_decode_(O, l: AttnLayer, m: AttnModel, gen: Generation, qkv, *,
                       advance: bool = False):
    """One decode step of the attention block (qwen35.jl:195-205), fused:
    qnorm_rope! + knorm_rope_append! + decode_attention + ``O .*= sigmoid.(q_gate)``.

    qkv :: (Dh, 2Hq+2Hkv, B) packed projection; O :: (Dh, Hq, B) = the Wo input.
    Reads gen.positions; with ``advance`` also bumps it on the device (so one
    call is a capturable (step!; advance!)). Allocates nothing.
    """
    cfg = m.cfg
    d = sizes(qkv=(qkv, f"Dh {2 * cfg.Hq + 2 * cfg.Hkv} B"), O=(O, f"Dh {cfg.Hq} B"),
              K_cache=(l.K_cache, "Dh Ctx Hkv B"), V_cache=(l.V_cache, "Dh Ctx Hkv B"),
              positions=(gen.positions, "B"))
    if qkv.stride(1) != d["Dh"] or O.stride(1) != d["Dh"]:
        raise ArgumentError("qkv and O must be packed along the head axis")
    if l.K_cache.stride() != l.V_cache.stride():
        raise ArgumentError("K_cache and V_cache must share strides")
    c = l.K_cache
    call("vm_gated_attn_decode", ops._p(O), O.stride(0), ops._p(qkv), qkv.stride(0),
         ops._p(l.K_cache), ops._p(l.V_cache), c.stride(2), c.stride(1), c.stride(0), d["Ctx"],
         ops._p(l.qw), ops._p(l.kw), ops._p(m.rope["cos"]), ops._p(m.rope["sin"]),
         ops._p(gen.positions), int(bool(advance)), d["B"], cfg.Hq, cfg.Hkv, d["Dh"],
         cfg.rot_half, float(cfg.eps), 1.0, m.n_splits, ops._p(m.space), m.space.numel(),
         ops._stream())
    return O


def gated_attn_prefill(l: AttnLayer, m: AttnModel, qkv, T: int, B: int, *, offset: int = 0,
                       prior=None, q_lengths=None, out=None, staged: StagedV | None = None):
    """Prefill / chunked prefill of the attention block (qwen35.jl:293-317), fused:
    head_rmsnorm + apply_rope of q and k, the K/V cache write at columns
    offset+1..offset+T, causal attention over columns 1..offset+T, and the
    sigmoid gate, written directly in the Wo input layout (Dh*Hq, T*B).

    qkv :: (Dh*(2Hq+2Hkv), T*B) (any view reshapeable to torch (B, T, 2Hq+2Hkv, Dh)).
    ``offset`` is the uniform prior cache length (the reference's keyword);
    ``prior``/``q_lengths`` (B,) int32 device tensors make the batch ragged
    (each sequence b appends q_lengths[b] <= T tokens after prior[b]).
    ``staged`` (this layer's StagedV) keeps the V^T workspace between chunks, so
    the call stages only the chunk (vm_gated_attn_prefill_staged; same outputs).
    Returns out :: torch (B, T, Hq*Dh).
    """
    cfg = m.cfg
    S = 2 * cfg.Hq + 2 * cfg.Hkv
    ops._need(qkv, torch.bfloat16, "qkv")
    qkv4 = qkv.reshape(B, T, S, cfg.Dh)
    if qkv4.stride(3) != 1 or qkv4.stride(2) != cfg.Dh:
        raise ArgumentError("qkv must be packed along the slot axis")
    if prior is None:
        prior = torch.full((B,), int(offset), dtype=torch.int32, device="cuda")
    d = sizes(K_cache=(l.K_cache, "Dh Ctx Hkv B"), V_cache=(l.V_cache, "Dh Ctx Hkv B"),
              prior=(prior, "B"), q_lengths=(q_lengths, "B"), out=(out, f"{cfg.Hq * cfg.Dh} T B"))
    if d["B"] != B:
        raise DimensionMismatch(f"size(K_cache, 4) = {d['B']} does not match B = {B}")
    if d["Dh"] != cfg.Dh or d["Hkv"] != cfg.Hkv:
        raise DimensionMismatch(f"K_cache (Dh, Hkv) = ({d['Dh']}, {d['Hkv']}) does not match "
                                f"the config ({cfg.Dh}, {cfg.Hkv})")
    if out is not None and d["T"] != T:
        raise DimensionMismatch(f"size(out, 2) = {d['T']} does not match T = {T}")
    ops._need(l.K_cache, torch.bfloat16, "K_cache")
    ops._need(l.V_cache, torch.bfloat16, "V_cache")
    if l.K_cache.stride() != l.V_cache.stride():
        raise ArgumentError("K_cache and V_cache must share strides")
    ops._need(prior, torch.int32, "prior")
    ops._need(q_lengths, torch.int32, "q_lengths")
    # the reference's cache view K_cache[:, offset+1:offset+T, :, :] (qwen35.jl:306)
    # throws a BoundsError past the capacity; a device-side prior is the caller's
    # contract (prior[b] + q_lengths[b] <= Ctx), keys past the cache are masked
    if int(offset) < 0 or int(offset) + T > d["Ctx"]:
        raise BoundsError(f"attempt to access cache columns {int(offset) + 1}:{int(offset) + T} "
                          f"of a cache with Ctx = {d['Ctx']}")
    if out is None:
        out = torch.empty((B, T, cfg.Hq * cfg.Dh), dtype=torch.bfloat16, device="cuda")
    else:
        ops._need(out, torch.bfloat16, "out")
    c = l.K_cache
    args = (ops._p(out), out.stride(1), out.stride(0), ops._p(qkv4), qkv4.stride(1),
            qkv4.stride(0), ops._p(l.K_cache), ops._p(l.V_cache), c.stride(2), c.stride(1),
            c.stride(0), d["Ctx"], ops._p(l.qw), ops._p(l.kw), ops._p(m.rope["cos"]),
            ops._p(m.rope["sin"]), ops._p(prior), ops._p(q_lengths), B, T, cfg.Hq, cfg.Hkv,
            cfg.Dh, cfg.rot_half, float(cfg.eps), 1.0)
    if staged is None:
        ws = m.prefill_workspace(B, d["Ctx"])
        call("vm_gated_attn_prefill", *args, ops._p(ws), ws.numel(), ops._stream())
        return out
    if staged.B != B or staged.ctx != d["Ctx"]:
        raise DimensionMismatch(f"StagedV for (B, Ctx) = ({staged.B}, {staged.ctx}) used with "
                                f"({B}, {d['Ctx']})")
    if staged.cache != l.V_cache.data_ptr():  # another layer's tiles: stage everything
        staged.reset_()
        staged.cache = l.V_cache.data_ptr()
    call("vm_gated_attn_prefill_staged", *args, ops._p(staged.state), ops._p(staged.vt),
         staged.vt.numel(), ops._stream())
    return out


def _need_proj(l: AttnLayer, cfg: AttnConfig):
    S = 2 * cfg.Hq + 2 * cfg.Hkv
    if l.Wqkv is None or l.Wo is None:
        raise ArgumentError("this layer has no projections (Wqkv, Wo)")
    sizes(Wqkv=(l.Wqkv, f"{cfg.D} {S * cfg.Dh}"), Wo=(l.Wo, f"{cfg.Hq * cfg.Dh} {cfg.D}"))


def decode_(h, l: AttnLayer, m: AttnModel, gen: Generation, xn, *, advance: bool = False,
            project: bool = True):
    """decode!(h, l::AttnLayer, m, gen, xn) — qwen35.jl:187-208, hidden state to
    hidden state for one token per sequence: qkv = linear(xn, Wqkv) (:194), the
    fused gated attention (:195-205) into O, h = linear(O, Wo) (:206). xn, h ::
    (D, B) (torch (B, D)). The temporaries are the model's decode buffers, so the
    step allocates nothing once warm (capturable with ``advance``). With
    ``project=False`` the Wo projection is left to the caller (the step fuses it
    with the residual norm) and the Wo input (Hq·Dh, B) is returned."""
    cfg = m.cfg
    _need_proj(l, cfg)
    d = sizes(xn=(xn, f"{cfg.D} B"), h=(h, f"{cfg.D} B"))
    if d["B"] != cfg.B:
        raise DimensionMismatch(f"size(xn, 2) = {d['B']} does not match B = {cfg.B}")
    qkv, O = m.decode_buffers()
    q2, O2 = qkv.view(cfg.B, -1), O.view(cfg.B, -1)
    ws = m.decode_workspace(max(ops.linear_workspace_bytes(xn, l.Wqkv, q2),
                                ops.linear_workspace_bytes(O2, l.Wo, h)))
    ops.linear_({"y": q2}, xn, l.Wqkv, workspace=ws)
    gated_attn_decode_(O, l, m, gen, qkv, advance=advance)
    if not project:
        return O2
    ops.linear_({"y": h}, O2, l.Wo, workspace=ws)
    return h


def forward(l: AttnLayer, m: AttnModel, xn, T: int, B: int, *, offset: int = 0, prior=None,
            q_lengths=None, staged: StagedV | None = None):
    """forward(l::AttnLayer, m, xn, T, B; offset) — qwen35.jl:292-318, hidden
    state to hidden state for a prompt chunk: qkv = linear(xn, Wqkv) (:296), the
    fused gated prefill (:297-315) into the Wo input, h = linear(·, Wo)
    (:316-317). xn :: (D, T*B) (torch (B, T, D)); returns h, torch (B, T, D).
    Eager: allocates its temporaries, as the reference's prefill does. ``staged``:
    as for gated_attn_prefill."""
    cfg = m.cfg
    _need_proj(l, cfg)
    xn2 = xn.reshape(B * T, cfg.D)
    qkv = ops.linear(xn2, l.Wqkv, workspace=m.linear_workspace(
        ops.linear_workspace_bytes(xn2, l.Wqkv)))["y"]
    o = gated_attn_prefill(l, m, qkv.view(B, T, 2 * cfg.Hq + 2 * cfg.Hkv, cfg.Dh), T, B,
                           offset=offset, prior=prior, q_lengths=q_lengths, staged=staged)
    o2 = o.reshape(B * T, cfg.Hq * cfg.Dh)
    ws = m.linear_workspace(ops.linear_workspace_bytes(o2, l.Wo))
    return ops.linear(o2, l.Wo, workspace=ws)["y"].view(B, T, cfg.D)


class CaptureSession:
    """A captured decode step (generate.jl:158-196): capture once, replay many.

    ``capture(fn)`` records everything ``fn`` launches on a private stream into
    a hipGraph; ``launch()`` replays it on torch's current stream. The step must
    be device-driven (positions read and advanced on the device), which decode_
    with ``advance=True`` is.
    """

    def __init__(self):
        self.exec = None
        self.stream = None
        self.n_warm = 0     # eager warm-up steps spent (generate.jl:149-152)

    def capture(self, fn, models=()):
        """``models``: the AttnModels whose decode workspace ``fn`` uses; they
        are frozen (a later larger need raises instead of freeing the buffer
        the graph holds)."""
        for am in models:
            am.dec_frozen = True
        if self.exec is not None:
            raise ArgumentError("session already holds a graph")
        self.stream = torch.cuda.Stream()
        self.stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(self.stream):
            s = ctypes.c_void_p(self.stream.cuda_stream)
            call("vm_graph_begin_capture", s)
            try:
                fn()
            finally:
                ge = ctypes.c_void_p()
                call("vm_graph_end_capture", s, ctypes.byref(ge))
        self.exec = ge
        return self

    def launch(self):
        call("vm_graph_launch", self.exec, ops._stream())

    def close(self):
        if self.exec is not None:
            call("vm_graph_destroy", self.exec)
            self.exec = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
