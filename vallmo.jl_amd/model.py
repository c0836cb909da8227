"""The decode engine around the decoder layers — src/llm/qwen35.jl:168-185
(reset!), :220-273 (step!, the MLP), :369-395 (prefill!), :397-427 (snapshot /
restore!) and src/llm/generate.jl:54-196 (the clock, eager and captured
generation).

A model here is a stack of decoder layers whose mixer is either the gated
full-attention block (AttnLayer) or the Gated DeltaNet linear-attention block
(DeltaNetLayer), in the checkpoint's layer_types order (Qwen3.5: every
full_attention_interval-th layer is full attention, gguf_llamacpp.jl:47), each
with its two RMSNorms and MLP, between an embedding table and an lm head (the
embedding itself when tied). Greedy decoding only, as the reference's
lm_head_argmax!.

Every temporary of a decode step lives in buffers the model allocates once (the
reference's Arena frames, qwen35.jl:1-6): the residual stream x, the normed xn,
the mixer / MLP output h, the MLP's packed gate-up gu and mid, the DeltaNet
layers' projections, conv output and gated output, the lm-head partials, the
projections' workspace. So ``step_`` allocates nothing once warm, every step
uses the same addresses, and (step_; advance_) captures into a hipGraph that
replays self-advancing: the decode loop is one graph launch per token and
nothing else on the host. The DeltaNet state and conv ring advance in place and
carry across generations until ``reset_`` (qwen35.jl:168-185).
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field

import torch

from . import deltanet_layer as dn
from . import ops
from ._lib import ArgumentError, DimensionMismatch
from .deltanet_layer import DeltaNetConfig, DeltaNetLayer, DeltaNetSpace
from .layer import (AttnConfig, AttnLayer, AttnModel, CaptureSession, Generation, attn_layer,
                    decode_, forward)


@dataclass(frozen=True)
class ModelConfig:
    """The text-config facts the step reads (qwen35.jl:82-96): the attention
    block's (with D the hidden size and B, Ctx the decode batch and capacity),
    the linear-attention block's, the MLP's intermediate size, the vocabulary,
    the layer count and pattern: with ``interval`` k > 0, layer i (1-based) is
    full attention when i % k == 0 and DeltaNet otherwise (Qwen3.5: k = 4,
    gguf_llamacpp.jl:47-49); k = 0 makes every layer full attention."""
    attn: AttnConfig = field(default_factory=AttnConfig)
    inter: int = 9216
    vocab: int = 151936
    n_layers: int = 8
    tied: bool = True           # tie_word_embeddings: the head IS the embedding
    linear: DeltaNetConfig = field(default_factory=DeltaNetConfig)
    interval: int = 0           # full_attention_interval (0: all full attention)

    @property
    def D(self) -> int:
        return self.attn.D

    @property
    def B(self) -> int:
        return self.attn.B

    @property
    def layer_types(self) -> tuple:
        k = self.interval
        return tuple("full_attention" if k == 0 or i % k == 0 else "linear_attention"
                     for i in range(1, self.n_layers + 1))


class Model:
    """Qwen35 (qwen35.jl:46-55): cfg, the embedding E (D, vocab) (torch (vocab,
    D)), the head (E itself when tied), the final norm weight, the layers
    (AttnLayer / DeltaNetLayer), and the decode space."""

    def __init__(self, cfg: ModelConfig, layers, E, head, norm_w):
        if len(layers) == 0:
            raise ArgumentError("a model needs at least one layer")
        D, B, I = cfg.D, cfg.B, cfg.inter
        if tuple(E.shape) != (cfg.vocab, D) or tuple(head.shape) != (cfg.vocab, D):
            raise DimensionMismatch(f"E / head must be (D, vocab) = ({D}, {cfg.vocab})")
        self.cfg, self.layers, self.E, self.head, self.norm_w = cfg, list(layers), E, head, norm_w
        self.attn = AttnModel(cfg.attn)
        bf = dict(dtype=torch.bfloat16, device="cuda")
        # the step frame (qwen35.jl:248-250) and the layer frame's MLP temporaries
        # (qwen35.jl:235-238), one set for the whole stack
        self.x = torch.empty((B, D), **bf)
        self.xn = torch.empty((B, D), **bf)
        self.h = torch.empty((B, D), **bf)
        self.gu = torch.empty((B, 2 * I), **bf)
        self.mid = torch.empty((B, I), **bf)
        self.lm_scratch = torch.empty(max(ops.lm_head_argmax_scratch_bytes(self.xn, head), 16),
                                      dtype=torch.uint8, device="cuda")
        self.dn_layers = [l for l in self.layers if isinstance(l, DeltaNetLayer)]
        self.dn = DeltaNetSpace(cfg.linear, B) if self.dn_layers else None
        for l in self.dn_layers:
            dn.check_layer(l, cfg.linear, D, B)
        self._ws_need = None

    def workspace(self) -> torch.Tensor:
        """The projections' workspace, sized for every decode-step problem (grown
        here, eagerly, so a captured step finds it already large enough)."""
        if self._ws_need is None:
            l0 = self.layers[0]
            need = max(ops.linear_workspace_bytes(self.xn, l0.Wgu, self.gu),
                       ops.linear_silu_mul_workspace_bytes(self.xn, l0.Wgu),
                       ops.linear_workspace_bytes(self.mid, l0.Wd, self.h),
                       ops.linear_add_rms_norm_workspace_bytes(self.mid, l0.Wd))
            if self.dn_layers:
                l, c = self.dn_layers[0], self.cfg.linear
                O2 = self.dn.O.view(self.cfg.B, -1)
                need = max(need, ops.linear_workspace_bytes(self.xn, l.W_in, self.dn.qzab),
                           ops.linear_causal_conv1d_workspace_bytes(self.xn, l.W_in, self.dn.qzab),
                           ops.linear_workspace_bytes(O2, l.Wout, self.h),
                           ops.linear_add_rms_norm_workspace_bytes(O2, l.Wout))
            attn = [l for l in self.layers if not isinstance(l, DeltaNetLayer)]
            if attn:
                qkv, O = self.attn.decode_buffers()
                O2 = O.view(self.cfg.B, -1)
                need = max(need, ops.linear_add_rms_norm_workspace_bytes(O2, attn[0].Wo),
                           ops.linear_workspace_bytes(self.xn, attn[0].Wqkv, qkv.view(self.cfg.B, -1)),
                           ops.linear_workspace_bytes(O2, attn[0].Wo, self.h))
            self._ws_need = need
        # the decode workspace (never the eager prefill one): a captured step
        # replays this address, and it is sized here for every step problem
        return self.attn.decode_workspace(self._ws_need)

    def reset_(self):
        """reset!(m) — qwen35.jl:167-185: zero every DeltaNet state and conv ring
        (they carry across generations; the K/V caches need no reset)."""
        for l in self.dn_layers:
            l.reset_()
        return self

    def snapshot(self) -> list:
        """snapshot(m) — qwen35.jl:399-414: copies of each DeltaNet layer's
        (S, conv ring), None for attention layers."""
        return [(l.S.clone(), l.conv_state.clone()) if isinstance(l, DeltaNetLayer) else None
                for l in self.layers]

    def snapshot_(self, snap: list) -> list:
        """snapshot!(snap, m) — qwen35.jl:415-420: refresh a snapshot in place."""
        for s_, l in zip(snap, self.layers):
            if s_ is not None:
                s_[0].copy_(l.S)
                s_[1].copy_(l.conv_state)
        return snap

    def restore_(self, snap: list):
        """restore!(m, snap) — qwen35.jl:422-427: put a snapshot's states back
        (before a suffix prefill with offset)."""
        for s_, l in zip(snap, self.layers):
            if s_ is not None:
                l.S.copy_(s_[0])
                l.conv_state.copy_(s_[1])
        return self


def random_model(cfg: ModelConfig, *, seed: int = 0) -> Model:
    """A model of `cfg` with seeded synthetic weights on the device (the fill
    stream the CPU tests reproduce), layers in cfg.layer_types order:
    projections N(0, 1/K), RMSNorm weights N(0, 0.05) (applied as w + 1),
    embedding N(0, 1); DeltaNet layers: conv weight N(0, 1/K_conv), no conv bias
    (Qwen3.5's conv1d has none), A_log N(0.5, 0.5), dt_bias N(0, 0.5), gated-norm
    weight N(1, 0.05), zero state and ring."""
    a, D, I, c = cfg.attn, cfg.D, cfg.inter, cfg.linear
    S = 2 * a.Hq + 2 * a.Hkv

    def w(shape, s, scale, shift=0.0):
        t = torch.empty(shape, dtype=torch.bfloat16, device="cuda")
        return ops.fill_normal_(t, s, scale=scale, shift=shift)

    layers = []
    for i, kind in enumerate(cfg.layer_types):
        s0 = seed * 1000 + 16 * i
        if kind == "full_attention":
            l = attn_layer(a, w((a.Dh,), s0 + 1, 0.05), w((a.Dh,), s0 + 2, 0.05),
                           Wqkv=w((S * a.Dh, D), s0 + 3, D ** -0.5),
                           Wo=w((D, a.Hq * a.Dh), s0 + 4, (a.Hq * a.Dh) ** -0.5))
        else:
            HvDv = c.Hv * c.Dv
            l = dn.deltanet_layer(
                c, cfg.B, Wqz=w((c.n + HvDv, D), s0 + 9, D ** -0.5),
                Wab=w((2 * c.Hv, D), s0 + 10, D ** -0.5),
                Wout=w((D, HvDv), s0 + 11, HvDv ** -0.5),
                conv_w=w((c.convK, c.n), s0 + 12, c.convK ** -0.5),
                A_log=w((c.Hv,), s0 + 13, 0.5, 0.5).float(),
                dt_bias=w((c.Hv,), s0 + 14, 0.5).float(),
                gnorm_w=w((c.Dv,), s0 + 15, 0.05, 1.0))
        l.norm1 = w((D,), s0 + 5, 0.05)
        l.norm2 = w((D,), s0 + 6, 0.05)
        l.Wgu = w((2 * I, D), s0 + 7, D ** -0.5)
        l.Wd = w((D, I), s0 + 8, I ** -0.5)
        layers.append(l)
    E = w((cfg.vocab, D), seed * 1000 + 997, 1.0)
    head = E if cfg.tied else w((cfg.vocab, D), seed * 1000 + 998, 1.0)
    return Model(cfg, layers, E, head, w((D,), seed * 1000 + 999, 0.05))


def _need_layer(l):
    if isinstance(l, DeltaNetLayer):
        dn.need(l)
        return
    for n in ("norm1", "norm2", "Wgu", "Wd", "Wqkv", "Wo"):
        if getattr(l, n) is None:
            raise ArgumentError(f"decoder layer has no {n}")


def _mixer_decode(l, m: "Model", gen: Generation, xn):
    """The mixer up to its out projection: (its input, its weight)."""
    if isinstance(l, DeltaNetLayer):
        o = dn.decode_(None, l, m.cfg.linear, m.dn, xn, eps=m.cfg.attn.eps,
                       workspace=m.workspace(), project=False)
        return o, l.Wout
    return decode_(None, l, m.attn, gen, xn, project=False), l.Wo


def mlp_(h, l, m: Model, xn):
    """mlp!(h, mlp, cfg, xn) — qwen35.jl:234-243: gu = linear(xn, Wgu), mid =
    silu(gate) .* up, h = linear(mid, Wd); temporaries in the model's space."""
    ws = m.workspace()
    ops.linear_({"y": m.gu}, xn, l.Wgu, workspace=ws)
    ops.silu_mul_(m.mid, m.gu)
    ops.linear_({"y": h}, m.mid, l.Wd, workspace=ws)
    return h


def step_(m: Model, gen: Generation):
    """step!(m, gen) — qwen35.jl:245-273, one token per sequence, the capture
    target: x = E[:, result]; xn = rms_norm(x, norm1 of layer 1); per layer the
    mixer, the fused residual add + norm2, the MLP, the fused residual add + the
    next layer's norm1 (the final norm after the last); result = argmax of the
    head's logits. Reads gen.result and gen.positions only; writes gen.result.
    Every norm is applied as (w + 1) (offset = 1)."""
    cfg = m.cfg
    if gen.B != cfg.B:
        raise DimensionMismatch(f"Generation has B = {gen.B}, the model B = {cfg.B}")
    eps = cfg.attn.eps
    x, xn, h = m.x, m.xn, m.h
    ops.embed_(x, m.E, gen.result)
    ops.rms_norm_({"Y": xn}, x, m.layers[0].norm1, eps=eps, offset=1.0)
    n = len(m.layers)
    ws = m.workspace()
    for i, l in enumerate(m.layers):
        _need_layer(l)
        # the mixer, then its out projection fused with the residual add + norm2
        # (linear! + fused_add_rms_norm!, :206 + :265, bit-identical)
        o, W_out = _mixer_decode(l, m, gen, xn)
        ops.linear_add_rms_norm_({"Y": xn, "X": x}, o, W_out, l.norm2, eps=eps, offset=1.0,
                                 workspace=ws)
        # the MLP (mlp!, :234-243): the gate-up projection and silu .* mul in one
        # call (gu never written), the down projection fused with the next norm
        ops.linear_silu_mul_(m.mid, xn, l.Wgu, workspace=ws)
        next_w = m.norm_w if i == n - 1 else m.layers[i + 1].norm1
        ops.linear_add_rms_norm_({"Y": xn, "X": x}, m.mid, l.Wd, next_w, eps=eps, offset=1.0,
                                 workspace=ws)
    ops.lm_head_argmax_({"Result": gen.result}, xn, m.head, scratch=m.lm_scratch)
    return gen


def prefill_(m: Model, gen: Generation, ids, *, offset: int = 0):
    """prefill!(m, gen, ids; offset) — qwen35.jl:369-395, eager: ids (T, B)
    (torch (B, T) int32, 1-based) continue a resident prefix of `offset` tokens;
    fills every layer's cache columns offset+1 .. offset+T, puts the first
    generated token in gen.result (the last token's final-normed hidden row
    is left in m.xn) and, last, seeds the clock: positions = offset + T + 1."""
    cfg = m.cfg
    if ids.dim() != 2 or ids.dtype != torch.int32:
        raise ArgumentError("ids must be a (B, T) int32 tensor of 1-based token ids")
    B, T = ids.shape
    if B != cfg.B:
        raise DimensionMismatch(f"size(ids, 2) = {B} does not match B = {cfg.B}")
    if offset + T > cfg.attn.Ctx:
        raise ArgumentError(f"prefill past Ctx: offset {offset} + {T} tokens > {cfg.attn.Ctx}")
    eps = cfg.attn.eps
    x = torch.empty((B, T, cfg.D), dtype=torch.bfloat16, device="cuda")
    ops.embed_(x.view(B * T, cfg.D), m.E, ids.reshape(-1).contiguous())
    xn = ops.rms_norm(x, m.layers[0].norm1, eps=eps, offset=1.0)["Y"]
    n = len(m.layers)
    ws_for = lambda x_, W_: m.attn.linear_workspace(ops.linear_workspace_bytes(x_, W_))
    for i, l in enumerate(m.layers):
        _need_layer(l)
        if isinstance(l, DeltaNetLayer):
            h = dn.forward(l, cfg.linear, xn, T, B, eps=eps, offset=offset, workspace_for=ws_for)
        else:
            h = forward(l, m.attn, xn, T, B, offset=offset)
        ops.fused_add_rms_norm_({"Y": xn, "Xp": x}, x, h, l.norm2, eps=eps, offset=1.0)
        ws = m.attn.linear_workspace(ops.linear_workspace_bytes(xn, l.Wgu))
        gu = ops.linear(xn, l.Wgu, workspace=ws)["y"]
        mid = torch.empty((B, T, cfg.inter), dtype=torch.bfloat16, device="cuda")
        ops.silu_mul_(mid, gu)
        ws = m.attn.linear_workspace(ops.linear_workspace_bytes(mid, l.Wd))
        h = ops.linear(mid, l.Wd, workspace=ws)["y"]
        next_w = m.norm_w if i == n - 1 else m.layers[i + 1].norm1
        ops.fused_add_rms_norm_({"Y": xn, "Xp": x}, x, h, next_w, eps=eps, offset=1.0)
    # the last token's final-normed row goes to the step's xn buffer (the head's
    # input, qwen35.jl:392), where callers can read it
    m.xn.copy_(xn[:, T - 1, :])
    ops.lm_head_argmax_({"Result": gen.result}, m.xn, m.head, scratch=m.lm_scratch)
    gen.positions.fill_(offset + T + 1)   # the final act: seed the clock
    return gen


def _run(m: Model, gen: Generation, ids, *, max_new_tokens: int, launch_step, eos, poll_every,
         on_tokens, prefill_offset: int = 0):
    """_run! (generate.jl:95-130): prefill, harvest its token as row 1, then
    launch_step() per token with an amortised device->host poll every
    `poll_every` tokens for streaming and EOS."""
    if max_new_tokens < 1 or max_new_tokens > gen.max_new:
        raise ArgumentError(f"max_new_tokens = {max_new_tokens} outside 1..{gen.max_new}")
    gen.reset_()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    ev[0].record()
    prefill_(m, gen, ids, offset=prefill_offset)
    gen.advance_()                       # harvest prefill's token as row 1
    ev[1].record()
    n, polled, stop = 1, 0, False
    ev[2].record()
    while n < max_new_tokens and not stop:
        launch_step()
        n += 1
        if n - polled >= poll_every or n == max_new_tokens:
            chunk = gen.poll(polled + 1, n)
            if on_tokens is not None:
                on_tokens(chunk)
            if eos is not None:
                stop = bool((chunk == int(eos)).any())
            polled = n
    ev[3].record()
    torch.cuda.synchronize()
    tokens = gen.poll(1, n)
    prefill_s = ev[0].elapsed_time(ev[1]) * 1e-3
    decode_s = ev[2].elapsed_time(ev[3]) * 1e-3
    timing = dict(prefill_s=prefill_s, decode_s=decode_s, decode_tokens=n - 1,
                  tok_s=(n - 1) / decode_s if n > 1 else 0.0,
                  itl_ms=1e3 * decode_s / (n - 1) if n > 1 else 0.0)
    return tokens, timing


def generate_(m: Model, gen: Generation, ids, *, max_new_tokens: int, eos=None,
              poll_every: int = 8, on_tokens=None, prefill_offset: int = 0):
    """generate!(model, gen, ids; max_new_tokens, ...) (generate.jl:132-145):
    eager, every step launched from the host; the baseline the captured run
    must match token for token. Returns (tokens (n, B) numpy int32, timing)."""
    return _run(m, gen, ids, max_new_tokens=max_new_tokens, eos=eos, poll_every=poll_every,
                on_tokens=on_tokens, prefill_offset=prefill_offset,
                launch_step=lambda: (step_(m, gen), gen.advance_()))


def generate_captured_(m: Model, gen: Generation, ids, *, max_new_tokens: int, warmup: int = 3,
                       session: CaptureSession | None = None, eos=None, poll_every: int = 8,
                       on_tokens=None, prefill_offset: int = 0):
    """generate_captured!(model, gen, ids; max_new_tokens, warmup, session, ...)
    (generate.jl:147-196): `warmup` eager (step; advance) pairs, then one pair
    captured into a hipGraph and replayed for the remaining tokens. Capture
    records without executing, so warm-up's last state flows into the first
    replay. A session passed across calls (same model and generation) keeps its
    graph and warm-up count."""
    s = session if session is not None else CaptureSession()

    def launch_step():
        if s.n_warm < warmup:
            step_(m, gen)
            gen.advance_()
            s.n_warm += 1
        else:
            if s.exec is None:
                m.workspace()  # sized before capture, then fixed
                s.capture(lambda: (step_(m, gen), gen.advance_()), models=(m.attn,))
            s.launch()

    return _run(m, gen, ids, max_new_tokens=max_new_tokens, eos=eos, poll_every=poll_every,
                on_tokens=on_tokens, prefill_offset=prefill_offset, launch_step=launch_step)
