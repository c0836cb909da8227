"""Linear-attention (Gated DeltaNet) layer verbs — src/llm/qwen35.jl:144-165
(the layer), :210-232 (decode!) and :320-365 (forward).

Per token the layer projects the normed hidden state into [q | k | v | z] (Wqz)
and [alpha | beta] (Wab), runs the q | k | v channels through the depthwise
causal conv1d with its ring state (silu), then the gated delta-rule recurrence
on the per-value-head state S (fp32), the gated RMSNorm with the z gate, and the
out projection (Wout):

    decode_(h, l, m, xn)            decode!(h, l::DeltaNetLayer, m, gen, xn),
                                    qwen35.jl:210-232
    forward(l, m, xn, T, B; offset) forward(l::DeltaNetLayer, m, xn, T, B; offset),
                                    qwen35.jl:320-365

Both the ring and S are updated in place, as the reference's output_override
does (qwen35.jl:223, :229, :358); they carry across generations until
``reset_`` (qwen35.jl:168-185).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops
from ._lib import ArgumentError, DimensionMismatch
from .sizes import sizes


@dataclass(frozen=True)
class DeltaNetConfig:
    """The linear-attention facts of a Qwen3.5 text config (qwen35.jl:90-92):
    Dk = Dv = 128, 16 qk heads, 32 value heads, conv kernel 4 (Qwen3.5-4B)."""
    Dk: int = 128
    Dv: int = 128
    Hk: int = 16
    Hv: int = 32
    convK: int = 4

    @property
    def n(self) -> int:
        """conv channels: the q | k | v rows of the projection (qwen35.jl:147)."""
        return 2 * self.Dk * self.Hk + self.Dv * self.Hv


@dataclass
class DeltaNetLayer:
    """DeltaNetLayer (qwen35.jl:149-164): projections K-major (torch (M, K)), the
    conv weight (D, K) (torch (K, n)), bias or None, the ring (n, K, B) (torch
    (B, K, n)) bf16, A_log and dt_bias (Hv,) fp32, the gated-norm weight (Dv,),
    the state S (Dk, Dv, Hv, B) fp32 (torch (B, Hv, Dv, Dk)), and the decoder
    parts around the mixer (the two RMSNorms and the MLP).

    The reference runs [qkv | z] and [a | b] as two GEMVs because 12352 rows do
    not divide by Dk for its tiles (qwen35.jl:152-154); the narrow GEMV here
    needs only M % 4 == 0, so the layer stores them as one (n + Dv Hv + 2 Hv)-row
    projection W_in and keeps Wqz and Wab as its row blocks: one launch per
    token instead of two (the 64-row one alone cost a whole launch)."""
    W_in: torch.Tensor          # (D, n + Dv Hv + 2 Hv): [Wqz | Wab] in one projection
    Wqz: torch.Tensor           # (D, n + Dv Hv) -> torch (n + Dv Hv, D), a view of W_in
    Wab: torch.Tensor           # (D, 2 Hv) -> torch (2 Hv, D), a view of W_in
    Wout: torch.Tensor          # (Dv Hv, D) -> torch (D, Dv Hv)
    conv_w: torch.Tensor        # (n, K) -> torch (K, n)
    conv_b: torch.Tensor | None
    conv_state: torch.Tensor    # (n, K, B) -> torch (B, K, n), bf16
    A_log: torch.Tensor         # (Hv,) fp32
    dt_bias: torch.Tensor       # (Hv,) fp32
    gnorm_w: torch.Tensor       # (Dv,) bf16
    S: torch.Tensor             # (Dk, Dv, Hv, B) -> torch (B, Hv, Dv, Dk), fp32
    norm1: torch.Tensor | None = None
    norm2: torch.Tensor | None = None
    Wgu: torch.Tensor | None = None
    Wd: torch.Tensor | None = None

    def reset_(self):
        """Zero the recurrent state and the ring (qwen35.jl:175-185)."""
        self.S.zero_()
        self.conv_state.zero_()
        return self


def deltanet_layer(c: DeltaNetConfig, B: int, *, Wqz, Wab, Wout, conv_w, A_log, dt_bias, gnorm_w,
                   conv_b=None) -> DeltaNetLayer:
    """Allocate a layer with zeroed state (qwen35.jl:159-162)."""
    dev = Wqz.device
    if Wqz.shape[-1] != Wab.shape[-1]:
        raise DimensionMismatch(f"Wqz and Wab have different input widths "
                                f"({Wqz.shape[-1]}, {Wab.shape[-1]})")
    W_in = torch.cat([Wqz, Wab], 0)
    m = Wqz.shape[0]
    return DeltaNetLayer(
        W_in=W_in, Wqz=W_in[:m], Wab=W_in[m:], Wout=Wout, conv_w=conv_w, conv_b=conv_b,
        conv_state=torch.zeros((B, c.convK, c.n), dtype=torch.bfloat16, device=dev),
        A_log=A_log, dt_bias=dt_bias, gnorm_w=gnorm_w,
        S=torch.zeros((B, c.Hv, c.Dv, c.Dk), dtype=torch.float32, device=dev))


class DeltaNetSpace:
    """The decode step's temporaries of a DeltaNet layer (the layer frame of
    qwen35.jl:212-213, :222, :227), allocated once for the whole stack."""

    def __init__(self, c: DeltaNetConfig, B: int, device="cuda"):
        bf = dict(dtype=torch.bfloat16, device=device)
        m = c.n + c.Dv * c.Hv
        self.qzab = torch.empty((B, m + 2 * c.Hv), **bf)   # W_in's output
        self.qz, self.ab = self.qzab[:, :m], self.qzab[:, m:]
        self.conv = torch.empty((B, c.n), **bf)
        self.O = torch.empty((B, c.Hv, c.Dv), **bf)


def check_layer(l: DeltaNetLayer, c: DeltaNetConfig, D: int, B: int):
    n, HvDv = c.n, c.Hv * c.Dv
    sizes(W_in=(l.W_in, f"{D} {n + HvDv + 2 * c.Hv}"), Wqz=(l.Wqz, f"{D} {n + HvDv}"),
          Wab=(l.Wab, f"{D} {2 * c.Hv}"),
          Wout=(l.Wout, f"{HvDv} {D}"), conv_w=(l.conv_w, f"{n} {c.convK}"),
          conv_state=(l.conv_state, f"{n} {c.convK} {B}"), A_log=(l.A_log, f"{c.Hv}"),
          dt_bias=(l.dt_bias, f"{c.Hv}"), gnorm_w=(l.gnorm_w, f"{c.Dv}"),
          S=(l.S, f"{c.Dk} {c.Dv} {c.Hv} {B}"))


def _views(qz, c: DeltaNetConfig):
    """(conv input, z) of the projection rows: [q | k | v] then z (qwen35.jl:214-217)."""
    return qz[..., :c.n], qz[..., c.n:]


def decode_(h, l: DeltaNetLayer, c: DeltaNetConfig, space: DeltaNetSpace, xn, *, eps: float,
            workspace, project: bool = True):
    """decode!(h, l::DeltaNetLayer, m, gen, xn) — qwen35.jl:210-232: one token per
    sequence, hidden state to hidden state; the ring and S advance in place. xn,
    h :: (D, B) (torch (B, D)). Reads no clock: the recurrence carries position.
    With ``project=False`` the out projection is left to the caller and its
    input (Dv·Hv, B) is returned."""
    B = xn.shape[0]
    if space.qz.shape[0] != B:
        raise DimensionMismatch(f"size(xn, 2) = {B} does not match the decode space's B")
    # the projection [qz | ab] (:212-213), the conv of its first n channels
    # (:222-223) and the fused recurrence (:224-229) in one call: at B <= 32 the
    # projection's partials go straight to one kernel per (qk head, sequence)
    ops.linear_deltanet_decode_({"O": space.O, "y": space.qzab, "Y": space.conv,
                                 "Sp_ring": l.conv_state, "Sp": l.S}, xn, l.W_in, l.conv_state,
                                l.conv_w, l.conv_b, l.A_log, l.dt_bias, l.gnorm_w, l.S, Dk=c.Dk,
                                Dv=c.Dv, Hk=c.Hk, Hv=c.Hv, eps=eps, workspace=workspace)
    if not project:
        return space.O.view(B, c.Hv * c.Dv)
    ops.linear_({"y": h}, space.O.view(B, c.Hv * c.Dv), l.Wout, workspace=workspace)
    return h


def forward(l: DeltaNetLayer, c: DeltaNetConfig, xn, T: int, B: int, *, eps: float, offset: int,
            workspace_for):
    """forward(l::DeltaNetLayer, m, xn, T, B; offset) — qwen35.jl:320-365, a prompt
    chunk of T tokens per sequence: projections, the sequence conv (zero left
    context at offset 0, else the ring's last K-1 prefix inputs, read in place
    rather than copied, :333-344), the prep (l2 norms, gates), the recurrence in
    place on S (deltanet_sequence! in its chunked, MFMA form), the gated norm
    with z, Wout. xn :: (D, T*B) (torch (B, T, D));
    returns h, torch (B, T, D). Eager: allocates its temporaries.
    ``workspace_for(x, W)`` returns a projection workspace for that problem."""
    D = xn.shape[-1]
    xn2 = xn.reshape(B * T, D)
    m = c.n + c.Dv * c.Hv
    qzab = ops.linear(xn2, l.W_in, workspace=workspace_for(xn2, l.W_in))["y"].view(B, T, -1)
    qz, ab = qzab[..., :m], qzab[..., m:]                               # :322-323
    X, z = _views(qz, c)
    f32 = dict(dtype=torch.float32, device=xn.device)
    p = {"Q": torch.empty((B, c.Hk, T, c.Dk), **f32), "K": torch.empty((B, c.Hk, T, c.Dk), **f32),
         "V": torch.empty((B, c.Hv, T, c.Dv), **f32), "Beta": torch.empty((B, T, c.Hv), **f32),
         "Gate": torch.empty((B, T, c.Hv), **f32)}
    # the sequence conv (silu) and the prep in one pass: the conv output stays in
    # registers (causal_conv1d_sequence! then :347-356, bit for bit)
    ops.deltanet_conv_prep_(p, X, l.conv_w, ab, l.A_log, l.dt_bias, l.conv_b, Dk=c.Dk, Dv=c.Dv,
                            Hk=c.Hk, Hv=c.Hv, Sp=l.conv_state,
                            S=l.conv_state if offset > 0 else None)
    y = torch.empty((B, T, c.Hv, c.Dv), dtype=torch.bfloat16, device=xn.device)
    # the recurrence in place on S with the gated norm fused into its output
    # kernel (:357-364: O never reaches memory)
    ops.deltanet_sequence_chunked_gated_norm_({"Y": y, "Sp": l.S}, z.unflatten(-1, (c.Hv, c.Dv)),
                                              l.gnorm_w, p["Q"], p["K"], p["V"], p["Beta"],
                                              p["Gate"], l.S, eps=eps)
    y2 = y.view(B * T, c.Hv * c.Dv)
    return ops.linear(y2, l.Wout, workspace=workspace_for(y2, l.Wout))["y"].view(B, T, D)


def need(l: DeltaNetLayer):
    for n in ("norm1", "norm2", "Wgu", "Wd"):
        if getattr(l, n) is None:
            raise ArgumentError(f"decoder layer has no {n}")
