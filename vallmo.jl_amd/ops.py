"""Operators of the gated-attention path — the call surface of src/kernels/*.jl.

Each function keeps the reference's name (Julia's mutating ``op!`` is ``op_``
here), argument order, keyword arguments and error behaviour, and forwards to
the C ABI of libvallmo_attn.so. Tensors are torch tensors on the GPU (torch is
only the device-memory and stream plumbing); their shapes are the reference's
column-major dims reversed (Julia ``Q :: (D, Hq, B)`` is torch ``(B, Hq, D)``),
so strides map one to one. Launches go on torch's current stream, allocate
nothing (the allocating variants allocate outputs only) and never synchronise.

bf16 tensors are torch.bfloat16; lengths/positions torch.int32; tables float32.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import ArgumentError, DimensionMismatch, call
from .sizes import sizes

__all__ = [
    "rope_tables", "qnorm_rope_", "knorm_rope_append_", "attention_", "attention",
    "decode_attention_", "decode_attention", "decode_scratch_bytes", "sigmoid_gate_",
    "sigmoid", "fill_normal_", "linear_", "linear", "linear_workspace_bytes", "linear_tune",
    "rms_norm_", "rms_norm", "fused_add_rms_norm_", "fused_add_rms_norm", "silu_mul_",
    "embed_", "lm_head_argmax_", "lm_head_argmax", "lm_head_argmax_scratch_bytes",
    "causal_conv1d_", "causal_conv1d", "causal_conv1d_sequence_", "causal_conv1d_sequence",
    "fused_deltanet_decode_", "fused_deltanet_decode", "deltanet_recurrent_decode_",
    "deltanet_recurrent_decode", "deltanet_sequence_", "deltanet_sequence",
    "deltanet_prefill_prep_", "deltanet_conv_prep_", "gated_rms_norm_", "linear_add_rms_norm_",
    "deltanet_sequence_chunked_", "deltanet_sequence_workspace_bytes",
    "deltanet_sequence_chunked_gated_norm_", "linear_deltanet_decode_",
    "linear_add_rms_norm_workspace_bytes",
]


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _need(t, dtype, name):
    if t is None:
        return
    if not t.is_cuda:
        raise ArgumentError(f"{name} must be a GPU tensor")
    if t.dtype != dtype:
        raise ArgumentError(f"{name} must be {dtype}, got {t.dtype}")
    if t.dim() > 0 and t.stride(-1) != 1:
        raise ArgumentError(f"{name}: innermost dimension must be contiguous")


def _need_contig(t, name):
    if t is not None and not t.is_contiguous():
        raise ArgumentError(f"{name} must be contiguous")


def sigmoid(x):
    """1 / (1 + exp(-x)) — src/kernels/kernels.jl:34 (host-side scalar helper)."""
    import math
    return 1.0 / (1.0 + math.exp(-x))


def rope_tables(cfg) -> dict:
    """(cos, sin) :: (HALF_ROT, Ctx) fp32 — src/llm/qwen35.jl:115-119.

    ``cfg`` needs ``rot_half``, ``theta`` and ``Ctx``. Built on the device by
    vm_rope_tables; torch shape (Ctx, HALF_ROT).
    """
    half, ctx, theta = int(cfg.rot_half), int(cfg.Ctx), float(cfg.theta)
    cos = torch.empty((ctx, half), dtype=torch.float32, device="cuda")
    sin = torch.empty((ctx, half), dtype=torch.float32, device="cuda")
    call("vm_rope_tables", _p(cos), _p(sin), half, ctx, theta, _stream())
    return {"cos": cos, "sin": sin}


def qnorm_rope_(Q, QW, Cos, Sin, *, positions, eps, offset):
    """In-place per-head RMSNorm ``(w + offset)`` then partial RoPE on Q.

    src/kernels/qknorm_rope_append.jl:100-117. Q :: (D, Hq, B) (may be a strided
    view of the packed projection), QW :: (D,), Cos/Sin :: (HALF_ROT, Ctx),
    positions :: (B,) int32, 1-based column = rope column. D: a power of two
    from 16 to 512.
    """
    d = sizes(Q=(Q, "D Hq B"), QW=(QW, "D"), Cos=(Cos, "HALF_ROT Ctx"),
              Sin=(Sin, "HALF_ROT Ctx"), positions=(positions, "B"))
    if d["D"] & (d["D"] - 1):
        raise ArgumentError(f"D = {d['D']} must be a power of two")
    _need(Q, torch.bfloat16, "Q"); _need(QW, torch.bfloat16, "QW")
    _need(Cos, torch.float32, "Cos"); _need(Sin, torch.float32, "Sin")
    _need(positions, torch.int32, "positions")
    _need_contig(Cos, "Cos"); _need_contig(Sin, "Sin")
    call("vm_qnorm_rope", _p(Q), Q.stride(1), Q.stride(0), _p(QW), _p(Cos), _p(Sin), d["Ctx"],
         _p(positions), d["B"], d["Hq"], d["D"], d["HALF_ROT"], float(eps), float(offset),
         _stream())
    return Q


def knorm_rope_append_(K_cache, V_cache, K_raw, V_raw, KW, Cos, Sin, *, positions, eps, offset):
    """K norm + RoPE written into K_cache at column positions[b]; V copied alongside.

    src/kernels/qknorm_rope_append.jl:119-141. K_cache :: (Dk, Ctx, Hk, B),
    V_cache :: (Dv, Ctx, Hk, B), K_raw :: (Dk, Hk, B), V_raw :: (Dv, Hk, B)
    (views of the packed projection), KW :: (Dk,). Dk, Dv: powers of two from
    16 to 512.
    """
    d = sizes(K_cache=(K_cache, "Dk Ctx Hk B"), V_cache=(V_cache, "Dv Ctx Hk B"),
              K_raw=(K_raw, "Dk Hk B"), V_raw=(V_raw, "Dv Hk B"), KW=(KW, "Dk"),
              Cos=(Cos, "HALF_ROT Ctx"), Sin=(Sin, "HALF_ROT Ctx"), positions=(positions, "B"))
    for t, n in ((K_cache, "K_cache"), (V_cache, "V_cache"), (K_raw, "K_raw"), (V_raw, "V_raw"),
                 (KW, "KW")):
        _need(t, torch.bfloat16, n)
    _need(positions, torch.int32, "positions")
    _need_contig(Cos, "Cos"); _need_contig(Sin, "Sin")
    call("vm_knorm_rope_append", _p(K_cache), K_cache.stride(2), K_cache.stride(1),
         K_cache.stride(0), _p(V_cache), V_cache.stride(2), V_cache.stride(1), V_cache.stride(0),
         d["Ctx"], _p(K_raw), K_raw.stride(1), K_raw.stride(0), _p(V_raw), V_raw.stride(1),
         V_raw.stride(0), _p(KW), _p(Cos), _p(Sin), _p(positions), d["B"], d["Hk"], d["Dk"],
         d["Dv"], d["HALF_ROT"], float(eps), float(offset), _stream())


def _out(outs, key="O"):
    return outs[key] if isinstance(outs, dict) else getattr(outs, key)


def attention_(outs, Q, K, V, *, causal=False, k_lengths=None, q_lengths=None):
    """Flash attention forward (prefill) — src/kernels/attention.jl:93-129.

    Q :: (Dk, L, H, B), K :: (Dk, Lk, Hk, B), V :: (Dv, Lk, Hk, B) (typically
    cache prefixes), O :: (Dv, L, H, B). Queries are the suffix of keys: the
    causal offset is k_len - q_len per sequence. Optional k_lengths/q_lengths ::
    (B,) int32 make the batch ragged; rows past q_len are not written.
    """
    O = _out(outs)
    d = sizes(Q=(Q, "Dk L H B"), K=(K, "Dk Lk Hk B"), V=(V, "Dv Lk Hk B"), O=(O, "Dv L H B"),
              k_lengths=(k_lengths, "B"), q_lengths=(q_lengths, "B"))
    if d["H"] % d["Hk"]:
        raise DimensionMismatch(
            f"Attention heads ({d['H']}) is not a multiple of key-value heads ({d['Hk']})")
    for t, n in ((Q, "Q"), (K, "K"), (V, "V"), (O, "O")):
        _need(t, torch.bfloat16, n)
    _need(k_lengths, torch.int32, "k_lengths"); _need(q_lengths, torch.int32, "q_lengths")
    call("vm_attention_fwd", _p(O), O.stride(2), O.stride(1), O.stride(0), _p(Q), Q.stride(2),
         Q.stride(1), Q.stride(0), _p(K), K.stride(2), K.stride(1), K.stride(0), _p(V),
         V.stride(2), V.stride(1), V.stride(0), _p(k_lengths), _p(q_lengths), d["B"], d["H"],
         d["Hk"], d["Dk"], d["Dv"], d["L"], d["Lk"], int(bool(causal)), _stream())
    return outs


def attention(Q, K, V, **kw) -> dict:
    """Allocating attention (src/kernels/attention.jl:131-134): returns {"O": O}."""
    B, H, L, _ = Q.shape
    O = torch.empty((B, H, L, V.shape[-1]), dtype=Q.dtype, device=Q.device)
    return attention_({"O": O}, Q, K, V, **kw)


def decode_scratch_bytes(Q, K, V=None, *, n_splits=0) -> int:
    """Scratch the split-KV decode needs (Pol.scratch, attention_decode.jl:186-197);
    V (default: K) gives Dv."""
    B, H, _ = Q.shape
    Hk, L = K.shape[1], K.shape[2]
    Dv = (K if V is None else V).shape[3]
    return int(_lib.load().vm_decode_scratch_bytes(B, H, Hk, Dv, L, int(n_splits)))


def decode_attention_(outs, Q, K, V, *, lengths, n_splits=0, scratch=None):
    """Split-KV flash-decoding — src/kernels/attention_decode.jl:134-181.

    Q :: (Dk, H, Batch) normalised+rotated, K/V :: (Dk, L, Hk, Batch) caches,
    lengths :: (Batch,) int32 attended keys, O :: (Dv, H, Batch). The keys of
    all (sequence, kv-head) pairs form one stream cut into equal chunks, one per
    wave: n_splits = 0 uses 4 waves per CU, n_splits > 0 uses n_splits waves per
    (sequence, kv-head) on average (the reference's default is 8 fixed splits);
    ``scratch`` is a uint8 GPU tensor of >= decode_scratch_bytes (allocated if None).
    """
    O = _out(outs)
    d = sizes(Q=(Q, "Dk H Batch"), K=(K, "Dk L Hk Batch"), V=(V, "Dv L Hk Batch"),
              O=(O, "Dv H Batch"), lengths=(lengths, "Batch"))
    if d["H"] % d["Hk"]:
        raise DimensionMismatch(
            f"Attention heads ({d['H']}) is not a multiple of key-value heads ({d['Hk']})")
    for t, n in ((Q, "Q"), (K, "K"), (V, "V"), (O, "O")):
        _need(t, torch.bfloat16, n)
    _need(lengths, torch.int32, "lengths")
    need = decode_scratch_bytes(Q, K, V, n_splits=n_splits)
    if scratch is None:
        scratch = torch.empty(max(need, 16), dtype=torch.uint8, device=Q.device)
    call("vm_decode_attention", _p(O), O.stride(1), O.stride(0), _p(Q), Q.stride(1), Q.stride(0),
         _p(K), K.stride(2), K.stride(1), K.stride(0), _p(V), V.stride(2), V.stride(1),
         V.stride(0), d["L"], _p(lengths), d["Batch"], d["H"], d["Hk"], d["Dk"], d["Dv"],
         int(n_splits), _p(scratch), scratch.numel(), _stream())
    return outs


def decode_attention(Q, K, V, *, lengths, **kw) -> dict:
    """Allocating decode attention (attention_decode.jl:183-184, 200): returns {"O": O}."""
    O = torch.empty((Q.shape[0], Q.shape[1], V.shape[-1]), dtype=Q.dtype, device=Q.device)
    return decode_attention_({"O": O}, Q, K, V, lengths=lengths, **kw)


def sigmoid_gate_(O, G):
    """O .*= sigmoid.(G) in place — the decode gate of src/llm/qwen35.jl:205.

    O, G :: (D, H, B) bf16 (G typically the stride-2 gate view of the projection).
    """
    d = sizes(O=(O, "D H B"), G=(G, "D H B"))
    _need(O, torch.bfloat16, "O"); _need(G, torch.bfloat16, "G")
    call("vm_sigmoid_gate", _p(O), O.stride(1), O.stride(0), _p(G), G.stride(1), G.stride(0),
         d["B"], d["H"], d["D"], _stream())
    return O


_TUNED = set()


def _tune(M, N, K, ldw, ldx, ldy):
    """vm_linear_tune once per problem and device, outside any stream capture
    (the timing allocates and waits); under capture the plan keeps the
    heuristic's first, as the reference's does."""
    key = (torch.cuda.current_device(), M, N, K, ldw, ldx, ldy)
    if key in _TUNED or torch.cuda.is_current_stream_capturing():
        return
    call("vm_linear_tune", M, N, K, ldw, ldx, ldy)
    _TUNED.add(key)


def linear_tune(x, W, y=None):
    """Time the candidate algorithms of this problem's plan and keep the fastest
    (vm_linear_tune: a load-time call that allocates scratch and synchronises;
    no counterpart in the reference, whose plan keeps the heuristic's first).
    linear_workspace_bytes calls it for a new problem when no capture runs."""
    N, K, M = _rows(x), x.shape[-1], W.shape[0]
    ldy = M if y is None else y.stride(-2) if y.dim() > 1 else M
    _tune(M, N, K, W.stride(0), _ld(x), ldy)


def linear_workspace_bytes(x, W, y=None) -> int:
    """Workspace the cached plan of this problem needs (builds the plan on first
    use, linear.jl:22-38; tuned first when no capture runs, see linear_tune)."""
    N, K = _rows(x), x.shape[-1]
    M = W.shape[0]
    ldy = M if y is None else y.stride(-2) if y.dim() > 1 else M
    _tune(M, N, K, W.stride(0), _ld(x), ldy)
    n = _lib.load().vm_linear_workspace_bytes(M, N, K, W.stride(0), _ld(x), ldy)
    if n == ctypes.c_size_t(-1).value:
        _lib.check(_lib.VM_E_UNSUPPORTED, "vm_linear_workspace_bytes")
    return int(n)


def _rows(t):
    return 1 if t.dim() == 1 else int(t.numel() // t.shape[-1])


def _ld(t):
    """Column stride of the reference's column-major (K, N) view of a torch
    (..., K) tensor whose leading dims collapse into N."""
    if t.dim() == 1:
        return t.shape[-1]
    st = t.stride()
    for d in range(t.dim() - 2, 0, -1):
        if st[d - 1] != st[d] * t.shape[d]:
            raise ArgumentError("leading dimensions must collapse into one column axis")
    return st[-2]


def linear_(outs, x, W, *, workspace=None):
    """y .= W^T x — src/linear.jl:40-57 (hipBLASLt, fp32 accumulation).

    x :: (K, N) (torch (..., K), leading dims collapse into N), W :: (K, M)
    K-major (torch (M, K)), y :: (M, N) (torch (..., M)). ``workspace`` is a
    uint8 GPU tensor of >= linear_workspace_bytes (the reference takes it from
    the ambient arena, linear.jl:62-66); allocated here when None.
    """
    y = _out(outs, "y")
    K, N, M = x.shape[-1], _rows(x), W.shape[0]
    if W.dim() != 2 or W.shape[1] != K:
        raise DimensionMismatch(f"size(W, 1) = {W.shape[-1]} does not match K = {K} (= size(x, 1))")
    if y.shape[-1] != M or _rows(y) != N:
        raise DimensionMismatch(f"y is ({y.shape[-1]}, {_rows(y)}), expected (M, N) = ({M}, {N})")
    for t, n in ((x, "x"), (W, "W"), (y, "y")):
        _need(t, torch.bfloat16, n)
    need = linear_workspace_bytes(x, W, y)
    if workspace is None:
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=x.device)
    call("vm_linear", _p(y), _ld(y), _p(x), _ld(x), _p(W), W.stride(0), M, N, K,
         _p(workspace), workspace.numel(), _stream())
    return outs


def linear(x, W, **kw) -> dict:
    """Allocating linear (linear.jl:68-79): returns {"y": y}, torch (..., M)."""
    y = torch.empty(tuple(x.shape[:-1]) + (W.shape[0],), dtype=x.dtype, device=x.device)
    return linear_({"y": y}, x, W, **kw)


def linear_add_rms_norm_workspace_bytes(a, W) -> int:
    """Workspace of linear_add_rms_norm_ for this problem."""
    M, K, N = W.shape[0], a.shape[-1], _rows(a)
    _tune(M, N, K, W.stride(0), _ld(a), M)
    n = _lib.load().vm_linear_add_rms_norm_workspace_bytes(M, N, K, W.stride(0), _ld(a))
    if n == ctypes.c_size_t(-1).value:
        _lib.check(_lib.VM_E_UNSUPPORTED, "vm_linear_add_rms_norm_workspace_bytes")
    return int(n)


def linear_add_rms_norm_(outs, a, W, norm_w, *, eps, offset, workspace=None):
    """linear! then fused_add_rms_norm! in one call, bit-identical to the two
    (the decode step's pairs at src/llm/qwen35.jl:206 + :265, :241 + :268):
    h = bf16(W^T a); X = bf16(X + h) in place; Y = rms_norm(X) (w + offset).
    outs: "Y" (D, N) and "X" (D, N), the residual stream updated in place;
    a :: (K, N), W :: (K, D) K-major (torch (D, K)). No reference counterpart
    as one op; saves the reduce launch of a split GEMV and the bf16 h."""
    Y, X = _out(outs, "Y"), _out(outs, "X")
    D, N, ys = _cols(Y, "Y")
    Dx, Nx, xs = _cols(X, "X")
    K, Na, as_ = _cols(a, "a")
    if W.dim() != 2 or tuple(W.shape) != (D, K) or (Dx, Nx) != (D, N) or Na != N:
        raise DimensionMismatch(f"linear_add_rms_norm: a ({K}, {Na}), W {tuple(W.shape)}, "
                                f"X ({Dx}, {Nx}), Y ({D}, {N})")
    _need(W, torch.bfloat16, "W")
    _need(norm_w, torch.bfloat16, "norm_w")
    sizes(norm_w=(norm_w, f"{D}"))
    need = linear_add_rms_norm_workspace_bytes(a, W)
    if workspace is None:
        workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=a.device)
    call("vm_linear_add_rms_norm", _p(Y), ys, _p(X), xs, _p(a), as_, _p(W), W.stride(0),
         _p(norm_w), D, N, K, float(eps), float(offset), _p(workspace), workspace.numel(),
         _stream())
    return outs


def linear_silu_mul_workspace_bytes(x, W) -> int:
    """Workspace of linear_silu_mul_ for this problem."""
    M, K, N = W.shape[0], x.shape[-1], _rows(x)
    _tune(M, N, K, W.stride(0), _ld(x), M)  # the two-call path's plan (N > 32)
    n = _lib.load().vm_linear_silu_mul_workspace_bytes(M // 2, N, K, W.stride(0), _ld(x))
    if n == ctypes.c_size_t(-1).value:
        _lib.check(_lib.VM_E_UNSUPPORTED, "vm_linear_silu_mul_workspace_bytes")
    return int(n)


def linear_silu_mul_(mid, x, W, *, workspace=None):
    """linear! then silu .* mul in one call (the MLP's first half,
    src/llm/qwen35.jl:234-243): gu = bf16(W^T x), mid = bf16(silu(gate) .* up).
    x :: (K, N), W :: (K, 2I) K-major (torch (2I, K)), gate rows first; mid ::
    (I, N) (torch (..., I)). No reference counterpart as one op: at N <= 32 the
    projection's fp32 partials go straight to the silu kernel, gu is never
    written."""
    I, N, ms = _cols(mid, "mid")
    K, Nx, xs = _cols(x, "x")
    if W.dim() != 2 or tuple(W.shape) != (2 * I, K) or Nx != N:
        raise DimensionMismatch(f"linear_silu_mul: x ({K}, {Nx}), W {tuple(W.shape)}, "
                                f"mid ({I}, {N}): expected W (2I, K) = ({2 * I}, {K})")
    _need(W, torch.bfloat16, "W")
    need = linear_silu_mul_workspace_bytes(x, W)
    if workspace is None:
        workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=x.device)
    call("vm_linear_silu_mul", _p(mid), ms, _p(x), xs, _p(W), W.stride(0), I, N, K,
         _p(workspace), workspace.numel(), _stream())
    return mid


def _cols(t, name, M=None):
    """(M, N, column stride) of the reference's column-major (M, N) view of a
    torch (..., M) bf16 tensor."""
    _need(t, torch.bfloat16, name)
    return t.shape[-1], _rows(t), _ld(t)


def rms_norm_(outs, X, W, *, eps, offset=0.0):
    """rms_norm!((; Y), X, W; eps, offset) — src/kernels/rms_norm.jl:33-50.
    X, Y :: (M, N) (torch (..., M)), W :: (M,)."""
    Y = _out(outs, "Y")
    M, N, xs = _cols(X, "X")
    My, Ny, ys = _cols(Y, "Y")
    sizes(W=(W, f"{M}"))
    if (My, Ny) != (M, N):
        raise DimensionMismatch(f"Y is ({My}, {Ny}), X is ({M}, {N})")
    _need(W, torch.bfloat16, "W")
    call("vm_rms_norm", _p(Y), ys, _p(X), xs, _p(W), M, N, float(eps), float(offset), _stream())
    return outs


def rms_norm(X, W, **kw) -> dict:
    """Allocating rms_norm (rms_norm.jl:52-57): {"Y": Y}."""
    return rms_norm_({"Y": torch.empty_like(X)}, X, W, **kw)


def fused_add_rms_norm_(outs, X, dX, W, *, eps, offset):
    """fused_add_rms_norm!((; Y, X′), X, ΔX, W; eps, offset) —
    src/kernels/residual_norm.jl:39-60: X′ = X + ΔX, Y = rms_norm(X′). X′ may be
    X itself (the decode step's in-place residual, qwen35.jl:265). Keys "Y" and
    "Xp" (X′)."""
    Y, Xp = _out(outs, "Y"), _out(outs, "Xp")
    M, N, xs = _cols(X, "X")
    for t, n in ((dX, "dX"), (Y, "Y"), (Xp, "Xp")):
        Mt, Nt, _ = _cols(t, n)
        if (Mt, Nt) != (M, N):
            raise DimensionMismatch(f"{n} is ({Mt}, {Nt}), X is ({M}, {N})")
    sizes(W=(W, f"{M}"))
    _need(W, torch.bfloat16, "W")
    call("vm_fused_add_rms_norm", _p(Y), _ld(Y), _p(Xp), _ld(Xp), _p(X), xs, _p(dX), _ld(dX),
         _p(W), M, N, float(eps), float(offset), _stream())
    return outs


def fused_add_rms_norm(X, dX, W, **kw) -> dict:
    """Allocating fused_add_rms_norm (residual_norm.jl:62-65): {"Y": Y, "Xp": X′}."""
    return fused_add_rms_norm_({"Y": torch.empty_like(X), "Xp": torch.empty_like(X)}, X, dX, W,
                               **kw)


def silu_mul_(mid, gu):
    """mid .= silu.(gate) .* up, (gate; up) the two halves of each column of the
    packed gate-up projection gu :: (2I, N) — the MLP of src/llm/qwen35.jl:234-243.
    mid :: (I, N) (torch (..., I))."""
    I2, N, gs = _cols(gu, "gu")
    I, Nm, ms = _cols(mid, "mid")
    if I2 != 2 * I or Nm != N:
        raise DimensionMismatch(f"gu is ({I2}, {N}), mid is ({I}, {Nm}): expected (2I, N), (I, N)")
    call("vm_silu_mul", _p(mid), ms, _p(gu), gs, I, N, _stream())
    return mid


def embed_(x, E, ids):
    """x .= E[:, ids] — the decode step's embedding gather (src/llm/qwen35.jl:251).
    E :: (D, vocab) (torch (vocab, D)), ids :: (B,) int32 1-based, x :: (D, B)."""
    D, B, xs = _cols(x, "x")
    De, vocab, es = _cols(E, "E")
    if De != D:
        raise DimensionMismatch(f"size(E, 1) = {De} does not match size(x, 1) = {D}")
    sizes(ids=(ids, f"{B}"))
    _need(ids, torch.int32, "ids")
    call("vm_embed", _p(x), xs, _p(E), es, _p(ids), D, B, vocab, _stream())
    return x


def lm_head_argmax_scratch_bytes(X, W) -> int:
    """Per-wave partials of lm_head_argmax! (the reference's LocalMax / LocalIdx,
    lm_head_topk.jl:149-160)."""
    return int(_lib.load().vm_lm_head_argmax_scratch_bytes(X.shape[-1], _rows(W), _rows(X)))


def lm_head_argmax_(outs, X, W, *, scratch=None):
    """lm_head_argmax!((; Result), X, W) — src/kernels/lm_head_topk.jl:109-147:
    Result[b] = argmax(W^T X[:, b]), 1-based, ties to the smallest index, the
    logits never written. X :: (K, B) (torch (B, K)), W :: (K, N) K-major (torch
    (N, K): the embedding table itself for a tied head)."""
    R = _out(outs, "Result")
    K, B, xs = _cols(X, "X")
    Kw, N, ws = _cols(W, "W")
    if Kw != K:
        raise DimensionMismatch(f"size(W, 1) = {Kw} does not match size(X, 1) = {K}")
    sizes(Result=(R, f"{B}"))
    _need(R, torch.int32, "Result")
    need = lm_head_argmax_scratch_bytes(X, W)
    if scratch is None:
        scratch = torch.empty(max(need, 16), dtype=torch.uint8, device=X.device)
    call("vm_lm_head_argmax", _p(R), _p(X), xs, _p(W), ws, K, N, B, _p(scratch), scratch.numel(),
         _stream())
    return outs


def lm_head_argmax(X, W, **kw) -> dict:
    """Allocating lm_head_argmax (lm_head_topk.jl:149-163): {"Result": (B,) int32}."""
    R = torch.empty((_rows(X),), dtype=torch.int32, device=X.device)
    return lm_head_argmax_({"Result": R}, X, W, **kw)


# ---- the linear-attention layer parts (src/kernels/causal_conv1d.jl,
# deltanet_recurrent.jl, deltanet_fused.jl) -----------------------------------

def _st(t, dim, canon):
    """Stride of dim, or the canonical one when the extent is 1 (any stride is
    valid there, torch may report an odd one)."""
    return t.stride(dim) if t.shape[dim] > 1 else canon


def _act(sigma):
    if sigma is None:
        return 0
    if sigma == "silu" or getattr(sigma, "__name__", "") == "silu":
        return 1
    raise ArgumentError(f"σ = {sigma!r}: the kernels apply silu or nothing")


def causal_conv1d_(outs, X, S, Weight, Bias=None, *, sigma=None):
    """causal_conv1d!((; Y, S′), X, S, Weight, Bias; σ) — src/kernels/causal_conv1d.jl:43-61:
    one decode step. X, Y :: (D, B) (torch (B, D), rows may be strided), the ring
    S, S′ :: (D, K, B) (torch (B, K, D)), Weight :: (D, K) (torch (K, D)), Bias ::
    (D,) or None; σ None or "silu". S′ may be S itself (in place, qwen35.jl:223)."""
    Y, Sp = _out(outs, "Y"), _out(outs, "Sp")
    dims = sizes(Y=(Y, "D B"), X=(X, "D B"), S=(S, "D K B"), Sp=(Sp, "D K B"),
                 Weight=(Weight, "D K"), Bias=(Bias, "D"))
    D, K, B = dims["D"], dims["K"], dims["B"]
    for t, n in ((Y, "Y"), (X, "X"), (S, "S"), (Sp, "S′"), (Weight, "Weight"), (Bias, "Bias")):
        _need(t, torch.bfloat16, n)
    if S.stride() != Sp.stride():
        raise ArgumentError("S and S′ must share strides")
    call("vm_causal_conv1d", _p(Y), _st(Y, 0, D), _p(X), _st(X, 0, D), _p(S), _p(Sp),
         _st(S, 1, D), _st(S, 0, K * D), _p(Weight), _st(Weight, 0, D), _p(Bias), D, K, B,
         _act(sigma), _stream())
    return outs


def linear_causal_conv1d_workspace_bytes(x, W, y) -> int:
    """Workspace of linear_causal_conv1d_ for this problem."""
    M, K, N = W.shape[0], x.shape[-1], _rows(x)
    _tune(M, N, K, W.stride(0), _ld(x), _ld(y))  # the two-call path's plan (N > 32)
    n = _lib.load().vm_linear_causal_conv1d_workspace_bytes(M, N, K, W.stride(0), _ld(x), _ld(y))
    if n == ctypes.c_size_t(-1).value:
        _lib.check(_lib.VM_E_UNSUPPORTED, "vm_linear_causal_conv1d_workspace_bytes")
    return int(n)


def linear_causal_conv1d_(outs, x, W, S, Weight, Bias=None, *, sigma=None, workspace=None):
    """linear! then causal_conv1d! on the projection's first D channels in one
    call (the DeltaNet layer's decode step, src/llm/qwen35.jl:212-223):
    y = bf16(W^T x) (every channel written), then causal_conv1d!((; Y, S′),
    y[1:D, :], S, Weight, Bias; σ). outs: "y" (M, N) (torch (N, M)), "Y" (D, N),
    "Sp" (D, K, N), which may be S itself. x :: (K, N), W :: (K, M) K-major (torch
    (M, K)). No reference counterpart as one op: at N <= 32 the projection's fp32
    partials go straight to the conv kernel."""
    y, Y, Sp = _out(outs, "y"), _out(outs, "Y"), _out(outs, "Sp")
    M, N, ldy = _cols(y, "y")
    K, Nx, ldx = _cols(x, "x")
    if W.dim() != 2 or tuple(W.shape) != (M, K) or Nx != N:
        raise DimensionMismatch(f"linear_causal_conv1d: x ({K}, {Nx}), W {tuple(W.shape)}, "
                                f"y ({M}, {N})")
    dims = sizes(Y=(Y, "D B"), S=(S, "D Kc B"), Sp=(Sp, "D Kc B"), Weight=(Weight, "D Kc"),
                 Bias=(Bias, "D"))
    D, Kc = dims["D"], dims["Kc"]
    if dims["B"] != N:
        raise DimensionMismatch(f"linear_causal_conv1d: the conv has B = {dims['B']}, x has N = {N}")
    for t, n in ((W, "W"), (Y, "Y"), (S, "S"), (Sp, "S′"), (Weight, "Weight"), (Bias, "Bias")):
        _need(t, torch.bfloat16, n)
    if S.stride() != Sp.stride():
        raise ArgumentError("S and S′ must share strides")
    need = linear_causal_conv1d_workspace_bytes(x, W, y)
    if workspace is None:
        workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=x.device)
    call("vm_linear_causal_conv1d", _p(y), ldy, _p(x), ldx, _p(W), W.stride(0), M, N, K,
         _p(Y), _st(Y, 0, D), _p(S), _p(Sp), _st(S, 1, D), _st(S, 0, Kc * D), _p(Weight),
         _st(Weight, 0, D), _p(Bias), D, Kc, _act(sigma), _p(workspace), workspace.numel(),
         _stream())
    return outs


def linear_deltanet_decode_(outs, x, W, S_ring, Weight, Bias, A_log, DtBias, NormWeight, S, *,
                            Dk, Dv, Hk, Hv, eps=1e-6, workspace=None):
    """The DeltaNet layer's decode step up to its out projection in one call
    (src/llm/qwen35.jl:212-232): linear! of W (the in projection [q | k | v | z |
    alpha | beta], torch (M, K)) over x (K, B) (torch (B, K)) into outs["y"] (M, B),
    causal_conv1d! (silu) of its q | k | v channels on the ring S_ring into
    outs["Y"] (D, B) and outs["Sp_ring"], then fused_deltanet_decode! into
    outs["O"] (Dv, Hv, B) and outs["Sp"] (S′; either ring or state may be in
    place). Results equal linear_causal_conv1d_ then fused_deltanet_decode_ bit
    for bit. At B <= 32 on aligned views y and Y are not written (the projection's
    partials feed one kernel per (qk head, sequence)). No reference counterpart
    as one op."""
    O, y, Y = _out(outs, "O"), _out(outs, "y"), _out(outs, "Y")
    Sp_ring, Sp = _out(outs, "Sp_ring"), _out(outs, "Sp")
    M, N, ldy = _cols(y, "y")
    K, Nx, ldx = _cols(x, "x")
    if W.dim() != 2 or tuple(W.shape) != (M, K) or Nx != N:
        raise DimensionMismatch(f"linear_deltanet_decode: x ({K}, {Nx}), W {tuple(W.shape)}, "
                                f"y ({M}, {N})")
    dims = sizes(Y=(Y, "D B"), S_ring=(S_ring, "D Kc B"), Sp_ring=(Sp_ring, "D Kc B"),
                 Weight=(Weight, "D Kc"), Bias=(Bias, "D"), S=(S, "Dk Dv Hv B"),
                 Sp=(Sp, "Dk Dv Hv B"), O=(O, "Dv Hv B"), A_log=(A_log, "Hv"),
                 DtBias=(DtBias, "Hv"), NormWeight=(NormWeight, "Dv"))
    D, Kc = dims["D"], dims["Kc"]
    if dims["B"] != N or (dims["Dk"], dims["Dv"], dims["Hv"]) != (Dk, Dv, Hv):
        raise DimensionMismatch(f"linear_deltanet_decode: B {dims['B']} vs N {N}, state "
                                f"({dims['Dk']}, {dims['Dv']}, {dims['Hv']}) vs ({Dk}, {Dv}, {Hv})")
    for t, n in ((W, "W"), (y, "y"), (Y, "Y"), (S_ring, "S_ring"), (Sp_ring, "S_ring′"),
                 (Weight, "Weight"), (Bias, "Bias"), (O, "O"), (NormWeight, "NormWeight")):
        _need(t, torch.bfloat16, n)
    for t, n in ((A_log, "A_log"), (DtBias, "DtBias"), (S, "S"), (Sp, "S′")):
        _need(t, torch.float32, n)
    _need_contig(S, "S")
    _need_contig(Sp, "S′")
    if S_ring.stride() != Sp_ring.stride():
        raise ArgumentError("S_ring and S_ring′ must share strides")
    if O.dim() == 3 and O.stride(1) != O.shape[2]:
        raise ArgumentError("O: heads must be contiguous")
    need = linear_causal_conv1d_workspace_bytes(x, W, y)
    if workspace is None:
        workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=x.device)
    call("vm_linear_deltanet_decode", _p(O), _st(O, 0, Hv * Dv), _p(y), ldy, _p(Y),
         _st(Y, 0, D), _p(x), ldx, _p(W), W.stride(0), M, K, _p(S_ring), _p(Sp_ring),
         _st(S_ring, 1, D), _st(S_ring, 0, Kc * D), _p(Weight), _st(Weight, 0, D), _p(Bias), Kc,
         _p(A_log), _p(DtBias), _p(NormWeight), _p(S), _p(Sp), Dk, Dv, Hk, Hv, N, float(eps),
         _p(workspace), workspace.numel(), _stream())
    return outs


def causal_conv1d(X, S, Weight, Bias=None, *, sigma=None, Sp=None) -> dict:
    """Allocating causal_conv1d (causal_conv1d.jl:63-66): {"Y", "Sp"}; pass Sp=S for
    the in-place ring (the reference's output_override, qwen35.jl:222-223)."""
    Y = torch.empty((X.shape[0], X.shape[-1]), dtype=X.dtype, device=X.device)
    return causal_conv1d_({"Y": Y, "Sp": torch.empty_like(S) if Sp is None else Sp}, X, S,
                          Weight, Bias, sigma=sigma)


def causal_conv1d_sequence_(outs, X, Weight, Bias=None, *, sigma=None, Sp=None, S=None):
    """causal_conv1d_sequence!((; Y), X, Weight, Bias; σ, S′) — causal_conv1d.jl:130-149.
    X, Y :: (D, T, B) (torch (B, T, D), token rows may be strided); Sp :: (D, K, B)
    receives the ring a decode step continues from. S (not in the reference's
    signature): a prefix's ring whose columns 2..K are the left context, the
    suffix prefill of qwen35.jl:333-344 without its copy; None = zeros."""
    Y = _out(outs, "Y")
    dims = sizes(Y=(Y, "D T B"), X=(X, "D T B"), Weight=(Weight, "D K"), Bias=(Bias, "D"),
                 Sp=(Sp, "D K B"), S=(S, "D K B"))
    D, T, B, K = dims["D"], dims["T"], dims["B"], dims["K"]
    for t, n in ((Y, "Y"), (X, "X"), (Weight, "Weight"), (Bias, "Bias"), (Sp, "S′"), (S, "S")):
        _need(t, torch.bfloat16, n)
    ring = Sp if Sp is not None else S
    if Sp is not None and S is not None and S.stride() != Sp.stride():
        raise ArgumentError("S and S′ must share strides")
    s_cs = _st(ring, 1, D) if ring is not None else D
    s_sb = _st(ring, 0, K * D) if ring is not None else K * D
    call("vm_causal_conv1d_sequence", _p(Y), _st(Y, 1, D), _st(Y, 0, T * D), _p(X),
         _st(X, 1, D), _st(X, 0, T * D), _p(Weight), _st(Weight, 0, D), _p(Bias), _p(S), _p(Sp),
         s_cs, s_sb, D, K, T, B, _act(sigma), _stream())
    return outs


def causal_conv1d_sequence(X, Weight, Bias=None, **kw) -> dict:
    """Allocating causal_conv1d_sequence (causal_conv1d.jl:151-154): {"Y"}."""
    Y = torch.empty(X.shape, dtype=X.dtype, device=X.device)
    return causal_conv1d_sequence_({"Y": Y}, X, Weight, Bias, **kw)


def fused_deltanet_decode_(outs, Q_raw, K_raw, V, Alpha, BetaRaw, Z, A_log, DtBias, NormWeight,
                           S, *, eps=1e-6):
    """fused_deltanet_decode!((; O, S′), Q_raw, K_raw, V, Alpha, BetaRaw, Z, A_log,
    DtBias, NormWeight, S; eps) — src/kernels/deltanet_fused.jl:109-141. Q_raw,
    K_raw :: (Dk, Hk, B), V, Z, O :: (Dv, Hv, B), Alpha, BetaRaw :: (Hv, B) bf16
    (torch reversed; the per-sequence dim may be strided, e.g. views of the
    projection); A_log, DtBias :: (Hv,) fp32; NormWeight :: (Dv,) bf16; S, S′ ::
    (Dk, Dv, Hv, B) fp32 contiguous (S′ may be S)."""
    O, Sp = _out(outs, "O"), _out(outs, "Sp")
    dims = sizes(O=(O, "Dv Hv B"), Q_raw=(Q_raw, "Dk Hk B"), K_raw=(K_raw, "Dk Hk B"),
                 V=(V, "Dv Hv B"), Alpha=(Alpha, "Hv B"), BetaRaw=(BetaRaw, "Hv B"),
                 Z=(Z, "Dv Hv B"), A_log=(A_log, "Hv"), DtBias=(DtBias, "Hv"),
                 NormWeight=(NormWeight, "Dv"), S=(S, "Dk Dv Hv B"), Sp=(Sp, "Dk Dv Hv B"))
    Dk, Dv, Hk, Hv, B = (dims[n] for n in ("Dk", "Dv", "Hk", "Hv", "B"))
    if Hv % Hk:
        raise DimensionMismatch(f"Value heads ({Hv}) is not a multiple of qk heads ({Hk})")
    for t, n in ((O, "O"), (Q_raw, "Q_raw"), (K_raw, "K_raw"), (V, "V"), (Alpha, "Alpha"),
                 (BetaRaw, "BetaRaw"), (Z, "Z"), (NormWeight, "NormWeight")):
        _need(t, torch.bfloat16, n)
        if t.dim() == 3 and t.stride(1) != t.shape[2]:
            raise ArgumentError(f"{n}: heads must be contiguous")
    for t, n in ((A_log, "A_log"), (DtBias, "DtBias"), (S, "S"), (Sp, "S′")):
        _need(t, torch.float32, n)
    _need_contig(S, "S")
    _need_contig(Sp, "S′")
    call("vm_fused_deltanet_decode", _p(O), _st(O, 0, Hv * Dv), _p(Q_raw), _st(Q_raw, 0, Hk * Dk),
         _p(K_raw), _st(K_raw, 0, Hk * Dk), _p(V), _st(V, 0, Hv * Dv), _p(Alpha),
         _st(Alpha, 0, Hv), _p(BetaRaw), _st(BetaRaw, 0, Hv), _p(Z), _st(Z, 0, Hv * Dv),
         _p(A_log), _p(DtBias), _p(NormWeight), _p(S), _p(Sp), Dk, Dv, Hk, Hv, B, float(eps),
         _stream())
    return outs


def fused_deltanet_decode(Q_raw, K_raw, V, Alpha, BetaRaw, Z, A_log, DtBias, NormWeight, S, *,
                          eps=1e-6, Sp=None) -> dict:
    """Allocating fused_deltanet_decode (deltanet_fused.jl:143-147): {"O", "Sp"}; pass
    Sp=S for the in-place state (qwen35.jl:227-229)."""
    O = torch.empty(V.shape, dtype=V.dtype, device=V.device)
    return fused_deltanet_decode_({"O": O, "Sp": torch.empty_like(S) if Sp is None else Sp},
                                  Q_raw, K_raw, V, Alpha, BetaRaw, Z, A_log, DtBias, NormWeight,
                                  S, eps=eps)


def _deltanet_fp32(name, outs, Q, K, V, Beta, Gate, S, spec_qk, spec_v, spec_g):
    O, Sp = _out(outs, "O"), _out(outs, "Sp")
    dims = sizes(O=(O, spec_v), Q=(Q, spec_qk), K=(K, spec_qk), V=(V, spec_v),
                 Beta=(Beta, spec_g), Gate=(Gate, spec_g), S=(S, "Dk Dv Hv B"),
                 Sp=(Sp, "Dk Dv Hv B"))
    Hk, Hv = dims["Hk"], dims["Hv"]
    if Hv % Hk:
        raise DimensionMismatch(f"value heads ({Hv}) is not a multiple of key heads ({Hk})")
    for t, n in ((O, "O"), (Q, "Q"), (K, "K"), (V, "V"), (Beta, "Beta"), (Gate, "Gate"),
                 (S, "S"), (Sp, "S′")):
        _need(t, torch.float32, n)
        _need_contig(t, n)
    return O, Sp, dims


def deltanet_recurrent_decode_(outs, Q, K, V, Beta, Gate, S):
    """deltanet_recurrent_decode!((; O, S′), Q, K, V, Beta, Gate, S) —
    src/kernels/deltanet_recurrent.jl:72-95, fp32: Q, K :: (Dk, Hk, B), V, O ::
    (Dv, Hv, B), Beta, Gate :: (Hv, B) (decay = exp(Gate)), S, S′ :: (Dk, Dv, Hv, B)."""
    O, Sp, d = _deltanet_fp32("deltanet_recurrent_decode", outs, Q, K, V, Beta, Gate, S,
                              "Dk Hk B", "Dv Hv B", "Hv B")
    call("vm_deltanet_recurrent_decode", _p(O), _p(Q), _p(K), _p(V), _p(Beta), _p(Gate), _p(S),
         _p(Sp), d["Dk"], d["Dv"], d["Hk"], d["Hv"], d["B"], _stream())
    return outs


def deltanet_recurrent_decode(Q, K, V, Beta, Gate, S, *, Sp=None) -> dict:
    """Allocating deltanet_recurrent_decode (deltanet_recurrent.jl:97-100)."""
    O = torch.empty(V.shape, dtype=torch.float32, device=V.device)
    return deltanet_recurrent_decode_({"O": O, "Sp": torch.empty_like(S) if Sp is None else Sp},
                                      Q, K, V, Beta, Gate, S)


def deltanet_sequence_(outs, Q, K, V, Beta, Gate, S):
    """deltanet_sequence!((; O, S′), Q, K, V, Beta, Gate, S) — deltanet_recurrent.jl:
    174-198, fp32: Q, K :: (Dk, T, Hk, B), V, O :: (Dv, T, Hv, B), Beta, Gate ::
    (Hv, T, B), S, S′ :: (Dk, Dv, Hv, B) (S′ may be S, qwen35.jl:358)."""
    O, Sp, d = _deltanet_fp32("deltanet_sequence", outs, Q, K, V, Beta, Gate, S,
                              "Dk T Hk B", "Dv T Hv B", "Hv T B")
    call("vm_deltanet_sequence", _p(O), _p(Q), _p(K), _p(V), _p(Beta), _p(Gate), _p(S), _p(Sp),
         d["Dk"], d["Dv"], d["T"], d["Hk"], d["Hv"], d["B"], _stream())
    return outs


def deltanet_sequence_workspace_bytes(T: int, Hv: int, B: int) -> int:
    """Workspace of deltanet_sequence_chunked_ (about 197 KB per 64-token chunk per
    value head and sequence: the scan's operands, each chunk's start state and
    its delta)."""
    return int(_lib.load().vm_deltanet_sequence_workspace_bytes(T, Hv, B))


def deltanet_sequence_chunked_(outs, Q, K, V, Beta, Gate, S, *, workspace=None):
    """deltanet_sequence! computed per 64-token chunk (a triangular solve and fp32
    MFMA products, the chunks' state carried by one scan): the same operator and
    arguments as deltanet_sequence_ (deltanet_recurrent.jl:174-198), results
    equal to fp32 rounding. workspace: a uint8 GPU tensor of at least
    deltanet_sequence_workspace_bytes(T, Hv, B), 256-byte aligned (allocated
    here when None)."""
    O, Sp, d = _deltanet_fp32("deltanet_sequence", outs, Q, K, V, Beta, Gate, S,
                              "Dk T Hk B", "Dv T Hv B", "Hv T B")
    need = deltanet_sequence_workspace_bytes(d["T"], d["Hv"], d["B"])
    if workspace is None:
        workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=Q.device)
    call("vm_deltanet_sequence_chunked", _p(O), _p(Q), _p(K), _p(V), _p(Beta), _p(Gate), _p(S),
         _p(Sp), d["Dk"], d["Dv"], d["T"], d["Hk"], d["Hv"], d["B"], _p(workspace),
         workspace.numel(), _stream())
    return outs


def deltanet_sequence(Q, K, V, Beta, Gate, S, *, Sp=None) -> dict:
    """Allocating deltanet_sequence (deltanet_recurrent.jl:200-203)."""
    O = torch.empty(V.shape, dtype=torch.float32, device=V.device)
    return deltanet_sequence_({"O": O, "Sp": torch.empty_like(S) if Sp is None else Sp}, Q, K, V,
                              Beta, Gate, S)


def deltanet_sequence_chunked_gated_norm_(outs, Z, NormWeight, Q, K, V, Beta, Gate, S, *, eps,
                                          workspace=None):
    """forward(::DeltaNetLayer)'s recurrence and gated norm in one call
    (src/llm/qwen35.jl:357-364): deltanet_sequence! in its chunked form with
    y = O rstd NormWeight silu(Z) applied in the output kernel, so O never
    reaches memory. outs "Y" :: (Dv, Hv, T, B) bf16 (torch (B, T, Hv, Dv), token
    and sequence dims may be strided, heads contiguous), "Sp" the state out
    (may be S); Z like Y; Q, K, V, Beta, Gate, S as deltanet_sequence_chunked_."""
    Y, Sp = _out(outs, "Y"), _out(outs, "Sp")
    dims = sizes(Y=(Y, "Dv Hv T B"), Z=(Z, "Dv Hv T B"), NormWeight=(NormWeight, "Dv"),
                 Q=(Q, "Dk T Hk B"), K=(K, "Dk T Hk B"), V=(V, "Dv T Hv B"),
                 Beta=(Beta, "Hv T B"), Gate=(Gate, "Hv T B"), S=(S, "Dk Dv Hv B"),
                 Sp=(Sp, "Dk Dv Hv B"))
    Dk, Dv, Hk, Hv, T, B = (dims[n] for n in ("Dk", "Dv", "Hk", "Hv", "T", "B"))
    if Hv % Hk:
        raise DimensionMismatch(f"value heads ({Hv}) is not a multiple of key heads ({Hk})")
    for t, n in ((Q, "Q"), (K, "K"), (V, "V"), (Beta, "Beta"), (Gate, "Gate"), (S, "S"),
                 (Sp, "S′")):
        _need(t, torch.float32, n)
        _need_contig(t, n)
    for t, n in ((Z, "Z"), (Y, "Y"), (NormWeight, "NormWeight")):
        _need(t, torch.bfloat16, n)
        if t.dim() == 4 and t.stride(2) != Dv:
            raise ArgumentError(f"{n}: heads must be contiguous")
    need = deltanet_sequence_workspace_bytes(T, Hv, B)
    if workspace is None:
        workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=Q.device)
    call("vm_deltanet_sequence_chunked_gated_norm", _p(Y), _st(Y, 1, Hv * Dv),
         _st(Y, 0, T * Hv * Dv), _p(Z), _st(Z, 1, Hv * Dv), _st(Z, 0, T * Hv * Dv),
         _p(NormWeight), float(eps), _p(Q), _p(K), _p(V), _p(Beta), _p(Gate), _p(S), _p(Sp), Dk,
         Dv, T, Hk, Hv, B, _p(workspace), workspace.numel(), _stream())
    return outs


def deltanet_prefill_prep_(outs, CV, AB, A_log, DtBias, *, Dk, Dv, Hk, Hv):
    """The prefill's inputs to deltanet_sequence! (src/llm/qwen35.jl:347-356): CV ::
    (2 Hk Dk + Hv Dv, T, B) conv output, AB :: (2 Hv, T, B) (alpha | beta), bf16
    (torch (B, T, n), token rows may be strided) -> outs "Q", "K" (Dk, T, Hk, B),
    "V" (Dv, T, Hv, B), "Beta", "Gate" (Hv, T, B), fp32 contiguous."""
    n = 2 * Hk * Dk + Hv * Dv
    dims = sizes(CV=(CV, f"{n} T B"), AB=(AB, f"{2 * Hv} T B"), A_log=(A_log, f"{Hv}"),
                 DtBias=(DtBias, f"{Hv}"), Q=(outs["Q"], f"{Dk} T {Hk} B"),
                 K=(outs["K"], f"{Dk} T {Hk} B"), V=(outs["V"], f"{Dv} T {Hv} B"),
                 Beta=(outs["Beta"], f"{Hv} T B"), Gate=(outs["Gate"], f"{Hv} T B"))
    T, B = dims["T"], dims["B"]
    _need(CV, torch.bfloat16, "CV")
    _need(AB, torch.bfloat16, "AB")
    for n_ in ("Q", "K", "V", "Beta", "Gate"):
        _need(outs[n_], torch.float32, n_)
        _need_contig(outs[n_], n_)
    call("vm_deltanet_prefill_prep", _p(outs["Q"]), _p(outs["K"]), _p(outs["V"]),
         _p(outs["Beta"]), _p(outs["Gate"]), _p(CV), _st(CV, 1, n), _st(CV, 0, T * n), _p(AB),
         _st(AB, 1, 2 * Hv), _st(AB, 0, T * 2 * Hv), _p(A_log), _p(DtBias), Dk, Dv, Hk, Hv, T, B,
         _stream())
    return outs


def deltanet_conv_prep_(outs, X, Weight, AB, A_log, DtBias, Bias=None, *, Dk, Dv, Hk, Hv, Sp=None,
                        S=None):
    """The prefill's sequence conv and prep in one pass (src/llm/qwen35.jl:333-356):
    causal_conv1d_sequence_ of X (the q | k | v rows of the projection, (n, T, B),
    torch (B, T, n), token rows may be strided) with σ = silu, Weight (n, K), Bias,
    the ring S / S′ (Sp) as there, then deltanet_prefill_prep_ of its output and AB
    into outs "Q", "K", "V", "Beta", "Gate" — the same values bit for bit, the conv
    output never written."""
    n = 2 * Hk * Dk + Hv * Dv
    dims = sizes(X=(X, f"{n} T B"), Weight=(Weight, f"{n} K"), Bias=(Bias, f"{n}"),
                 Sp=(Sp, f"{n} K B"), S=(S, f"{n} K B"), AB=(AB, f"{2 * Hv} T B"),
                 A_log=(A_log, f"{Hv}"), DtBias=(DtBias, f"{Hv}"),
                 Q=(outs["Q"], f"{Dk} T {Hk} B"), K=(outs["K"], f"{Dk} T {Hk} B"),
                 V=(outs["V"], f"{Dv} T {Hv} B"), Beta=(outs["Beta"], f"{Hv} T B"),
                 Gate=(outs["Gate"], f"{Hv} T B"))
    T, B, K = dims["T"], dims["B"], dims["K"]
    for t, nm in ((X, "X"), (Weight, "Weight"), (Bias, "Bias"), (Sp, "S′"), (S, "S"), (AB, "AB")):
        _need(t, torch.bfloat16, nm)
    for n_ in ("Q", "K", "V", "Beta", "Gate"):
        _need(outs[n_], torch.float32, n_)
        _need_contig(outs[n_], n_)
    ring = Sp if Sp is not None else S
    if Sp is not None and S is not None and S.stride() != Sp.stride():
        raise ArgumentError("S and S′ must share strides")
    s_cs = _st(ring, 1, n) if ring is not None else n
    s_sb = _st(ring, 0, K * n) if ring is not None else K * n
    call("vm_deltanet_conv_prep", _p(outs["Q"]), _p(outs["K"]), _p(outs["V"]), _p(outs["Beta"]),
         _p(outs["Gate"]), _p(X), _st(X, 1, n), _st(X, 0, T * n), _p(Weight), _st(Weight, 0, n),
         _p(Bias), _p(S), _p(Sp), s_cs, s_sb, K, _p(AB), _st(AB, 1, 2 * Hv),
         _st(AB, 0, T * 2 * Hv), _p(A_log), _p(DtBias), Dk, Dv, Hk, Hv, T, B, _stream())
    return outs


def gated_rms_norm_(Y, O, Z, NormWeight, *, eps):
    """The prefill's gated RMSNorm + z gate (src/llm/qwen35.jl:360-364): O ::
    (Dv, T, Hv, B) fp32, Z :: (Dv, Hv, T, B) bf16 (torch (B, T, Hv, Dv), token and
    sequence dims may be strided) -> Y :: (Dv, Hv, T, B) bf16 = O rstd NormWeight
    silu(Z), the out projection's input."""
    dims = sizes(O=(O, "Dv T Hv B"), Z=(Z, "Dv Hv T B"), Y=(Y, "Dv Hv T B"),
                 NormWeight=(NormWeight, "Dv"))
    Dv, Hv, T, B = (dims[n] for n in ("Dv", "Hv", "T", "B"))
    _need(O, torch.float32, "O")
    _need_contig(O, "O")
    for t, n in ((Z, "Z"), (Y, "Y"), (NormWeight, "NormWeight")):
        _need(t, torch.bfloat16, n)
        if t.dim() == 4 and t.stride(2) != Dv:
            raise ArgumentError(f"{n}: heads must be contiguous")
    call("vm_gated_rms_norm", _p(Y), _st(Y, 1, Hv * Dv), _st(Y, 0, T * Hv * Dv), _p(O), _p(Z),
         _st(Z, 1, Hv * Dv), _st(Z, 0, T * Hv * Dv), _p(NormWeight), Dv, Hv, T, B, float(eps),
         _stream())
    return Y


def fill_normal_(X, seed: int, *, scale: float = 1.0, shift: float = 0.0):
    """Fill a contiguous bf16 GPU tensor with the seeded N(0,1) synthetic stream
    (SplitMix64 + Box-Muller, the generator the CPU tests use)."""
    _need(X, torch.bfloat16, "X")
    _need_contig(X, "X")
    call("vm_fill_normal_bf16", _p(X), X.numel(), int(seed) & (2 ** 64 - 1), float(scale),
         float(shift), _stream())
    return X
