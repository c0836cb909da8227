"""ctypes binding of libvallmo_attn.so (include/vallmo_attn.h).

The library is built in-tree (``csrc/libvallmo_attn.so``). There is no fallback:
if it is missing, importing the operators raises, so no CPU or PyTorch path can
stand in for the HIP kernels.

Status codes map onto the reference's exceptions: VM_E_DIM ->
DimensionMismatch (src/sizes.jl:3-22, src/kernels/attention.jl:110-111),
VM_E_ARG -> ArgumentError, VM_E_UNSUPPORTED -> UnsupportedShape, VM_E_SCRATCH ->
ArgumentError, > 0 -> HIPError (a hipError_t).
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "csrc" / "libvallmo_attn.so"

VM_E_ARG, VM_E_DIM, VM_E_UNSUPPORTED, VM_E_SCRATCH = -1, -2, -3, -4
# kernel classes of vm_profile_read
(VM_K_ROWS, VM_K_DECODE_SPLIT, VM_K_DECODE_COMBINE, VM_K_PREFILL, VM_K_ADVANCE, VM_K_LM_HEAD,
 VM_K_DELTANET, VM_K_CONV) = range(8)


class DimensionMismatch(ValueError):
    """Non-conforming extents (Julia's Base.DimensionMismatch)."""


class ArgumentError(ValueError):
    """Invalid argument (Julia's Base.ArgumentError)."""


class BoundsError(IndexError):
    """Out-of-range index (Julia's Base.BoundsError)."""


class UnsupportedShape(ArgumentError):
    """A shape the compiled kernels do not cover (e.g. head_dim != 256)."""


class HIPError(RuntimeError):
    """A HIP runtime error passed through by the library."""


_c_i = ctypes.c_int
_c_i64 = ctypes.c_int64
_c_f = ctypes.c_float
_c_d = ctypes.c_double
_c_sz = ctypes.c_size_t
_c_u64 = ctypes.c_uint64
_p = ctypes.c_void_p

# name -> (restype, argtypes); every pointer (device or stream) is a void*.
_SIGS = {
    "vm_last_error": (ctypes.c_char_p, []),
    "vm_abi_version": (_c_i, []),
    "vm_profile_enable": (_c_i, [_c_i]),
    "vm_profile_read": (_c_i, [_c_i, ctypes.POINTER(_c_i), ctypes.POINTER(_c_d)]),
    "vm_profile_select": (_c_i, [ctypes.c_uint]),
    "vm_malloc": (_c_i, [ctypes.POINTER(_p), _c_sz]),
    "vm_free": (_c_i, [_p]),
    "vm_memcpy_h2d": (_c_i, [_p, _p, _c_sz, _p]),
    "vm_memcpy_d2h": (_c_i, [_p, _p, _c_sz, _p]),
    "vm_memcpy_d2d": (_c_i, [_p, _p, _c_sz, _p]),
    "vm_memset": (_c_i, [_p, _c_i, _c_sz, _p]),
    "vm_stream_create": (_c_i, [ctypes.POINTER(_p)]),
    "vm_stream_destroy": (_c_i, [_p]),
    "vm_stream_sync": (_c_i, [_p]),
    "vm_device_sync": (_c_i, []),
    "vm_event_create": (_c_i, [ctypes.POINTER(_p)]),
    "vm_event_destroy": (_c_i, [_p]),
    "vm_event_record": (_c_i, [_p, _p]),
    "vm_event_elapsed_ms": (_c_i, [ctypes.POINTER(_c_f), _p, _p]),
    "vm_graph_begin_capture": (_c_i, [_p]),
    "vm_graph_end_capture": (_c_i, [_p, ctypes.POINTER(_p)]),
    "vm_graph_launch": (_c_i, [_p, _p]),
    "vm_graph_destroy": (_c_i, [_p]),
    "vm_rope_tables": (_c_i, [_p, _p, _c_i, _c_i64, _c_d, _p]),
    "vm_qnorm_rope": (_c_i, [_p, _c_i64, _c_i64, _p, _p, _p, _c_i64, _p,
                             _c_i, _c_i, _c_i, _c_i, _c_f, _c_f, _p]),
    "vm_knorm_rope_append": (_c_i, [_p, _c_i64, _c_i64, _c_i64, _p, _c_i64, _c_i64, _c_i64,
                                    _c_i64, _p, _c_i64, _c_i64, _p, _c_i64, _c_i64, _p, _p, _p,
                                    _p, _c_i, _c_i, _c_i, _c_i, _c_i, _c_f, _c_f, _p]),
    "vm_decode_scratch_bytes": (_c_sz, [_c_i, _c_i, _c_i, _c_i, _c_i64, _c_i]),
    "vm_decode_attention": (_c_i, [_p, _c_i64, _c_i64, _p, _c_i64, _c_i64, _p, _c_i64, _c_i64,
                                   _c_i64, _p, _c_i64, _c_i64, _c_i64, _c_i64, _p, _c_i, _c_i,
                                   _c_i, _c_i, _c_i, _c_i, _p, _c_sz, _p]),
    "vm_sigmoid_gate": (_c_i, [_p, _c_i64, _c_i64, _p, _c_i64, _c_i64, _c_i, _c_i, _c_i, _p]),
    "vm_gated_attn_decode": (_c_i, [_p, _c_i64, _p, _c_i64, _p, _p, _c_i64, _c_i64, _c_i64,
                                    _c_i64, _p, _p, _p, _p, _p, _c_i, _c_i, _c_i, _c_i, _c_i,
                                    _c_i, _c_f, _c_f, _c_i, _p, _c_sz, _p]),
    "vm_gated_attn_decode_noalloc": (_c_i, [_p, _c_i64, _p, _c_i64, _p, _p, _c_i64, _c_i64,
                                            _c_i64, _c_i64, _p, _p, _p, _p, _p, _c_i, _c_i, _c_i,
                                            _c_i, _c_i, _c_i, _c_f, _c_f, _c_i, _p]),
    "vm_advance_positions": (_c_i, [_p, _c_i, _p]),
    "vm_attention_fwd": (_c_i, [_p, _c_i64, _c_i64, _c_i64, _p, _c_i64, _c_i64, _c_i64, _p,
                                _c_i64, _c_i64, _c_i64, _p, _c_i64, _c_i64, _c_i64, _p, _p, _c_i,
                                _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _p]),
    "vm_prefill_kv_append": (_c_i, [_p, _p, _c_i64, _c_i64, _c_i64, _c_i64, _p, _c_i64, _c_i64,
                                    _p, _p, _p, _p, _p, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i,
                                    _c_f, _c_f, _p]),
    "vm_prefill_q_norm_rope": (_c_i, [_p, _c_i64, _c_i64, _c_i64, _p, _c_i64, _c_i64, _p, _p,
                                      _p, _p, _p, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_f,
                                      _c_f, _p]),
    "vm_prefill_scratch_bytes": (_c_sz, [_c_i, _c_i, _c_i, _c_i64]),
    "vm_gated_attn_prefill": (_c_i, [_p, _c_i64, _c_i64, _p, _c_i64, _c_i64, _p, _p, _c_i64,
                                     _c_i64, _c_i64, _c_i64, _p, _p, _p, _p, _p, _p, _c_i, _c_i,
                                     _c_i, _c_i, _c_i, _c_i, _c_f, _c_f, _p, _c_sz, _p]),
    "vm_gated_attn_prefill_staged": (_c_i, [_p, _c_i64, _c_i64, _p, _c_i64, _c_i64, _p, _p,
                                            _c_i64, _c_i64, _c_i64, _c_i64, _p, _p, _p, _p, _p,
                                            _p, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_f, _c_f,
                                            _p, _p, _c_sz, _p]),
    "vm_linear_workspace_bytes": (_c_sz, [_c_i, _c_i, _c_i, _c_i64, _c_i64, _c_i64]),
    "vm_linear_tune": (_c_i, [_c_i, _c_i, _c_i, _c_i64, _c_i64, _c_i64]),
    "vm_linear_plan_state": (_c_i, [_c_i, _c_i, _c_i, _c_i64, _c_i64, _c_i64]),
    "vm_linear": (_c_i, [_p, _c_i64, _p, _c_i64, _p, _c_i64, _c_i, _c_i, _c_i, _p, _c_sz, _p]),
    "vm_rms_norm": (_c_i, [_p, _c_i64, _p, _c_i64, _p, _c_i, _c_i, _c_f, _c_f, _p]),
    "vm_linear_causal_conv1d_workspace_bytes": (_c_sz, [_c_i, _c_i, _c_i, _c_i64, _c_i64, _c_i64]),
    "vm_linear_causal_conv1d": (_c_i, [_p, _c_i64, _p, _c_i64, _p, _c_i64, _c_i, _c_i, _c_i, _p,
                                       _c_i64, _p, _p, _c_i64, _c_i64, _p, _c_i64, _p, _c_i,
                                       _c_i, _c_i, _p, _c_sz, _p]),
    "vm_linear_deltanet_decode": (_c_i, [_p, _c_i64, _p, _c_i64, _p, _c_i64, _p, _c_i64, _p,
                                         _c_i64, _c_i, _c_i, _p, _p, _c_i64, _c_i64, _p, _c_i64,
                                         _p, _c_i, _p, _p, _p, _p, _p, _c_i, _c_i, _c_i, _c_i,
                                         _c_i, _c_f, _p, _c_sz, _p]),
    "vm_linear_silu_mul_workspace_bytes": (_c_sz, [_c_i, _c_i, _c_i, _c_i64, _c_i64]),
    "vm_linear_silu_mul": (_c_i, [_p, _c_i64, _p, _c_i64, _p, _c_i64, _c_i, _c_i, _c_i, _p, _c_sz,
                                  _p]),
    "vm_linear_add_rms_norm_workspace_bytes": (_c_sz, [_c_i, _c_i, _c_i, _c_i64, _c_i64]),
    "vm_linear_add_rms_norm": (_c_i, [_p, _c_i64, _p, _c_i64, _p, _c_i64, _p, _c_i64, _p, _c_i,
                                      _c_i, _c_i, _c_f, _c_f, _p, _c_sz, _p]),
    "vm_fused_add_rms_norm": (_c_i, [_p, _c_i64, _p, _c_i64, _p, _c_i64, _p, _c_i64, _p, _c_i,
                                     _c_i, _c_f, _c_f, _p]),
    "vm_silu_mul": (_c_i, [_p, _c_i64, _p, _c_i64, _c_i, _c_i, _p]),
    "vm_embed": (_c_i, [_p, _c_i64, _p, _c_i64, _p, _c_i, _c_i, _c_i, _p]),
    "vm_generation_advance": (_c_i, [_p, _p, _p, _p, _p, _c_i, _c_i, _p]),
    "vm_lm_head_argmax_scratch_bytes": (_c_sz, [_c_i, _c_i, _c_i]),
    "vm_lm_head_argmax": (_c_i, [_p, _p, _c_i64, _p, _c_i64, _c_i, _c_i, _c_i, _p, _c_sz, _p]),
    "vm_causal_conv1d": (_c_i, [_p, _c_i64, _p, _c_i64, _p, _p, _c_i64, _c_i64, _p, _c_i64, _p,
                                _c_i, _c_i, _c_i, _c_i, _p]),
    "vm_causal_conv1d_sequence": (_c_i, [_p, _c_i64, _c_i64, _p, _c_i64, _c_i64, _p, _c_i64, _p,
                                         _p, _p, _c_i64, _c_i64, _c_i, _c_i, _c_i, _c_i, _c_i,
                                         _p]),
    "vm_fused_deltanet_decode": (_c_i, [_p, _c_i64, _p, _c_i64, _p, _c_i64, _p, _c_i64, _p,
                                        _c_i64, _p, _c_i64, _p, _c_i64, _p, _p, _p, _p, _p, _c_i,
                                        _c_i, _c_i, _c_i, _c_i, _c_f, _p]),
    "vm_deltanet_recurrent_decode": (_c_i, [_p] * 8 + [_c_i] * 5 + [_p]),
    "vm_deltanet_sequence": (_c_i, [_p] * 8 + [_c_i] * 6 + [_p]),
    "vm_deltanet_sequence_workspace_bytes": (_c_sz, [_c_i, _c_i, _c_i]),
    "vm_deltanet_sequence_chunked": (_c_i, [_p] * 8 + [_c_i] * 6 + [_p, _c_sz, _p]),
    "vm_deltanet_sequence_chunked_gated_norm": (_c_i, [_p, _c_i64, _c_i64, _p, _c_i64, _c_i64, _p,
                                                        _c_f] + [_p] * 7 + [_c_i] * 6
                                                + [_p, _c_sz, _p]),
    "vm_deltanet_prefill_prep": (_c_i, [_p] * 5 + [_p, _c_i64, _c_i64, _p, _c_i64, _c_i64, _p, _p]
                                 + [_c_i] * 6 + [_p]),
    "vm_deltanet_conv_prep": (_c_i, [_p] * 5 + [_p, _c_i64, _c_i64, _p, _c_i64, _p, _p, _p, _c_i64,
                                      _c_i64, _c_i, _p, _c_i64, _c_i64, _p, _p]
                              + [_c_i] * 6 + [_p]),
    "vm_gated_rms_norm": (_c_i, [_p, _c_i64, _c_i64, _p, _p, _c_i64, _c_i64, _p, _c_i, _c_i,
                                 _c_i, _c_i, _c_f, _p]),
    "vm_fill_normal_bf16": (_c_i, [_p, _c_i64, _c_u64, _c_f, _c_f, _p]),
}

EXPORTED = tuple(_SIGS)

_lib = None


def load(path: Path | None = None):
    """Load and type the library; raises ImportError if it was not built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise ImportError(
            f"{p} is missing: build it with `make -C {p.parent}` (or __graft_entry__.build()); "
            "the gated-attention operators have no fallback path")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in _SIGS.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    if path is None:
        _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    """Raise the reference-style exception for a non-zero status."""
    if rc == 0:
        return
    msg = load().vm_last_error().decode(errors="replace")
    if rc == VM_E_DIM:
        raise DimensionMismatch(msg)
    if rc == VM_E_UNSUPPORTED:
        raise UnsupportedShape(msg)
    if rc in (VM_E_ARG, VM_E_SCRATCH):
        raise ArgumentError(msg)
    if rc > 0:
        raise HIPError(f"{what}: {msg} (hipError_t {rc})")
    raise RuntimeError(f"{what}: status {rc}: {msg}")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args), name)


def profile_enable(on: bool = True) -> None:
    call("vm_profile_enable", int(bool(on)))


def profile_select(*kernels: int) -> None:
    """Bracket only these kernel classes while profiling (none given: all)."""
    mask = 0xFFFFFFFF if not kernels else sum(1 << int(k) for k in set(kernels))
    call("vm_profile_select", mask)


def profile_read(kernel: int) -> tuple[int, float]:
    """(launch count, summed ms) of one kernel class since profile_enable(True)."""
    n, t = ctypes.c_int(), ctypes.c_double()
    call("vm_profile_read", int(kernel), ctypes.byref(n), ctypes.byref(t))
    return n.value, t.value
