"""The C ABI library (CPU-side checks: no kernel is launched here).

- libvallmo_attn.so loads and exports every entry point include/vallmo_attn.h
  declares, and the Python binding types exactly that set;
- argument/shape validation runs on the host before any HIP call and reports
  the reference's error semantics (DimensionMismatch for H % Hk != 0,
  src/kernels/attention.jl:110-111; unsupported head_dim; scratch size).
"""
from __future__ import annotations

import ctypes
import re
import subprocess

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "vallmo_attn.h"


def header_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = header_symbols()
    for must in ("vm_gated_attn_decode", "vm_gated_attn_prefill", "vm_attention_fwd",
                 "vm_decode_attention", "vm_qnorm_rope", "vm_knorm_rope_append",
                 "vm_rope_tables", "vm_sigmoid_gate", "vm_advance_positions",
                 "vm_graph_begin_capture", "vm_last_error"):
        assert must in syms


def test_library_exports_every_declared_symbol(vm):
    lib = vm._lib.load()
    out = subprocess.run(["nm", "-D", "--defined-only", str(vm.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (vm_[a-z0-9_]+)$", out, flags=re.M))
    for s in header_symbols():
        assert s in exported, f"{s} declared in vallmo_attn.h but not exported"
        assert hasattr(lib, s)
    assert set(vm.EXPORTED) == set(header_symbols())


FAKE = 0x10000  # an aligned, never-dereferenced address: validation fails first


def _p(x):
    return ctypes.c_void_p(x)


def test_attention_rejects_gqa_mismatch(vm):
    lib = vm._lib.load()
    rc = lib.vm_attention_fwd(_p(FAKE), 256, 256 * 8, 256 * 8 * 16, _p(FAKE), 256, 256 * 8,
                              256 * 8 * 16, _p(FAKE), 256, 256 * 8, 256 * 8 * 3, _p(FAKE), 256,
                              256 * 8, 256 * 8 * 3, None, None, 1, 16, 3, 256, 256, 8, 8, 1, None)
    assert rc == vm._lib.VM_E_DIM
    assert lib.vm_last_error().decode() == \
        "Attention heads (16) is not a multiple of key-value heads (3)"
    with pytest.raises(vm.DimensionMismatch):
        vm._lib.check(rc, "attention")


def test_unsupported_head_dim(vm):
    """Head dims are powers of two from 16 to 512 (qknorm_rope_append.jl:108);
    the operators reject others before any launch."""
    lib = vm._lib.load()
    rc = lib.vm_attention_fwd(_p(FAKE), 96, 96, 96, _p(FAKE), 96, 96, 96, _p(FAKE), 96, 96, 96,
                              _p(FAKE), 96, 96, 96, None, None, 1, 16, 4, 96, 96, 8, 8, 1, None)
    assert rc == vm._lib.VM_E_UNSUPPORTED
    assert "Dk = 96" in lib.vm_last_error().decode()
    rc = lib.vm_attention_fwd(_p(FAKE), 1024, 1024, 1024, _p(FAKE), 128, 128, 128, _p(FAKE), 128,
                              128, 128, _p(FAKE), 1024, 1024, 1024, None, None, 1, 16, 4, 128,
                              1024, 8, 8, 1, None)
    assert rc == vm._lib.VM_E_UNSUPPORTED
    assert "Dv = 1024" in lib.vm_last_error().decode()
    rc = lib.vm_qnorm_rope(_p(FAKE), 128, 128 * 16, _p(FAKE), _p(FAKE), _p(FAKE), 512, _p(FAKE), 1,
                           16, 128, 65, 1e-6, 1.0, None)
    assert rc == vm._lib.VM_E_ARG  # the rotary part 2 * 65 exceeds D = 128
    assert "HALF_ROT = 65" in lib.vm_last_error().decode()


def test_misaligned_pointer_rejected(vm):
    lib = vm._lib.load()
    rc = lib.vm_attention_fwd(_p(FAKE + 2), 256, 256, 256, _p(FAKE), 256, 256, 256, _p(FAKE), 256,
                              256, 256, _p(FAKE), 256, 256, 256, None, None, 1, 16, 4, 256, 256, 8,
                              8, 1, None)
    assert rc == vm._lib.VM_E_ARG
    assert "aligned" in lib.vm_last_error().decode()


def test_bad_stride_rejected(vm):
    lib = vm._lib.load()
    rc = lib.vm_attention_fwd(_p(FAKE), 256, 256, 256, _p(FAKE), 250, 256, 256, _p(FAKE), 256,
                              256, 256, _p(FAKE), 256, 256, 256, None, None, 1, 16, 4, 256, 256, 8,
                              8, 1, None)
    assert rc == vm._lib.VM_E_ARG


def test_decode_scratch_size_and_shortfall(vm):
    lib = vm._lib.load()
    # B=32, H=16, Hk=4: n_splits=8 gives a stream partition of 8*B*Hk waves; one
    # partial slot (G*256 + 2G floats) per wave plus one per (b, hk) segment, then
    # the partition snapshot (1 + 2B int32) in its own 256-byte blocks
    n = lib.vm_decode_scratch_bytes(32, 16, 4, 256, 32768, 8)
    slots = 8 * 32 * 4 + 32 * 4
    body = slots * 4 * (256 + 2) * 4
    assert n == -(-body // 256) * 256 + -(-(1 + 2 * 32) * 4 // 256) * 256
    assert lib.vm_decode_scratch_bytes(1, 16, 3, 256, 512, 0) == 0  # invalid GQA -> 0
    rc = lib.vm_decode_attention(_p(FAKE), 256, 4096, _p(FAKE), 256, 4096, _p(FAKE), 256,
                                 256 * 512, 256 * 512 * 4, _p(FAKE), 256, 256 * 512,
                                 256 * 512 * 4, 512, _p(FAKE), 1, 16, 4, 256, 256, 0, _p(FAKE), 64,
                                 None)
    assert rc == vm._lib.VM_E_SCRATCH
    assert "scratch" in lib.vm_last_error().decode()


def test_generic_decode_scratch(vm):
    """Shapes outside the tuned decode (here Dv = 128, a group of 16) size one
    (Dv + 2)-float partial row per split, sequence and head: n_splits per (b,
    kv head) as given, or about four workgroups per CU for 0 (at least 128 keys
    per split); a short scratch is refused before any launch."""
    lib = vm._lib.load()
    assert lib.vm_decode_scratch_bytes(2, 16, 1, 128, 4096, 8) == -(-8 * 2 * 16 * 130 * 4 // 256) * 256
    # n_splits = 0: 1024 / (B Hk) = 512 splits' worth, capped at ctx / 128 = 32 splits
    assert lib.vm_decode_scratch_bytes(2, 16, 1, 128, 4096, 0) == -(-32 * 2 * 16 * 130 * 4 // 256) * 256
    assert lib.vm_decode_scratch_bytes(1, 16, 4, 96, 512, 0) == 0  # not a power of two
    rc = lib.vm_decode_attention(_p(FAKE), 128, 2048, _p(FAKE), 128, 2048, _p(FAKE), 128,
                                 128 * 512, 128 * 512, _p(FAKE), 128, 128 * 512, 128 * 512, 512,
                                 _p(FAKE), 1, 16, 1, 128, 128, 0, _p(FAKE), 64, None)
    assert rc == vm._lib.VM_E_SCRATCH


def test_decode_rejects_unsupported_head_dim(vm):
    lib = vm._lib.load()
    rc = lib.vm_decode_attention(_p(FAKE), 1024, 4096, _p(FAKE), 1024, 4096, _p(FAKE), 1024,
                                 1024 * 512, 1024 * 512, _p(FAKE), 1024, 1024 * 512, 1024 * 512,
                                 512, _p(FAKE), 1, 16, 1, 1024, 1024, 0, _p(FAKE), 1 << 30, None)
    assert rc == vm._lib.VM_E_UNSUPPORTED


def test_fused_prefill_checks_qkv_stride(vm):
    lib = vm._lib.load()
    # token stride smaller than the 40 packed slots of 256
    rc = lib.vm_gated_attn_prefill(_p(FAKE), 4096, 4096 * 8, _p(FAKE), 256 * 39, 256 * 39 * 8,
                                   _p(FAKE), _p(FAKE), 256, 256 * 64, 256 * 64 * 4, 64,
                                   _p(FAKE), _p(FAKE), _p(FAKE), _p(FAKE), None, None, 1, 8,
                                   16, 4, 256, 32, 1e-6, 1.0, _p(FAKE), 1 << 30, None)
    assert rc == vm._lib.VM_E_DIM


def test_fused_prefill_checks_scratch(vm):
    lib = vm._lib.load()
    need = lib.vm_prefill_scratch_bytes(1, 4, 256, 64)
    assert need == 1 * 4 * 2 * 32 * 256 * 2  # one 16-KB V^T tile per 32 keys per (b, hk)
    assert lib.vm_prefill_scratch_bytes(1, 4, 128, 64) == 0  # unsupported head_dim
    rc = lib.vm_gated_attn_prefill(_p(FAKE), 4096, 4096 * 8, _p(FAKE), 256 * 40, 256 * 40 * 8,
                                   _p(FAKE), _p(FAKE), 256, 256 * 64, 256 * 64 * 4, 64,
                                   _p(FAKE), _p(FAKE), _p(FAKE), _p(FAKE), None, None, 1, 8,
                                   16, 4, 256, 32, 1e-6, 1.0, _p(FAKE), need - 1, None)
    assert rc == vm._lib.VM_E_SCRATCH
    assert "vm_prefill_scratch_bytes" in lib.vm_last_error().decode()


def test_sizes_contract_messages(vm):
    import torch
    q = torch.empty(2, 16, 256)
    k = torch.empty(2, 4, 100, 128)
    with pytest.raises(vm.DimensionMismatch) as e:
        vm.sizes(Q=(q, "Dqk Hq B"), K=(k, "Dqk Lkv Hkv B"))
    assert str(e.value) == "size(K, 1) = 128 does not match Dqk = 256 (= size(Q, 1))"
    with pytest.raises(vm.DimensionMismatch) as e:
        vm.sizes(Q=(q, "Dqk Hq"))
    assert "Q has 3 dimensions, expected 2" in str(e.value)
    d = vm.sizes(Q=(q, "Dqk Hq B"), X=(None, "Dqk"), R=(torch.empty(16), "Hq"))
    assert d == {"Dqk": 256, "Hq": 16, "B": 2}
    with pytest.raises(vm.DimensionMismatch):
        vm.sizes(R=(torch.empty(3, 4), "4 3"), S=(torch.empty(5), "4"))


def test_noalloc_decode_rejects_steps_beyond_its_workspace(vm):
    """vm_gated_attn_decode_noalloc serves steps whose workspace fits its static
    16 MiB array and refuses larger ones with VM_E_SCRATCH, before any HIP call."""
    lib = vm._lib.load()
    B, Hq, Hk, ctx, n_splits = 1000, 16, 4, 4096, 8
    need = lib.vm_decode_scratch_bytes(B, Hq, Hk, 256, ctx, n_splits)
    assert need > (16 << 20)
    rc = lib.vm_gated_attn_decode_noalloc(_p(FAKE), 256 * Hq, _p(FAKE), 256 * 40, _p(FAKE),
                                          _p(FAKE), 256, 256 * ctx, 256 * ctx * Hk, ctx,
                                          _p(FAKE), _p(FAKE), _p(FAKE), _p(FAKE), _p(FAKE), 0, B,
                                          Hq, Hk, 256, 32, 1e-6, 1.0, n_splits, None)
    assert rc == vm._lib.VM_E_SCRATCH
    msg = lib.vm_last_error().decode()
    assert "static workspace" in msg and str(need) in msg
