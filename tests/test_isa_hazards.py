"""Hazards the compiler cannot see, checked on the compiled gfx950 ISA (CPU only).

The fused prefill kernel issues its LDS reads and its MFMAs from inline asm (the
lm head and the GEMVs of step.hip their LDS reads):
  * an asm output is taken to be ready at the asm statement, so the compiler may
    copy, spill or overwrite a load's destination before the data has landed;
  * the compiler inserts no wait states after an asm MFMA, so a VALU read of its
    result must be padded by the kernel itself.
Both would give wrong numbers with no error. These tests build the device ISA
with the library's own flags (``make _build/asm/<file>.s``) and check every
kernel by a data-flow pass over its basic blocks:
  1. no instruction reads or writes the destination of a pending load
     (global_load_dword*, ds_read*) before an s_waitcnt that covers it, counting
     every vector-memory / LDS operation in issue order;
  2. no instruction other than a dependent MFMA touches an MFMA's destination
     within 11 wait states of its issue (8-pass XDL write -> VALU read);
  3. the fused prefill drains its tile loads before each barrier after which it
     writes the LDS afresh (a pair's second item, the row-max re-prime).
The checks were validated against deliberately weakened builds (a vmcnt raised
by 8, a spill of a pending AGPR load) that they flag.
"""
from __future__ import annotations

import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "vallmo.jl_amd" / "csrc"

VM_OPS = ("global_load", "global_store", "buffer_load", "buffer_store", "scratch_load",
          "scratch_store", "global_atomic", "flat_")
LG_OPS = ("ds_", "s_load", "s_buffer_load")
MFMA_WAIT_STATES = 11


def build_asm(src: str) -> str:
    subprocess.run(["make", "-s", "-C", str(CSRC), f"_build/asm/{src}.s"], check=True,
                   stdout=subprocess.DEVNULL)
    return (CSRC / "_build" / "asm" / f"{src}.s").read_text()


def kernels(asm: str):
    """{symbol: [instruction lines]} for every kernel in the listing."""
    out, cur, name = {}, None, None
    for line in asm.split("\n"):
        m = re.match(r"^(_Z\w+):", line)
        if m and ".Lfunc_end" not in line:
            name, cur = m.group(1), []
            continue
        if cur is not None and line.startswith(".Lfunc_end"):
            out[name] = cur
            cur = None
            continue
        if cur is not None:
            cur.append(line.strip())
    return out


def regset(tok: str):
    m = re.match(r"([va])\[(\d+):(\d+)\]", tok)
    if m:
        return frozenset((m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1))
    m = re.match(r"([va])(\d+)$", tok)
    return frozenset({(m.group(1), int(m.group(2)))}) if m else frozenset()


def operands(line: str):
    line = line.split(";")[0].strip()
    parts = line.split(None, 1)
    if not parts:
        return "", []
    return parts[0], ([o.strip() for o in parts[1].split(",")] if len(parts) > 1 else [])


def step(state, line, report):
    """Transfer function. state = (pending loads, recent MFMA writes)."""
    pend, mf = state
    op, ops = operands(line)
    if not op or op.startswith("."):
        return state
    if op.startswith("s_waitcnt"):
        m = re.search(r"vmcnt\((\d+)\)", line)
        if m:
            k = int(m.group(1))
            pend = frozenset(p for p in pend if p[0] != "vm" or p[3] < k)
        m = re.search(r"lgkmcnt\((\d+)\)", line)
        if m:
            k = int(m.group(1))
            pend = frozenset(p for p in pend if p[0] != "lgkm" or p[3] < k)
        return pend, frozenset((r, w + 1) for r, w in mf if w + 1 < MFMA_WAIT_STATES)
    if op == "s_nop":
        n = int(ops[0], 0) + 1 if ops else 1
        return pend, frozenset((r, w + n) for r, w in mf if w + n < MFMA_WAIT_STATES)
    regs = [regset(o.split()[0]) for o in ops]
    dst = regs[0] if regs else frozenset()
    srcs = frozenset().union(*regs[1:]) if len(regs) > 1 else frozenset()
    if op.startswith(("global_load_lds", "global_store", "ds_write", "buffer_store", "scratch_store")):
        srcs, dst = frozenset().union(*regs) if regs else frozenset(), frozenset()
    is_load = (op.startswith("global_load_dword") and not op.startswith("global_load_lds")) \
        or op.startswith("ds_read")
    is_mfma = op.startswith("v_mfma")
    touched = srcs | dst
    for p in pend:
        if is_load and (p[1] & dst) and not (p[1] & srcs):
            continue  # a later load into the same registers replaces it
        if p[1] & touched:
            report.add(("load", line, p[2]))
    for r, w in mf:
        # a dependent MFMA accumulating into the same registers is interlocked
        if is_mfma and len(regs) > 3 and regs[3] == r and dst == r:
            continue
        if r & touched:
            report.add(("mfma", line, f"{w} wait states after an MFMA writing it"))
    kind = "vm" if op.startswith(VM_OPS) else "lgkm" if op.startswith(LG_OPS) else None
    if kind:
        pend = frozenset((p[0], p[1], p[2], min(p[3] + 1, 64)) if p[0] == kind else p for p in pend)
    if is_load:
        pend = frozenset(p for p in pend if not (p[1] & dst)) | {(kind, dst, line, 0)}
    mf = frozenset((r, w + 1) for r, w in mf if w + 1 < MFMA_WAIT_STATES and not (is_mfma and r == dst))
    if is_mfma:
        mf = mf | {(dst, 0)}
    return pend, mf


def check(body):
    labels = {}
    for n, l in enumerate(body):
        m = re.match(r"^(\.LBB\w+):", l)
        if m:
            labels[m.group(1)] = n
    empty = (frozenset(), frozenset())
    state_in, work, report = {0: empty}, [0], set()
    while work:
        n0 = work.pop()
        st, n = state_in[n0], n0
        while n < len(body):
            line = body[n]
            if n != n0 and re.match(r"^\.LBB\w+:", line):
                old = state_in.get(n, empty)
                new = (old[0] | st[0], old[1] | st[1])
                if n not in state_in or new != old:
                    state_in[n] = new
                    work.append(n)
                break
            st = step(st, line, report)
            op, ops = operands(line)
            if op.startswith("s_cbranch") or op == "s_branch":
                t = labels.get(ops[0]) if ops else None
                if t is not None:
                    old = state_in.get(t, empty)
                    new = (old[0] | st[0], old[1] | st[1])
                    if t not in state_in or new != old:
                        state_in[t] = new
                        work.append(t)
                if op == "s_branch":
                    break
            if op == "s_endpgm":
                break
            n += 1
    return sorted(report)


@pytest.fixture(scope="module")
def fused_asm():
    return build_asm("prefill_fused.hip")


def test_fused_prefill_kernels_present(fused_asm):
    names = [k for k in kernels(fused_asm) if "prefill_fused_kernel" in k]
    assert len(names) == 2, names  # causal and non-causal


@pytest.mark.parametrize("causal", [True, False])
def test_fused_prefill_no_async_or_mfma_hazard(fused_asm, causal):
    ks = kernels(fused_asm)
    name = next(k for k in ks if "prefill_fused_kernel" in k and ("ILb1" in k) == causal)
    bad = check(ks[name])
    assert not bad, "\n".join(f"{kind}: '{line}' touches {what}" for kind, line, what in bad[:20])


@pytest.mark.parametrize("causal", [True, False])
def test_fused_prefill_lds_reuse_waits_for_tile_loads_before_its_barrier(fused_asm, causal):
    """Where a workgroup starts writing LDS objects afresh -- a pair's second item
    staging its q rows and first K tiles, the row-max pass re-priming its K
    objects -- each wave must drain its own tile loads (vmcnt(0)) before the
    barrier that releases the LDS, so no wave's late tile load lands after another
    wave has started writing there. Such a restart is a global->LDS load after a
    barrier with no product between them (the steps put products first)."""
    ks = kernels(fused_asm)
    body = ks[next(k for k in ks if "prefill_fused_kernel" in k and ("ILb1" in k) == causal)]
    restarts = 0
    for i, line in enumerate(body):
        if not line.startswith("global_load_lds"):
            continue
        bars = [j for j in range(i) if body[j].startswith("s_barrier")]
        if not bars:
            continue  # the workgroup's first loads
        bar = bars[-1]
        if any(body[j].startswith("v_mfma") for j in range(bar, i)):
            continue  # a pipelined step: its loads target objects no wave still reads
        if any(body[j].startswith("global_load_lds") for j in range(bar, i)):
            continue  # checked at the first load after this barrier
        restarts += 1
        last_dma = max((j for j in range(bar) if body[j].startswith("global_load_lds")), default=-1)
        drains = [j for j in range(last_dma + 1, bar) if re.match(r"s_waitcnt vmcnt\(0\)", body[j])]
        assert drains, f"no vmcnt(0) between the last tile load (line {last_dma}) and the barrier at {bar}"
    assert restarts >= 1, "no LDS restart found (the pair's second item or the row-max re-prime)"


@pytest.fixture(scope="module")
def step_asm():
    return build_asm("step.hip")


def test_step_kernels_no_async_or_mfma_hazard(step_asm):
    """The lm head, the split-K GEMV and the stream-K GEMV issue their LDS
    operand reads from asm too: the same check over every kernel of step.hip."""
    ks = kernels(step_asm)
    for want in ("lm_head_split_kernel", "gemv_kernel", "gemv_sk_kernel", "silu_mul_sk_kernel"):
        assert any(want in k for k in ks), want
    for name, body in ks.items():
        bad = check(body)
        assert not bad, name + ":\n" + "\n".join(
            f"{kind}: '{line}' touches {what}" for kind, line, what in bad[:20])


def test_checker_flags_a_read_before_its_wait():
    body = ["ds_read_b128 v[0:3], v10 offset:0",
            "ds_read_b128 v[4:7], v10 offset:16",
            "s_waitcnt lgkmcnt(1)",
            "v_mov_b32_e32 v20, v0",      # fine: the first read is covered
            "v_mov_b32_e32 v21, v4",      # too early: the second is pending
            "s_endpgm"]
    bad = check(body)
    assert [b[1] for b in bad] == ["v_mov_b32_e32 v21, v4"]


def test_checker_flags_a_spill_of_a_pending_load():
    body = ["global_load_dwordx2 a[0:1], v[10:11], off offset:0",
            "scratch_store_dwordx2 off, a[0:1], off",
            "s_waitcnt vmcnt(0)",
            "s_endpgm"]
    assert len(check(body)) == 1


def test_checker_flags_an_early_mfma_result_read():
    mfma = "v_mfma_f32_32x32x16_bf16 v[32:47], v[0:3], a[0:3], v[32:47]"
    assert check([mfma, "s_nop 7", "v_mov_b32_e32 v1, v32", "s_endpgm"])
    assert not check([mfma, "s_nop 7", "s_nop 7", "v_mov_b32_e32 v1, v32", "s_endpgm"])
    # the dependent accumulation is interlocked by the hardware
    assert not check([mfma, mfma, "s_nop 7", "s_nop 7", "s_endpgm"])


def test_checker_follows_branches():
    body = ["ds_read_b128 v[0:3], v10 offset:0",
            "s_cbranch_scc1 .LBB0_2",
            "s_waitcnt lgkmcnt(0)",
            ".LBB0_2:",
            "v_mov_b32_e32 v20, v0",      # pending on the taken path
            "s_endpgm"]
    assert len(check(body)) == 1
