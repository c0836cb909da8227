"""The reference-side Julia bindings in INTEGRATION.md against the C header.

Every ``ccall((:vm_..., libvm), Ret, (ArgTypes...), args...)`` in the Julia
blocks of INTEGRATION.md must name an entry point that include/vallmo_attn.h
declares, with the same return type, the same number of parameters, each of a
matching C type, and must pass exactly that many arguments (``strides(X)[a:b]...``
splats count b - a + 1). A binding that drifts from the header would corrupt
the stack of the caller, so this is checked here on the CPU.
"""
from __future__ import annotations

import re

from conftest import ROOT

HEADER = ROOT / "include" / "vallmo_attn.h"
DOC = ROOT / "INTEGRATION.md"

# Julia ccall type -> the C types it may stand for
JL2C = {
    "Cint": {"int"},
    "Cuint": {"unsigned", "unsigned int"},
    "Int64": {"int64_t"},
    "UInt64": {"uint64_t"},
    "Csize_t": {"size_t"},
    "Cfloat": {"float"},
    "Cdouble": {"double"},
    "Cstring": {"const char*"},
}


def _split_top(s: str) -> list[str]:
    """Split on commas outside (), [] and {}."""
    out, depth, cur = [], 0, []
    for ch in s:
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        if ch == "," and depth == 0:
            out.append("".join(cur).strip())
            cur = []
        else:
            cur.append(ch)
    if "".join(cur).strip():
        out.append("".join(cur).strip())
    return out


def _balanced(s: str, start: int) -> int:
    """Index just past the bracket group opening at s[start]."""
    depth = 0
    for i in range(start, len(s)):
        if s[i] in "([{":
            depth += 1
        elif s[i] in ")]}":
            depth -= 1
            if depth == 0:
                return i + 1
    raise ValueError("unbalanced")


def header_prototypes() -> dict[str, tuple[str, list[str]]]:
    text = re.sub(r"/\*.*?\*/", " ", HEADER.read_text(), flags=re.S)
    text = re.sub(r"#.*", " ", text)
    protos = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(vm_\w+)\s*\(([^;{]*?)\)\s*;", text):
        ret = " ".join(m.group(1).split())
        params = [] if m.group(3).strip() in ("", "void") else [
            " ".join(p.split()) for p in m.group(3).split(",")]
        protos[m.group(2)] = (ret, params)
    return protos


def c_kind(decl: str) -> str:
    """The C type of a parameter declaration with its name removed."""
    decl = decl.replace("*", " * ")
    toks = decl.split()
    if len(toks) > 1 and toks[-1] not in ("*",) and re.match(r"^\w+$", toks[-1]):
        toks = toks[:-1]
    t = " ".join(toks).replace(" * ", "*").replace(" *", "*")
    if t.endswith("*") or t in ("vm_stream",):
        return "ptr:" + t
    return t


def julia_ccalls() -> list[tuple[str, str, list[str], list[str]]]:
    text = DOC.read_text()
    blocks = re.findall(r"```julia\n(.*?)```", text, flags=re.S)
    calls = []
    for blk in blocks:
        for m in re.finditer(r"ccall\(", blk):
            end = _balanced(blk, m.end() - 1)
            inner = blk[m.end():end - 1]
            parts = _split_top(inner)
            name = re.match(r"\(:(vm_\w+),", parts[0] + ",").group(1)
            ret = parts[1]
            types_s = parts[2].strip()
            assert types_s.startswith("(") and types_s.endswith(")"), types_s
            types = _split_top(types_s[1:-1])
            calls.append((name, ret, types, parts[3:]))
    return calls


def _arg_count(args: list[str]) -> int:
    n = 0
    for a in args:
        m = re.fullmatch(r"strides\([\w.]+\)\[(\d+):(\d+)\]\.\.\.", a)
        if m:
            n += int(m.group(2)) - int(m.group(1)) + 1
        else:
            assert not a.endswith("..."), f"uncountable splat {a}"
            n += 1
    return n


def _matches(jl: str, c: str) -> bool:
    if jl.startswith("Ptr{"):
        return c.startswith("ptr:")
    if c.startswith("ptr:"):
        return jl == "Cstring" and c == "ptr:const char*"
    return c in JL2C.get(jl, set())


def test_every_binding_matches_the_header():
    protos = header_prototypes()
    calls = julia_ccalls()
    assert len(calls) >= 12, "INTEGRATION.md lost its bindings"
    seen = set()
    for name, ret, types, args in calls:
        assert name in protos, f"{name} is not declared in vallmo_attn.h"
        cret, cparams = protos[name]
        ck = c_kind(cret + " x")
        assert _matches(ret, ck), f"{name}: return {ret} vs {cret}"
        assert len(types) == len(cparams), \
            f"{name}: {len(types)} Julia argument types vs {len(cparams)} C parameters"
        for i, (jt, cp) in enumerate(zip(types, cparams)):
            assert _matches(jt, c_kind(cp)), f"{name} parameter {i + 1}: {jt} vs {cp}"
        if name != "vm_last_error":
            assert _arg_count(args) == len(types), \
                f"{name}: passes {_arg_count(args)} arguments for {len(types)} types"
        seen.add(name)
    for must in ("vm_gated_attn_decode", "vm_gated_attn_prefill", "vm_attention_fwd",
                 "vm_decode_attention", "vm_qnorm_rope", "vm_knorm_rope_append",
                 "vm_decode_scratch_bytes", "vm_prefill_scratch_bytes", "vm_linear",
                 "vm_rms_norm", "vm_fused_add_rms_norm", "vm_silu_mul", "vm_embed",
                 "vm_generation_advance", "vm_lm_head_argmax", "vm_causal_conv1d",
                 "vm_causal_conv1d_sequence", "vm_fused_deltanet_decode",
                 "vm_deltanet_recurrent_decode", "vm_deltanet_sequence",
                 "vm_deltanet_prefill_prep", "vm_gated_rms_norm"):
        assert must in seen, f"INTEGRATION.md has no binding for {must}"


def test_binding_uses_reference_field_names():
    """The decode!/forward bindings read the reference's own fields
    (qwen35.jl:129-142: l.qw, l.kw) and the arena (qwen35.jl:193)."""
    text = DOC.read_text()
    assert "l.qw" in text and "l.kw" in text
    for stale in ("l.q_norm", "l.k_norm", "m.arena", "m.scratch", "take!("):
        assert stale not in text, stale
