"""Shape contracts at the verb — the @sizes macro of src/sizes.jl:23-65.

Tensors here are torch tensors whose shapes are the reference's column-major
dims reversed: Julia's Q :: (D, Hq, B) is a torch tensor of shape (B, Hq, D).
Declarations and messages use the reference's order, so ``size(Q, 1)`` is the
innermost (head_dim) extent, exactly as in the reference's error text:

    sizes(Q=(q, "D Hq B"), K=(k, "D Ctx Hk B"))   # binds D, Hq, B, Ctx, Hk

The first occurrence of a name binds it; every later occurrence checks it and
raises DimensionMismatch naming the binding site; "_" skips a dim; an integer
literal checks against its value; a tensor given as None skips its line.
"""
from __future__ import annotations

from ._lib import DimensionMismatch


def sizes(**decls):
    bound: dict[str, tuple[int, str]] = {}
    for name, (arr, spec) in decls.items():
        if arr is None:
            continue
        dims = spec.split()
        jl_shape = tuple(reversed(tuple(arr.shape)))
        if len(jl_shape) != len(dims):
            raise DimensionMismatch(
                f"{name} has {len(jl_shape)} dimensions, expected {len(dims)} from "
                f"({', '.join(dims)})")
        for i, (s, extent) in enumerate(zip(dims, jl_shape), start=1):
            site = f"size({name}, {i})"
            if s == "_":
                continue
            if s.lstrip("-").isdigit():
                if extent != int(s):
                    raise DimensionMismatch(f"{site} = {extent} does not match `{s}` = {s}")
                continue
            if s not in bound:
                bound[s] = (extent, site)
            elif bound[s][0] != extent:
                raise DimensionMismatch(
                    f"{site} = {extent} does not match {s} = {bound[s][0]} (= {bound[s][1]})")
    return {k: v[0] for k, v in bound.items()}
