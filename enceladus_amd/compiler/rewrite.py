"""Algebraic rewrites on the tile IR that save VALU work in the hot loops.

`fold_softmax_scale`: the online-softmax step of attention computes

    t = qk * s;  u = where(mask, t, -inf);  r = max(u, axis);  ...;  p = exp2(u - m[:, None])

with one multiply per score. For a scale s known to be positive, max commutes with the
scaling exactly (rounding is monotone, so max_i round(s * x_i) = round(s * max_i x_i), and
-inf * s = -inf), so the kernel can reduce the raw scores and scale only the row maxima:

    u' = where(mask, qk, -inf);  r = max(u', axis) * s;  ...;  p = exp2(fma(u', s, -m[:, None]))

The row maxima are bit-identical; each `u - m` becomes one fused multiply-add, so the
exponent's argument is rounded once instead of twice (within the attention tolerances).
Positivity comes from the launch: a float argument that is > 0 carries the `positive`
specialization fact, so a negative scale compiles the unrewritten kernel.
"""

from __future__ import annotations

import math

from enceladus_amd.compiler import ir
from enceladus_amd.language import core


def _positive(v: ir.Value, depth=0) -> bool:
    """Whether scalar `v` is provably > 0 (arguments with the `positive` fact, positive
    constants, and products/quotients/casts of those)."""
    if depth > 16 or not isinstance(v.type, ir.TType) or v.type.shape:
        return False
    op = v.op
    if op is None:
        return bool(v.facts.get("positive"))
    if op.name == "const":
        x = op.attrs.get("value")
        return isinstance(x, (int, float)) and not isinstance(x, bool) and x > 0
    if op.name in ("hint", "cast") and op.result.type.dtype.is_floating():
        return _positive(op.operands[0], depth + 1)
    if op.name == "binary" and op.attrs.get("op") in ("mul", "div"):
        return all(_positive(o, depth + 1) for o in op.operands)
    return False


def _splat_scalar(v: ir.Value):
    """The scalar a tile is a splat of (through broadcasts), or None."""
    while v.op is not None and v.op.name in ("broadcast", "expand_dims"):
        v = v.op.operands[0]
    if v.op is not None and v.op.name == "splat":
        return v.op.operands[0]
    return None


def _is_neg_inf(v: ir.Value) -> bool:
    while v.op is not None and v.op.name in ("broadcast", "expand_dims", "splat"):
        v = v.op.operands[0]
    if v.op is None or v.op.name != "const":
        return False
    x = v.op.attrs.get("value")
    return isinstance(x, float) and math.isinf(x) and x < 0


def _blocks(b: ir.Block):
    yield b
    for op in b.ops:
        for r in op.regions:
            yield from _blocks(r)


def fold_softmax_scale(fn: ir.Func) -> int:
    """Applies the rewrite above wherever it matches; returns how many times."""
    uses: dict[int, list] = {}
    where: dict[int, ir.Block] = {}
    for blk in _blocks(fn.body):
        for op in blk.ops:
            where[id(op)] = blk
            for o in op.operands:
                uses.setdefault(o.id, []).append(op)
    done = 0
    for blk in list(_blocks(fn.body)):
        for op in list(blk.ops):
            if op.name != "binary" or op.attrs.get("op") != "mul":
                continue
            t = op.result
            if t.type.dtype is not core.float32 or len(t.type.shape) != 2:
                continue
            x = s = None
            for a, b in (op.operands, op.operands[::-1]):
                sc = _splat_scalar(b)
                if sc is not None and a.type.shape == t.type.shape and _positive(sc):
                    x, s = a, sc
                    break
            if x is None:
                continue
            u, sel = t, None
            tu = uses.get(t.id, [])
            if len(tu) == 1 and tu[0].name == "select" and tu[0].operands[1] is t and \
                    _is_neg_inf(tu[0].operands[2]):
                sel = tu[0]
                u = sel.result
            uu = uses.get(u.id, [])
            reds = [o for o in uu if o.name == "reduce" and o.attrs.get("kind") == "max"]
            subs = [o for o in uu if o.name == "binary" and o.attrs.get("op") == "sub" and
                    o.operands[0] is u and o.operands[1] is not u]
            if not reds or not subs or len(reds) + len(subs) != len(uu):
                continue
            if sel is None and len(tu) != len(uu):
                continue
            # u' = where(mask, x, -inf) (or x itself)
            if sel is not None:
                sel.operands[1] = x
                new_u = u
            else:
                new_u = x
            for red in reds:
                red.operands[0] = new_u
                r = red.result
                rb = where[id(red)]
                sp = ir.Op("splat", [s], [r.type.with_shape(r.type.shape)], loc=red.loc) \
                    if r.type.shape else None
                sv = sp.result if sp is not None else s
                mul = ir.Op("binary", [r, sv], [r.type], {"op": "mul"}, loc=red.loc)
                i = rb.ops.index(red)
                rb.ops[i + 1:i + 1] = [o for o in (sp, mul) if o is not None]
                for user in list(uses.get(r.id, [])):
                    user.operands = [mul.result if o is r else o for o in user.operands]
            for sub in subs:
                sb = where[id(sub)]
                m = sub.operands[1]
                sp = ir.Op("splat", [s], [new_u.type], loc=sub.loc)
                neg = ir.Op("unary", [m], [m.type], {"op": "neg"}, loc=sub.loc)
                fma = ir.Op("fma", [new_u, sp.result, neg.result], [sub.result.type],
                            loc=sub.loc)
                i = sb.ops.index(sub)
                sb.ops[i:i + 1] = [sp, neg, fma]
                for user in list(uses.get(sub.result.id, [])):
                    user.operands = [fma.result if o is sub.result else o
                                     for o in user.operands]
            done += 1
    return done
