"""Static facts about access expressions used by the HIP code generator.

* ``split_const``: ``expr == core + c`` with every additive constant pulled
  to the top (through ``+``, ``<<`` and ``*`` by a constant), so ``c`` can be
  folded into the base pointer and kernels that differ only in offsets share
  one compiled binary.
* ``upper_bound``: an upper bound of an expression over its index ranges,
  to pick 32- or 64-bit index arithmetic.
* ``vec_class``: whether an access is contiguous and 4-aligned, or constant,
  over aligned groups of 4 consecutive indices (the float4 decision).

All index values the compiler produces are non-negative integers; the one
exception, ``Minus`` inside a concat branch, is only evaluated when that
branch is selected, where it is non-negative too.
"""
from ...expr import (Add, BitwiseAnd, Constant, Div, Global, LessThan, Minus, MoreThan, Mult,
                     Remainder, ShiftLeft, ShiftRight, Val, X, Y)


def const_of(e):
    if type(e) is Val and type(e.v) is Constant:
        return e.v.val
    if type(e) is Constant:
        return e.val
    return None


def split_const(e):
    """Return ``(core, c)`` with ``value(e) == value(core) + c``; ``core`` is a
    new tree (the input is not modified)."""
    c = const_of(e)
    if c is not None:
        return Val(Constant(0)), int(c)
    t = type(e)
    if t is Add:
        ca, ka = split_const(e.a)
        cb, kb = split_const(e.b)
        if const_of(ca) == 0:
            return cb, ka + kb
        if const_of(cb) == 0:
            return ca, ka + kb
        return Add(ca, cb), ka + kb
    if t is ShiftLeft and const_of(e.b) is not None:
        ca, ka = split_const(e.a)
        k = int(const_of(e.b))
        return (Val(Constant(0)) if const_of(ca) == 0 else ShiftLeft(ca, e.b)), ka << k
    if t is Mult and const_of(e.b) is not None:
        ca, ka = split_const(e.a)
        m = int(const_of(e.b))
        return (Val(Constant(0)) if const_of(ca) == 0 else Mult(ca, e.b)), ka * m
    if t is Mult and const_of(e.a) is not None:
        cb, kb = split_const(e.b)
        m = int(const_of(e.a))
        return (Val(Constant(0)) if const_of(cb) == 0 else Mult(e.a, cb)), kb * m
    if isinstance(e, (Global, X, Y)) or type(e) is Val:
        return e, 0
    return _rebuild(e), 0


def _rebuild(e):
    """Copy with every operand canonicalised internally (constants stay
    inside non-distributive operators)."""
    t = type(e)
    if t is Val or isinstance(e, (Global, X, Y, Constant)):
        return e
    a = _canon(e.a)
    b = _canon(e.b)
    return t(a, b)


def _canon(e):
    core, c = split_const(e)
    if c == 0:
        return core
    if const_of(core) == 0:
        return Val(Constant(c))
    return Add(core, Val(Constant(c)))


def upper_bound(e, gmax=0, xmax=0, ymax=0):
    """Largest value ``e`` can take (non-negative semantics)."""
    return _bounds(e, gmax, xmax, ymax)[1]


def interval(e, gmax=0, xmax=0, ymax=0):
    """``(lo, hi)``: smallest and largest value ``e`` can take for Global,
    X, Y in ``[0, gmax]``, ``[0, xmax]``, ``[0, ymax]`` (non-negative
    semantics: a difference is bounded below by 0)."""
    return _bounds(e, gmax, xmax, ymax)


def _bounds(e, gmax, xmax, ymax):
    c = const_of(e)
    if c is not None:
        return c, c
    if isinstance(e, Global):
        return 0, gmax
    if isinstance(e, X):
        return 0, xmax
    if isinstance(e, Y):
        return 0, ymax
    if type(e) is Val:
        return _bounds(e.v, gmax, xmax, ymax)
    alo, ahi = _bounds(e.a, gmax, xmax, ymax)
    blo, bhi = _bounds(e.b, gmax, xmax, ymax)
    t = type(e)
    if t is Add:
        return alo + blo, ahi + bhi
    if t is Minus:
        return max(0, alo - bhi), max(0, ahi - blo)
    if t is Mult:
        return alo * blo, ahi * bhi
    if t is Div:
        return (alo // bhi if bhi else 0), (ahi // blo if blo else ahi)
    if t is Remainder:
        return 0, min(ahi, bhi - 1 if bhi > 0 else 0)
    if t is ShiftLeft:
        return alo << blo, ahi << bhi
    if t is ShiftRight:
        return alo >> bhi, ahi >> blo
    if t is BitwiseAnd:
        return 0, min(ahi, bhi)
    if t in (MoreThan, LessThan):
        return 0, 1
    raise TypeError(f"bounds of {e!r}")


# ----------------------------------------------------------------- float4 analysis
AFF, INV, UNK = "aff", "inv", "unk"


class VC:
    """Abstract value over an aligned group v = 4t + i (i = 0..3):
    ``AFF``: f(4t+i) = f(4t) + i, ``al`` -> f(4t) % 4 == 0;
    ``INV``: f(4t+i) = f(4t), ``d4`` -> f(4t) % 4 == 0."""
    __slots__ = ("kind", "al")

    def __init__(self, kind, al=False):
        self.kind = kind
        self.al = al


def vec_class(e, var_type, zero=()):
    """Classify ``e`` as a function of the index variable of type
    ``var_type`` (Global, X or Y, or a tuple of types that all advance with
    the element index); variables whose type is in ``zero`` are 0; the other
    index variables are arbitrary per group (INV, unknown residue)."""
    c = const_of(e)
    if c is not None:
        return VC(INV, c % 4 == 0)
    if isinstance(e, (Global, X, Y)):
        if type(e) in zero:
            return VC(INV, True)
        moving = type(e) in var_type if isinstance(var_type, tuple) else type(e) is var_type
        return VC(AFF, True) if moving else VC(INV, False)
    if type(e) is Val:
        return vec_class(e.v, var_type, zero)
    t = type(e)
    a = vec_class(e.a, var_type, zero)
    kb = const_of(e.b)
    if t in (Add, Minus):
        b = vec_class(e.b, var_type, zero)
        if a.kind == AFF and b.kind == INV:
            return VC(AFF, a.al and b.al)
        if t is Add and a.kind == INV and b.kind == AFF:
            return VC(AFF, a.al and b.al)
        if a.kind == INV and b.kind == INV:
            return VC(INV, a.al and b.al)
        return VC(UNK)
    if t is Mult:
        b = vec_class(e.b, var_type, zero)
        if a.kind == INV and b.kind == INV:
            return VC(INV, a.al or b.al)
        if a.kind == AFF and kb == 1:
            return a
        return VC(UNK)
    if t is ShiftLeft and kb is not None:
        if a.kind == INV:
            return VC(INV, a.al or kb >= 2)
        if a.kind == AFF and kb == 0:
            return a
        return VC(UNK)
    if t is ShiftRight and kb is not None:
        if a.kind == INV:
            return VC(INV, False)
        if a.kind == AFF and a.al and kb >= 2:
            return VC(INV, False)
        if a.kind == AFF and kb == 0:
            return a
        return VC(UNK)
    if t is Div and kb is not None:
        if a.kind == INV:
            return VC(INV, False)
        if a.kind == AFF and a.al and kb % 4 == 0:
            return VC(INV, False)
        if a.kind == AFF and kb == 1:
            return a
        return VC(UNK)
    if t is Remainder and kb is not None:
        if a.kind == INV:
            return VC(INV, a.al and kb % 4 == 0)
        if a.kind == AFF and a.al and kb % 4 == 0:
            return VC(AFF, True)
        return VC(UNK)
    if t is BitwiseAnd and kb is not None:
        if a.kind == INV:
            return VC(INV, a.al or (kb & 3) == 0)
        if a.kind == AFF and a.al and (kb & 3) == 3:
            return VC(AFF, True)
        return VC(UNK)
    if t in (MoreThan, LessThan) and kb is not None:
        if a.kind == INV:
            return VC(INV, False)
        if a.kind == AFF and a.al:
            # f+i > c is constant over i in 0..3 iff c+1 is a multiple of 4
            edge = kb + 1 if t is MoreThan else kb
            if edge % 4 == 0:
                return VC(INV, False)
        return VC(UNK)
    if t in (MoreThan, LessThan):
        b = vec_class(e.b, var_type, zero)
        if a.kind == INV and b.kind == INV:
            return VC(INV, False)
        return VC(UNK)
    # other operators with a non-constant right operand
    b = vec_class(e.b, var_type, zero)
    if a.kind == INV and b.kind == INV:
        return VC(INV, False)
    return VC(UNK)
