"""Rewrite-rule simplifier for access expressions.

Restates autodiff/expr/simplify.py:6-166.  The reference writes the rules as
one Python ``match`` statement, which has a semantics this module keeps on
purpose because it decides the exact expression text every kernel sees:

* rules are tried in order and the FIRST rule whose pattern (and guard)
  matches is the only one considered;
* if that rule's condition then fails (e.g. ``x * 3``: the constant is not a
  power of two) no later rule is tried -- the node is left alone and only its
  operands are simplified.  This is why ``(((Global % 255) % 255) % 255)``
  survives (the generic ``% c`` rule shadows the ``(% c) % c`` and
  ``% size`` rules);
* operands are rewritten in place (``expr.a = ...``), so shared subtrees are
  simplified once for every parent that holds them;
* ``simplify_expr`` loops until the printed form stops changing and then runs
  one more pass.

Each rule below is a function ``rule(expr, size) -> (matched, result)``;
``result is None`` means "matched but declined".
"""
import math

from . import (Add, BitwiseAnd, Constant, Div, Global, Minus, MoreThan, Mult,
               Remainder, ShiftLeft, ShiftRight, Val, Value)


def _const(e):
    """The integer held by ``Val(Constant(c))``, else None."""
    if type(e) is Val and type(e.v) is Constant:
        return e.v.val
    return None


def _is_const(e, value):
    c = _const(e)
    return c is not None and c == value


def _is_pow2(c) -> bool:
    return math.log2(c).is_integer()


def _r_div_one(e, size):
    if type(e) is Div and _is_const(e.b, 1):
        return True, simpl_expr_inner(e.a, size)
    return False, None


def _r_mult_one_right(e, size):
    if type(e) is Mult and _is_const(e.b, 1):
        return True, simpl_expr_inner(e.a, size)
    return False, None


def _r_mult_one_left(e, size):
    if type(e) is Mult and _is_const(e.a, 1):
        return True, simpl_expr_inner(e.b, size)
    return False, None


def _r_add_zero_right(e, size):
    if type(e) is Add and _is_const(e.b, 0):
        return True, simpl_expr_inner(e.a, size)
    return False, None


def _r_add_zero_left(e, size):
    if type(e) is Add and _is_const(e.a, 0):
        return True, simpl_expr_inner(e.b, size)
    return False, None


def _r_zero_result(e, size):
    """``_*0``, ``0*_``, ``_&0``, ``0<<_``, ``0>>_`` -> 0 (simplify.py:36-57)."""
    t = type(e)
    hit = ((t is Mult and (_is_const(e.b, 0) or _is_const(e.a, 0)))
           or (t is BitwiseAnd and _is_const(e.b, 0))
           or (t in (ShiftLeft, ShiftRight) and _is_const(e.a, 0)))
    if hit:
        return True, Val(Constant(0))
    return False, None


def _r_minus_minus(e, size):
    if type(e) is Minus and type(e.a) is Minus:
        n1, n2 = _const(e.a.b), _const(e.b)
        if n1 is not None and n2 is not None:
            return True, simpl_expr_inner(Minus(e.a.a, Val(Constant(n1 + n2))), size)
    return False, None


def _r_more_minus(e, size):
    if type(e) is MoreThan and type(e.a) is Minus:
        n1, n2 = _const(e.a.b), _const(e.b)
        if n1 is not None and n2 is not None:
            return True, simpl_expr_inner(MoreThan(e.a.a, Val(Constant(n1 + n2))), size)
    return False, None


def _r_pow2_strength(e, size):
    """``*2^p -> <<p``, ``/2^p -> >>p``, ``%2^p -> &(2^p-1)`` (simplify.py:64-78).

    Matches every Mult/Div/Remainder with a constant right operand; for a
    constant that is not a power of two it declines, which also shadows the
    later ``%``-rules."""
    t = type(e)
    if t not in (Mult, Div, Remainder):
        return False, None
    c = _const(e.b)
    if c is None:
        return False, None
    if not _is_pow2(c):
        return True, None
    if t is Mult:
        return True, simpl_expr_inner(ShiftLeft(e.a, Val(Constant(int(math.log2(c))))), size)
    if t is Div:
        return True, simpl_expr_inner(ShiftRight(e.a, Val(Constant(int(math.log2(c))))), size)
    return True, simpl_expr_inner(BitwiseAnd(e.a, Val(Constant(c - 1))), size)


def _r_and_and(e, size):
    if type(e) is BitwiseAnd and type(e.a) is BitwiseAnd:
        c1, c2 = _const(e.a.b), _const(e.b)
        if c1 is not None and c2 is not None:
            if c1 == c2:
                return True, simpl_expr_inner(BitwiseAnd(e.a.a, Val(Constant(c1))), size)
            return True, None
    return False, None


def _r_split_mod(e, size):
    """``(((g >> v) & b) << v) + (g & a)`` -> ``g % 2^(log2(b+1)+log2(a+1))``
    when both masks are all-ones and the two shifts agree (simplify.py:98-120)."""
    if type(e) is not Add:
        return False, None
    left, right = e.a, e.b
    if not (type(left) is ShiftLeft and type(left.a) is BitwiseAnd
            and type(left.a.a) is ShiftRight and type(right) is BitwiseAnd):
        return False, None
    v1 = _const(left.a.a.b)
    b = _const(left.a.b)
    v = _const(left.b)
    a = _const(right.b)
    if None in (v1, b, v, a):
        return False, None
    gl, gl2 = left.a.a.a, right.a
    if gl == gl2 and v == v1 and _is_pow2(b + 1) and _is_pow2(a + 1):
        mod = int(pow(2, math.log2(b + 1) + math.log2(a + 1)))
        return True, simpl_expr_inner(Remainder(gl, Val(Constant(mod))), size)
    return True, None


def _r_mod_size(e, size):
    """``x % size -> x`` for a command of ``size`` elements (simplify.py:122-127).
    Unreachable behind ``_r_pow2_strength``; kept so the rule list is whole."""
    if size is None or type(e) is not Remainder:
        return False, None
    s = _const(e.b)
    if s is None:
        return False, None
    if s == size:
        return True, simpl_expr_inner(e.a, size)
    return True, None


def _r_and_size(e, size):
    """``x & (size-1) -> x``, and ``(Global >> c) & s -> Global >> c`` when
    ``(size-1) >> c <= s`` (simplify.py:129-145)."""
    if size is None or type(e) is not BitwiseAnd:
        return False, None
    s = _const(e.b)
    if s is None:
        return False, None
    if s + 1 == size:
        return True, simpl_expr_inner(e.a, size)
    val = e.a
    if type(val) is ShiftRight and type(val.a) is Global:
        c = _const(val.b)
        if c is not None and ((size - 1) >> c) <= s:
            return True, simpl_expr_inner(val, size)
    return True, None


_RULES = (
    _r_div_one,
    _r_mult_one_right,
    _r_mult_one_left,
    _r_add_zero_right,
    _r_add_zero_left,
    _r_zero_result,
    _r_minus_minus,
    _r_more_minus,
    _r_pow2_strength,
    _r_and_and,
    _r_split_mod,
    _r_mod_size,
    _r_and_size,
)


def simpl_expr_inner(expr, size):
    """One rewrite pass (simplify.py:6-153)."""
    if isinstance(expr, Value) or isinstance(expr, Val):
        return expr
    for rule in _RULES:
        matched, result = rule(expr, size)
        if matched:
            if result is not None:
                return result
            break
    if expr.is_binary():
        expr.a = simpl_expr_inner(expr.a, size)
        expr.b = simpl_expr_inner(expr.b, size)
    return expr


def simplify_expr(expr, size):
    """Rewrite until a pass leaves the printed form unchanged, then apply
    one more pass (the behaviour of simplify.py:158-166)."""
    prev, cur = expr, simpl_expr_inner(expr, size)
    while str(cur) != str(prev):
        prev, cur = cur, simpl_expr_inner(cur, size)
    return simpl_expr_inner(cur, size)
