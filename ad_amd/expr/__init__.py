"""Integer index expressions ("access expressions").

Every kernel operand address in the procedural IR is one of these trees.  The
leaf/operator vocabulary and the equality rules restate
autodiff/expr/__init__.py:6-156 of the reference:

* ``Value`` leaves (``Constant``, ``Global``, ``X``, ``Y``) compare by their
  printed form, except ``Constant`` which compares by value.
* Operator nodes compare structurally and only against the same node type.
* ``Val`` wraps a leaf so it can sit inside an operator node.

The printed form has no terminal colours (the reference colours its output);
equality and the simplifier's fixpoint test only ever compare two printed
forms with each other, so dropping colours changes neither.
"""


class Value:
    """Leaf value.  Equality is by printed form (expr/__init__.py:6-14)."""

    def __eq__(self, other):
        if isinstance(other, Value):
            return repr(self) == repr(other)
        return False

    __hash__ = None

    def get_const(self) -> int:
        raise TypeError("get_const at Value()")


class Constant(Value):
    __match_args__ = ("val",)

    def __init__(self, val):
        self.val = val

    def __eq__(self, other):
        if type(other) is Constant:
            return self.val == other.val
        return NotImplemented

    __hash__ = None

    def __repr__(self):
        return str(self.val)

    def get_const(self):
        return self.val


class Global(Value):
    def __repr__(self):
        return "Global"


class X(Value):
    def __repr__(self):
        return "X"


class Y(Value):
    def __repr__(self):
        return "Y"


class Expression:
    def get_const(self) -> int:
        raise TypeError("Expression is not a const")

    def __repr__(self) -> str:
        raise TypeError("Repr of expression invalid")

    def is_binary(self) -> bool:
        return True

    def __eq__(self, value):
        if isinstance(value, Expression):
            return repr(value) == repr(self)
        return False

    __hash__ = None


class NoneExpr(Expression):
    def __repr__(self):
        return "None"

    def is_binary(self):
        return False


class Val(Expression):
    """A leaf inside an expression tree."""
    __match_args__ = ("v",)

    def __init__(self, v):
        self.v = v

    def __eq__(self, other):
        if type(other) is Val:
            return self.v == other.v
        return NotImplemented

    __hash__ = None

    def __repr__(self):
        return repr(self.v)

    def is_binary(self):
        return False

    def get_const(self):
        return self.v.get_const()


class _BinExpr(Expression):
    """Operator node with operands ``a`` and ``b``; equal only to the same type."""
    __match_args__ = ("a", "b")
    SYMBOL = "?"

    def __init__(self, a, b):
        self.a = a
        self.b = b

    def __eq__(self, other):
        if type(other) is type(self):
            return self.a == other.a and self.b == other.b
        return NotImplemented

    __hash__ = None

    def __repr__(self):
        return f"({self.a!r} {self.SYMBOL} {self.b!r})"


class Add(_BinExpr):
    SYMBOL = "+"


class Minus(_BinExpr):
    SYMBOL = "-"


class Mult(_BinExpr):
    SYMBOL = "*"


class Div(_BinExpr):
    SYMBOL = "/"


class Remainder(_BinExpr):
    SYMBOL = "%"


class ShiftRight(_BinExpr):
    SYMBOL = ">>"


class ShiftLeft(_BinExpr):
    SYMBOL = "<<"


class BitwiseAnd(_BinExpr):
    SYMBOL = "&"


class MoreThan(_BinExpr):
    SYMBOL = ">"


class LessThan(_BinExpr):
    SYMBOL = "<"


BINARY_EXPR_TYPES = (Add, Minus, Mult, Div, Remainder, ShiftRight, ShiftLeft,
                     BitwiseAnd, MoreThan, LessThan)


def evaluate(expr, g=0, x=0, y=0):
    """Evaluate an expression with Python integers (C semantics for the
    non-negative operands these trees carry).  Used by tests and the codegen's
    range analysis, never on the execution path."""
    if isinstance(expr, Val):
        return evaluate(expr.v, g, x, y)
    if isinstance(expr, Constant):
        return expr.val
    if isinstance(expr, Global):
        return g
    if isinstance(expr, X):
        return x
    if isinstance(expr, Y):
        return y
    a = evaluate(expr.a, g, x, y)
    b = evaluate(expr.b, g, x, y)
    t = type(expr)
    if t is Add:
        return a + b
    if t is Minus:
        return a - b
    if t is Mult:
        return a * b
    if t is Div:
        q = abs(a) // abs(b)
        return q if (a >= 0) == (b >= 0) else -q
    if t is Remainder:
        r = abs(a) % abs(b)
        return r if a >= 0 else -r
    if t is ShiftRight:
        return a >> b
    if t is ShiftLeft:
        return a << b
    if t is BitwiseAnd:
        return a & b
    if t is MoreThan:
        return int(a > b)
    if t is LessThan:
        return int(a < b)
    raise TypeError(f"cannot evaluate {expr!r}")
