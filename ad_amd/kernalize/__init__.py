"""Operands of kernel statements.

After kernalize every operand and result slot of a node holds one of these
(the reference's kernel-arg vocabulary, autodiff/kernalize/__init__.py:6-128,
whose printed forms appear verbatim in Proc listings):

* ``KMatrix(id, access, shape)`` -- element ``access`` of buffer ``id``;
  ``is_temp`` marks a value that lives in a register of a fused kernel;
* ``KConcat(karg_one, karg_two, condition, shape)`` -- a concat folded into
  indexing: where ``condition`` holds the element comes from ``karg_two``,
  elsewhere from ``karg_one``;
* ``KConstant(value)`` -- a literal;
* ``NoneKernelArg()`` -- a slot kernalize has not filled yet.

Buffer renames and the temp marking act on the buffer references
(``KMatrix`` leaves) an operand contains, so the composite kinds implement
only their traversal (``_leaves``) and printing.
"""
from math import prod
from typing import Callable, Iterator, List, Optional

from ..expr import Add, Constant, Expression, Global, Val


def _indented(text: str, pad: str = "    ") -> str:
    return "\n".join(pad + line for line in text.splitlines())


class KernelArg:
    """Base of the operand kinds.  Subclasses yield their buffer references
    from ``_leaves``; renaming and temp marking apply to those."""

    def _leaves(self) -> Iterator["KMatrix"]:
        raise NotImplementedError(f"{type(self).__name__} has no buffer references")

    def __repr__(self):
        raise NotImplementedError(f"{type(self).__name__} cannot be printed")

    def is_none(self) -> bool:
        return False

    def get_ids(self, filter_temp: bool = False) -> List[int]:
        """Buffer ids read through this operand (temps left out when
        ``filter_temp``)."""
        raise NotImplementedError(f"{type(self).__name__} lists no buffer ids")

    def rename(self, fr: int, to: int, change_access: Optional[Callable[[Expression], Expression]] = None):
        """Point every reference to buffer ``fr`` at buffer ``to``, mapping
        its access through ``change_access`` if given."""
        for leaf in self._leaves():
            if leaf.id == fr:
                leaf.id = to
                if change_access is not None:
                    leaf.access = change_access(leaf.access)

    def change_to_temp(self, search: int):
        """Mark every reference to buffer ``search`` as a register temp."""
        for leaf in self._leaves():
            if leaf.id == search:
                leaf.is_temp = True

    def calc_offset(self):
        raise NotImplementedError(f"{type(self).__name__} has no contiguous offset")


class NoneKernelArg(KernelArg):
    """An operand slot not lowered yet."""

    def __repr__(self):
        return "None"

    def is_none(self):
        return True

    def rename(self, fr, to, change_access=None):
        raise NotImplementedError("an unlowered operand has no buffer to rename")


class KMatrix(KernelArg):
    def __init__(self, kern_id: int, access: Expression, shape: List[int]):
        self.id = kern_id
        self.access = access
        self.shape = shape
        self.is_temp = False
        self.offset = None

    def _leaves(self):
        yield self

    def __repr__(self):
        return f"Temp {self.id}" if self.is_temp else f"Mat (id: {self.id}, {self.access!r})"

    def get_ids(self, filter_temp=False):
        return [] if (filter_temp and self.is_temp) else [self.id]

    def calc_offset(self):
        """The first element of a contiguous read or write (Feeders and
        Receivers move one contiguous run of floats): 0 for ``Global``,
        ``c`` for ``Global + c``, and ``c`` for the constant access of a
        single element (autodiff/kernalize/__init__.py:74-83).  Any other
        access is not contiguous from a known start."""
        acc = self.access
        start = None
        if isinstance(acc, Global):
            start = 0
        elif type(acc) is Add and isinstance(acc.a, Global) and type(acc.b) is Val and type(acc.b.v) is Constant:
            start = acc.b.v.val
        elif type(acc) is Val and type(acc.v) is Constant and prod(self.shape) == 1:
            start = acc.v.val
        if start is None:
            raise Exception(f"access {acc} of buffer {self.id} is not a contiguous run from a fixed start; "
                            f"read or feed it through .contigious()")
        self.offset = start


class KConcat(KernelArg):
    def __init__(self, karg_one: KernelArg, karg_two: KernelArg, condition: Expression, shape: List[int]):
        self.karg_one = karg_one
        self.karg_two = karg_two
        self.condition = condition      # holds -> karg_two, else karg_one
        self.shape = shape

    def _leaves(self):
        yield from self.karg_one._leaves()
        yield from self.karg_two._leaves()

    def __repr__(self):
        body = f"1: {self.karg_one}\n2: {self.karg_two}\ncond: {self.condition}"
        return f"\nConcat (\n{_indented(body)}\n)\n"

    def get_ids(self, filter_temp=False):
        # the union of both sides, as a set (its iteration order is what
        # argument lists and dependency sets are built from)
        return list(set(self.karg_one.get_ids(filter_temp) + self.karg_two.get_ids(filter_temp)))


class KConstant(KernelArg):
    def __init__(self, constant: float):
        self.constant = constant

    def _leaves(self):
        return iter(())

    def __repr__(self):
        return f"{self.constant}"

    def get_ids(self, filter_temp=False):
        return []
