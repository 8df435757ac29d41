"""Kernel operand descriptors ("kernel args").

Restates autodiff/kernalize/__init__.py:6-128.  After kernalize every node
operand is one of:

* ``KMatrix``  -- buffer ``id`` read/written at integer ``access`` expression;
  ``is_temp`` marks a register-resident value inside a fused kernel;
* ``KConcat``  -- ``cond ? karg_two : karg_one`` (a concat folded into indexing);
* ``KConstant`` -- a float literal.
"""
from math import prod
from typing import Callable, List, Optional

from ..expr import Add, Constant, Expression, Global, Val


class KernelArg:
    def __repr__(self):
        raise NotImplementedError("Kernel arg __repr__ not implemented")

    def is_none(self) -> bool:
        return False

    def get_ids(self, filter_temp=False) -> List[int]:
        raise NotImplementedError("Kernel arg get_ids not implemented")

    def rename(self, fr, to, change_access: Optional[Callable[[Expression], Expression]] = None):
        raise NotImplementedError("rename not impl for base class")

    def change_to_temp(self, search: int):
        raise NotImplementedError("change_to_temp not impl for KernelArg")

    def calc_offset(self):
        raise NotImplementedError("calc_offset not available to kernel arg")


class NoneKernelArg(KernelArg):
    def __repr__(self):
        return "None"

    def rename(self, fr, to, change_access=None):
        raise NotImplementedError("Rename on none kernel arg")

    def is_none(self):
        return True


class KMatrix(KernelArg):
    def __init__(self, kern_id: int, access: Expression, shape: List[int]):
        self.id = kern_id
        self.access = access
        self.shape = shape
        self.is_temp = False
        self.offset = None

    def __repr__(self):
        if self.is_temp:
            return f"Temp {self.id}"
        return f"Mat (id: {self.id}, {self.access!r})"

    def get_ids(self, filter_temp=False):
        if filter_temp and self.is_temp:
            return []
        return [self.id]

    def rename(self, fr, to, change_access=None):
        if self.id == fr:
            self.id = to
            if change_access is not None:
                self.access = change_access(self.access)

    def change_to_temp(self, search):
        if self.id == search:
            self.is_temp = True

    def calc_offset(self):
        """Element offset of a contiguous operand: ``Global`` -> 0,
        ``Global + c`` -> c, a constant access of a 1-element tensor -> c
        (kernalize/__init__.py:74-83)."""
        acc = self.access
        if isinstance(acc, Global):
            self.offset = 0
        elif (type(acc) is Add and isinstance(acc.a, Global) and type(acc.b) is Val
              and type(acc.b.v) is Constant):
            self.offset = acc.b.v.val
        elif type(acc) is Val and type(acc.v) is Constant and prod(self.shape) == 1:
            self.offset = acc.v.val
        else:
            raise Exception(f"Invalid Feeder setting: {acc}. Make sure to call .contigious before Global() ")


class KConcat(KernelArg):
    def __init__(self, karg_one: KernelArg, karg_two: KernelArg, condition: Expression, shape: List[int]):
        self.karg_one = karg_one
        self.karg_two = karg_two
        self.condition = condition      # true -> karg_two, false -> karg_one
        self.shape = shape

    def __repr__(self):
        from ..context import indent_str
        body = indent_str(f"1: {self.karg_one}\n2: {self.karg_two}\ncond: {self.condition}")
        return f"\nConcat (\n{body}\n)\n"

    def get_ids(self, filter_temp=False):
        ids = self.karg_one.get_ids(filter_temp)
        ids.extend(self.karg_two.get_ids(filter_temp))
        return list(set(ids))

    def rename(self, fr, to, change_access=None):
        self.karg_one.rename(fr, to, change_access)
        self.karg_two.rename(fr, to, change_access)

    def change_to_temp(self, search):
        self.karg_one.change_to_temp(search)
        self.karg_two.change_to_temp(search)


class KConstant(KernelArg):
    def __init__(self, constant: float):
        self.constant = constant

    def __repr__(self):
        return f"{self.constant}"

    def get_ids(self, filter_temp=False):
        return []

    def rename(self, fr, to, change_access=None):
        pass

    def change_to_temp(self, search):
        pass
