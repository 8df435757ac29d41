"""Allocation planning: Alloc/Dealloc insertion, register temps, the
"tetris" arena packer and hoisting (autodiff/alloc/)."""
from dataclasses import dataclass
from typing import Optional

__all__ = ["LocationBase", "Location", "AllocCmds", "AllocEntry", "DeallocEntry", "alloc"]


@dataclass
class LocationBase:
    fused_id: Optional[int]
    proc_id: Optional[int]

    def __hash__(self):
        return hash((self.fused_id, self.proc_id))


@dataclass
class Location:
    loc: int
    fused_id: Optional[int]
    proc_id: Optional[int]

    def __add__(self, other):
        if type(other) == int:
            return Location(self.loc + other, fused_id=self.fused_id, proc_id=self.proc_id)
        raise TypeError(f"Invalid type for add loc: {type(other)}")

    def base(self) -> LocationBase:
        return LocationBase(fused_id=self.fused_id, proc_id=self.proc_id)


class AllocCmds:
    pass


class AllocEntry(AllocCmds):
    """Buffer ``id`` of ``size`` floats; ``content`` is a Tensor's host data."""

    def __init__(self, alloc_id: int, size: int, content=None):
        self.id = alloc_id
        self.size = size
        self.content = content
        self.is_temp = False

    def __repr__(self):
        head = "TEMP Alloc" if self.is_temp else "Alloc"
        size = "" if self.is_temp else f" {self.size}"
        return f"{head} {self.id}{size}" + (" (has content)" if self.content is not None else "")


class DeallocEntry(AllocCmds):
    def __init__(self, dealloc_id: int, size: int):
        self.id = dealloc_id
        self.size = size
        self.is_temp = False

    def __repr__(self):
        return f"{'TEMP ' if self.is_temp else ''}Dealloc {self.id} {self.size}"


def alloc(proc):
    """insert_alloc -> temp_alloc -> tetris_opt -> temp_clean
    (alloc/__init__.py:59-76)."""
    from .clean import temp_clean
    from .insert import insert_alloc
    from .temp import temp_alloc
    from .tetris_opt import tetris_opt
    fused = insert_alloc(proc)
    temp_alloc(proc, fused)
    tetris_opt(proc)
    temp_clean(proc)
    return proc
