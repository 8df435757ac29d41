"""Allocation planning of a linearized Proc (autodiff/alloc/__init__.py:59-76):

1. ``insert_alloc`` -- an ``AllocEntry`` before each buffer's first
   definition and a ``DeallocEntry`` after its last read;
2. ``temp_alloc`` -- buffers born and dead inside one fused group become
   register temps;
3. ``tetris_opt`` -- the remaining buffers of each Proc are packed into one
   shared region by lifetime;
4. ``temp_clean`` -- leftover allocations hoisted to the front, releases to
   the end.

The entries print as the reference's listings show them."""

__all__ = ["AllocCmds", "AllocEntry", "DeallocEntry", "alloc"]


class AllocCmds:
    """Marker base of the allocation commands in a Proc."""


class AllocEntry(AllocCmds):
    """Buffer ``id`` of ``size`` floats; ``content`` is the host array of a
    Tensor it is initialised from, if any; ``is_temp`` marks a register temp
    of a fused group."""

    def __init__(self, alloc_id: int, size: int, content=None):
        self.id = alloc_id
        self.size = size
        self.content = content
        self.is_temp = False

    def __repr__(self):
        if self.is_temp:
            text = f"TEMP Alloc {self.id}"
        else:
            text = f"Alloc {self.id} {self.size}"
        return text + (" (has content)" if self.content is not None else "")


class DeallocEntry(AllocCmds):
    """Release of buffer ``id`` (``size`` floats)."""

    def __init__(self, dealloc_id: int, size: int):
        self.id = dealloc_id
        self.size = size
        self.is_temp = False

    def __repr__(self):
        return ("TEMP " if self.is_temp else "") + f"Dealloc {self.id} {self.size}"


def alloc(proc):
    from .clean import temp_clean
    from .insert import insert_alloc
    from .temp import temp_alloc
    from .tetris_opt import tetris_opt
    temp_alloc(proc, insert_alloc(proc))
    tetris_opt(proc)
    temp_clean(proc)
    return proc
