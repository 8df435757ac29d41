"""Lifetimes to allocation commands (autodiff/alloc/insert.py:10-125).

Every command is visited at a *slot*: its index in its container (the main
Proc, a loop body, or a fused group's node list).  A buffer gets an
``AllocEntry`` at the slot of its first definition and a ``DeallocEntry``
one slot after its latest read; a result nobody reads is released at the
end of the main Proc.  Tensors become ``AllocEntry`` commands that carry
their host array.  The entries are then inserted container by container in
slot order; each insertion shifts the later slots of its container by one.

Three behaviours of the reference are kept because the tetris packing (and
so every arena offset) depends on them:

* a result defined again with a larger size keeps its first Alloc's size
  (insert.py:31 records the larger size on the location object instead);
* commands of a loop body are keyed by the *enclosing* Proc's id and
  inserted into the loop body registered last under that id
  (insert.py:68-70);
* the sort of all entries is stable, releases listed before allocations,
  each list in the order its buffer was first entered.
"""
from math import prod

from ..fusion import FuseBase
from ..fusion.helper import get_deps, get_res
from ..graph import Receiver, Tensor
from ..node import Node
from . import AllocEntry, DeallocEntry


class _Planner:
    def __init__(self, main_proc):
        self.main = main_proc
        self.first_def = {}        # buffer -> (slot key, AllocEntry); first definition only
        self.last_read = {}        # buffer -> (slot key, DeallocEntry); overwritten by later reads
        self.consumed = {}         # result id -> read by some command
        self.size_of = {}          # buffer -> floats
        self.groups = {}           # fuse_id -> group
        self.bodies = {}           # enclosing Proc id -> loop body (the last one seen)

    # slot keys: (loop key or None, fuse id or None, index)
    def visit(self, proc, loop_key=None):
        for index, cmd in enumerate(proc.procedure):
            if isinstance(cmd, FuseBase):
                self.groups[cmd.fuse_id] = cmd
                for member_index, member in enumerate(cmd.nodes):
                    if isinstance(member, Tensor):
                        cmd.nodes[member_index] = self._tensor_alloc(member)
                    else:
                        self._command(member, (None, cmd.fuse_id, member_index))
                continue
            if not isinstance(cmd, Node):
                raise TypeError(f"cannot plan allocations around a {type(cmd).__name__}")
            if isinstance(cmd, Tensor):
                proc.procedure[index] = self._tensor_alloc(cmd)
            elif cmd.get_proc() is not None:
                self.bodies[proc.id] = cmd.proc
                self.visit(cmd.proc, proc.id)
            else:
                self._command(cmd, (loop_key, None, index))

    def _tensor_alloc(self, t):
        self.size_of[t.id] = prod(t.shape)
        return AllocEntry(t.id, prod(t.shape), t.arr)

    def _command(self, node, slot):
        if not isinstance(node, Receiver):
            size = prod(node.shape)
            (res,) = list(get_res(node))
            if res not in self.first_def:
                if res in self.size_of:
                    # an in-place update writes a buffer that already exists
                    assert self.size_of[res] == size, \
                        f"in-place update of buffer {res} changes its size ({self.size_of[res]} -> {size})"
                else:
                    self.first_def[res] = (slot, AllocEntry(res, size))
            self.consumed[node.id] = False
            self.size_of[node.id] = size
        after = (slot[0], slot[1], slot[2] + 1)
        for dep in list(get_deps(node)):
            self.last_read[dep] = (after, DeallocEntry(dep, self.size_of[dep]))
            self.consumed[dep] = True

    def emit(self):
        end = (None, None, len(self.main.procedure))
        for buf in [b for b, read in self.consumed.items() if not read]:
            self.last_read[buf] = (end, DeallocEntry(buf, self.size_of[buf]))
        entries = list(self.last_read.values()) + list(self.first_def.values())
        entries.sort(key=lambda e: (-1 if e[0][0] is None else e[0][0], -1 if e[0][1] is None else e[0][1], e[0][2]))
        shift = {}
        for (loop_key, fuse_id, index), entry in entries:
            container = (fuse_id, loop_key)
            at = index + shift.get(container, 0)
            if fuse_id is not None:
                self.groups[fuse_id].nodes.insert(at, entry)
            elif loop_key is not None:
                self.bodies[loop_key].insert(at, entry)
            else:
                self.main.insert(at, entry)
            shift[container] = shift.get(container, 0) + 1


def insert_alloc(main_proc):
    """Insert the Alloc/Dealloc commands; returns the fused groups by
    fuse id (the next pass marks their register temps)."""
    planner = _Planner(main_proc)
    planner.visit(main_proc)
    planner.emit()
    return planner.groups
