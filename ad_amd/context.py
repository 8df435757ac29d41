"""Tracing state and the procedural IR container.

* ``Block`` -- the scope a program is traced into (the main program, or the
  body of an ``ir_for``).  It keeps the nodes no later node has consumed,
  in construction order: the sinks the compiler starts from.
* ``Proc`` -- the procedural IR: an ordered command list (nodes, fused
  groups, allocation commands, loops whose body is a ``Proc``) that a
  device executes in order.
* ``context`` -- the single global tracer: the open blocks and the id
  sequences.  Node ids, fusion ids, Proc ids and program ids are handed out
  at the same points as in the reference (autodiff/context.py:96-157), since
  every later pass orders its work by them.
"""
from typing import Callable, Dict, List


def indent_str(obj, size: int = 1, s: str = "    ") -> str:
    """``obj`` printed with every line indented ``size`` times by ``s``."""
    pad = s * size
    return "\n".join(pad + line for line in str(obj).splitlines())


class Proc:
    """An ordered command list with an id of its own."""

    def __init__(self, proc: List):
        self.procedure = proc
        self.id = context.get_proc_id()

    def __repr__(self):
        parts = []
        for cmd in self.procedure:
            parts.append(f"{cmd}\n")
            if hasattr(cmd, "proc"):               # a loop: its body, indented
                parts.append(indent_str(cmd.get_proc()) + "\n")
        return "".join(parts)

    def insert(self, idx, val):
        self.procedure.insert(idx, val)

    def append(self, val):
        self.procedure.append(val)

    def walk(self, func: Callable, step_fused: bool = True, step_proc: bool = True):
        """Replace every command ``c`` by ``func(c, self.id)`` in place; a
        ``None`` result deletes it.  With ``step_fused`` the members of a
        fused group are visited instead of the group, with ``step_proc`` the
        commands of a loop body (with that body's id) instead of the loop."""
        from .fusion.base import FuseBase
        from .node import Node
        for i, cmd in enumerate(self.procedure):
            if step_fused and isinstance(cmd, FuseBase):
                for j, member in enumerate(cmd.nodes):
                    cmd.nodes[j] = func(member, self.id)
                cmd.nodes = [m for m in cmd.nodes if m is not None]
            elif step_proc and isinstance(cmd, Node) and cmd.get_proc() is not None:
                cmd.proc.walk(func, step_fused, step_proc)
            else:
                self.procedure[i] = func(cmd, self.id)
        self.procedure = [c for c in self.procedure if c is not None]


class Block:
    """Traced scope.  While tracing, ``nodes`` maps id -> node for the nodes
    not yet consumed, in construction order; ``convert_to_nodes`` freezes it
    into that ordered list, which the compile passes then edit."""

    def __init__(self, id_override=None):
        self.nodes: Dict[int, object] = {}
        self.id = context.get_block_id() if id_override is None else id_override

    def add_to_dep(self, node):
        self.nodes.pop(node.id, None)
        self.nodes[node.id] = node

    def remove_from_dep(self, other):
        self.nodes.pop(other.id, None)

    def __len__(self):
        return len(self.nodes)

    def to_list(self):
        return self.nodes if isinstance(self.nodes, list) else list(self.nodes.values())

    def convert_to_nodes(self):
        self.nodes = self.to_list()

    def __repr__(self):
        return "".join(f"{i}) {n!r}\n" for i, n in enumerate(self.nodes, start=1))


class Context:
    """The global tracer: the stack of open blocks (``procedure[0]`` is the
    main program) and the id sequences."""

    def __init__(self):
        self._next = {"node": 0, "proc": 0, "block": 1, "program": 0}
        self.grads_seen = {}          # state of the reverse pass (node.backward)
        self.connections = {}
        self.conn_seen = set()
        self.procedure = [Block(0)]
        self.lock_proc = False        # set once compilation starts: no more tracing

    def _take(self, kind):
        value = self._next[kind]
        self._next[kind] = value + 1
        return value

    def get_id(self):
        return self._take("node")

    def get_proc_id(self):
        return self._take("proc")

    def get_block_id(self):
        return self._take("block")

    def get_prog_id(self):
        return self._take("program")

    def reset(self):
        """Forget the traced program: fresh ids and an empty main block (the
        reference gets this from running each program in its own process)."""
        self.__init__()
        from . import helper, linearize
        from .opt import simplify as opt_simplify
        helper.visited.clear()
        linearize.reset_state()
        opt_simplify.reset_state()

    def add_to_dep(self, node):
        if not self.lock_proc:
            self.procedure[-1].add_to_dep(node)

    def remove_from_dep(self, other):
        if not self.lock_proc:
            self.procedure[-1].remove_from_dep(other)

    def add_proc(self):
        """Open the block of a loop body."""
        self.procedure.append(Block())

    def pop_proc(self):
        """Close the innermost loop body and return its frozen block."""
        assert len(self.procedure) > 1, "no loop body is open; the main block stays"
        block = self.procedure.pop()
        block.convert_to_nodes()
        return block

    def prep_exec(self):
        self.lock_proc = True
        self.procedure[0].convert_to_nodes()

    def main_proc(self):
        return self.procedure[0]

    def __repr__(self):
        return repr(self.procedure[0])


context = Context()
