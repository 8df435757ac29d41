"""IR containers and the global id counters.

Restates autodiff/context.py:7-159.  ``Proc`` is the procedural IR the device
backend consumes; ``Block`` records construction order while a program is
traced; ``Context`` hands out ids.  Id allocation order decides node ids,
fusion ids, toposort tie-breaking and therefore arena offsets, so every id is
requested at the same point as in the reference.
"""
from typing import Callable, Dict, Optional, Tuple


def indent_str(obj, size: int = 1, s: str = "    ") -> str:
    pad = s * size
    return "\n".join(pad + line for line in str(obj).splitlines())


class Proc:
    """Ordered command list: nodes, fused groups, alloc entries, loops."""

    def __init__(self, proc):
        self.procedure = proc
        self.id = context.get_proc_id()

    def __repr__(self):
        out = ""
        for cmd in self.procedure:
            out += str(cmd) + "\n"
            if hasattr(cmd, "proc"):
                out += indent_str(str(cmd.get_proc())) + "\n"
        return out

    def insert(self, idx, val):
        self.procedure.insert(idx, val)

    def append(self, val):
        self.procedure.append(val)

    def walk(self, func: Callable, step_fused: bool = True, step_proc: bool = True):
        """Apply ``func(cmd, proc_id)`` to every command; ``None`` deletes it.

        Fused groups are entered when ``step_fused`` and loop bodies when
        ``step_proc`` (context.py:29-47)."""
        from .fusion.base import FuseBase
        from .node import Node
        for idx in range(len(self.procedure)):
            cmd = self.procedure[idx]
            if isinstance(cmd, FuseBase) and step_fused:
                cmd.nodes = [func(n, self.id) for n in cmd.nodes]
                cmd.nodes = [n for n in cmd.nodes if n is not None]
            elif isinstance(cmd, Node) and cmd.get_proc() is not None and step_proc:
                cmd.proc.walk(func, step_fused, step_proc)
            else:
                self.procedure[idx] = func(cmd, self.id)
        self.procedure = [c for c in self.procedure if c is not None]


class Block:
    """Nodes traced into one scope, keyed by id with their construction slot.

    A node is dropped from its block when a later node consumes it, so the
    block ends up holding the graph's sinks in construction order."""

    def __init__(self, id_override=None):
        self.nodes: Dict[int, Tuple[object, int]] = dict()
        self.position = 0
        self.id = id_override if id_override is not None else context.get_block_id()

    def add_to_dep(self, node):
        self.nodes[node.id] = (node, self.position)
        self.position += 1

    def __len__(self):
        return len(self.nodes)

    def remove_from_dep(self, other):
        if other.id in self.nodes:
            del self.nodes[other.id]

    def to_list(self):
        if isinstance(self.nodes, list):
            return self.nodes
        ordered = sorted(self.nodes.values(), key=lambda kv: kv[1])
        return [kv[0] for kv in ordered]

    def convert_to_nodes(self):
        if isinstance(self.nodes, list):
            return
        self.nodes = self.to_list()

    def __repr__(self):
        return "\n".join(f"{i + 1}) {n!r}" for i, n in enumerate(self.nodes)) + "\n"


class Context:
    """Global tracing state (context.py:96-157)."""

    def __init__(self):
        self.id = -1
        self.proc_id = -1
        self.block_id = 0
        self.program_id = -1
        self.grads_seen = dict()
        self.connections = dict()
        self.conn_seen = set()
        self.procedure = [Block(0)]
        self.lock_proc = False

    def reset(self):
        """Start a fresh program (the reference relies on process isolation)."""
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
        self.procedure.append(Block())

    def pop_proc(self):
        assert len(self.procedure) > 1, "Attempt to pop main procedure!"
        ret = self.procedure.pop(-1)
        ret.convert_to_nodes()
        return ret

    def prep_exec(self):
        self.lock_proc = True
        self.procedure[0].convert_to_nodes()

    def get_id(self):
        self.id += 1
        return self.id

    def get_proc_id(self):
        self.proc_id += 1
        return self.proc_id

    def get_block_id(self):
        self.block_id += 1
        return self.block_id

    def get_prog_id(self):
        self.program_id += 1
        return self.program_id

    def __repr__(self):
        return repr(self.procedure[0])

    def main_proc(self):
        return self.procedure[0]


context = Context()
