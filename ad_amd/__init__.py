"""ad_amd -- the ``ad`` ahead-of-time reverse-mode autodiff compiler with an
MI355X-native execution backend.

Public API as in autodiff/__init__.py:14-106: ``concat``, ``dot``,
``execute``, ``ir_for``, ``pg`` plus the node kinds.  ``execute`` runs the
reference's compile passes in the reference's order and hands the finished
procedural IR to a device backend; the backend is chosen by the ``device``
argument or the ``AD_DEVICE`` environment variable (``hip`` by default).
"""
import functools
import os
import sys
from math import prod
from typing import Callable, List

from .context import context
from .graph import (ConcatNode, Feeder, Node, Receiver, Tensor)  # noqa: F401
from .graph import *  # noqa: F401,F403

# Traced graphs are walked recursively; a 4-layer transformer step is far
# deeper than CPython's default limit.
if sys.getrecursionlimit() < 200000:
    sys.setrecursionlimit(200000)


def concat(nodes: List[Tensor], dim: int):
    """Left-nested ConcatNode chain along ``dim``, empty operands skipped
    (the behaviour of __init__.py:14-26)."""
    return functools.reduce(lambda joined, n: ConcatNode(joined, n, dim),
                            [n for n in nodes if prod(n.shape) != 0])


def dot(left: Node, right: Node) -> Node:
    from .graph import DotProdNode
    return DotProdNode(left, right)


def compile_proc():
    """Run every compile pass of autodiff/__init__.py:44-78 and return the
    allocated, program-id-numbered Proc."""
    from .alloc import alloc
    from .fusion.base import FuseBase
    from .kernalize.kernalize import kernalize
    from .linearize import linearize
    from .opt import dep_opt, mem_opt, repeat_opt, set_in_place
    from .opt.simplify import simpl_node

    context.prep_exec()
    dep_opt(context)
    simpl_node(context)
    repeat_opt(context)
    kernalize(context)
    proc = linearize(context.main_proc())
    proc = set_in_place(proc)
    proc = mem_opt(proc)
    alloc(proc)

    def number(cmd, _):
        # every command, loop bodies included, fused groups as one
        if isinstance(cmd, (Node, FuseBase)):
            cmd.program_id = context.get_prog_id()
        return cmd
    proc.walk(number, step_fused=False, step_proc=True)
    return proc


def make_device(device=None):
    name = device if device is not None else os.environ.get("AD_DEVICE", "hip")
    if not isinstance(name, str):
        return name
    if name == "hip":
        from .device.hip import HIPDevice
        return HIPDevice()
    raise ValueError(f"unknown device {name!r} (the product backend is 'hip')")


def execute(device=None):
    """Compile the traced program and run it (autodiff/__init__.py:34-85)."""
    proc = compile_proc()
    dev = make_device(device)
    dev.execute(proc)
    return proc


def ir_for(r: range, f: Callable):
    """Trace ``f`` once as the body of a loop run ``len(r)`` times."""
    from .graph import ForNode
    context.add_proc()
    f()
    proc = context.pop_proc()
    ForNode(proc, r)


def pg():
    print(context)


def reset():
    """Forget the traced program (fresh ids, empty main block)."""
    context.reset()
