"""HIPDevice -- the reference's device protocol on an MI355X.

Mirrors ``OpenCLDevice`` (autodiff/device/opencl/device.py:16-146): ``init``
and ``run`` dispatch on the command kind, ``_run_proc`` walks a Proc and
replays loop bodies, ``execute`` runs both passes.  Differences by design:

* every buffer lives in ONE device allocation (the arena) at a 256-byte
  aligned offset; the tetris region keeps the allocator's float offsets;
* kernels are generated per command (``codegen``), deduplicated by source
  text and compiled in parallel through hipRTC at the end of the init pass;
* a loop body without Receivers is captured once as a HIP graph and the
  graph is replayed ``len(r)`` times; a Feeder inside it copies from its own
  staging slot, refilled from the host before each replay;
* a Feeder writes at its arena offset (the reference OpenCL backend writes
  at offset 0, cl_helper.py:316,326 -- see ``oracle``);
* after the run, every Tensor's host array is refreshed from the device, as
  the reference's CL_MEM_USE_HOST_PTR buffers are on a CPU device.
"""
import os
import threading
from concurrent.futures import ThreadPoolExecutor
from math import prod

import numpy as np

from ...alloc import AllocEntry, DeallocEntry
from ...fusion import FuseBase
from ...graph import Feeder, ForNode, Receiver
from ...node import Node
from .. import Device
from . import codegen
from .runtime import HEADER_PATH, Context, compile_source

ALIGN = 256
_code_cache = {}            # source text -> code object (process-wide)
_code_lock = threading.Lock()


def _align(n):
    return (n + ALIGN - 1) // ALIGN * ALIGN


def _header():
    with open(HEADER_PATH) as fh:
        return fh.read()


class HIPDevice(Device):
    def __init__(self, device_index: int = 0, use_graphs: bool = True, jit_threads: int = None):
        super().__init__()
        self.kernels = {}            # program_id -> [KernelPlan]
        self.funcs = {}              # program_id -> launch callable
        self.buffers = {}            # buffer id -> arena byte offset
        self.buffers_size = {}       # buffer id -> floats
        self.use_graphs = use_graphs
        self.jit_threads = jit_threads or min(16, (os.cpu_count() or 4))
        self.ctx = Context(device_index)
        self._allocs = []
        self._contents = {}
        self._pending = []
        self._feeder_slots = {}      # feeder id -> staging byte offset
        self._graphs = {}            # ForNode id -> graph handle
        self.stats = {"kernels": 0, "unique_sources": 0, "lockstep_cmds": 0, "launches_per_iter": 0}

    # ------------------------------------------------------------------ init pass
    def init(self, cmd):
        if isinstance(cmd, Feeder):
            cmd.kres.calc_offset()
            self._feeder_slots[cmd.id] = None
            return
        if isinstance(cmd, Receiver):
            cmd.offsets, cmd.shapes, cmd.ids = [], [], []
            for k in cmd.kargs:
                k.calc_offset()
                cmd.ids.append(k.id)
                cmd.shapes.append(k.shape)
                cmd.offsets.append(k.offset)
            return
        if isinstance(cmd, AllocEntry):
            if not cmd.is_temp:
                self._allocs.append(cmd)
            return
        if isinstance(cmd, (DeallocEntry, ForNode)):
            return
        if isinstance(cmd, (Node, FuseBase)):
            self._pending.append(cmd)
            return
        raise AssertionError(f"Encountered unexpected cmd: {cmd}")

    def _layout(self):
        """Arena: every non-temp AllocEntry, then Feeder staging slots, then
        scratch for lockstep commands."""
        off = 0
        info = codegen.BufferInfo()
        for a in self._allocs:
            self.buffers[a.id] = off
            self.buffers_size[a.id] = a.size
            info.size[a.id] = a.size
            if a.content is not None:
                self._contents[a.id] = a.content
            off += _align(a.size * 4)
        return off, info

    def _finish_init(self):
        off, info = self._layout()
        # Feeder staging slots (used when a Feeder runs inside a captured graph)
        for fid in list(self._feeder_slots):
            self._feeder_slots[fid] = off
            size = self._feeder_size.get(fid, 0)
            off += _align(size * 4)
        scratch_base = off
        # generate plans
        scratch_need = 0
        plans = {}
        for cmd in self._pending:
            ps, need, lockstep = codegen.command_plans(cmd, info, 0)
            plans[cmd.program_id] = ps
            scratch_need = max(scratch_need, need)
            self.stats["lockstep_cmds"] += int(lockstep)
        off += _align(scratch_need * 4)
        self.ctx.reserve(max(off, ALIGN))
        self.scratch_off = scratch_base
        for bid, content in self._contents.items():
            assert content.dtype == np.float32, "Content is not np.float32"
            self.ctx.write(self.buffers[bid], np.ascontiguousarray(content))
        self._compile_and_bind(plans)
        self._pending = []

    def _compile_and_bind(self, plans):
        header = _header()
        sources = {}
        for ps in plans.values():
            for p in ps:
                sources.setdefault(p.source, p.name)
        todo = [s for s in sources if s not in _code_cache]

        def build(src):
            return src, compile_source(header + src)
        if todo:
            with ThreadPoolExecutor(self.jit_threads) as pool:
                for src, code in pool.map(build, todo):
                    with _code_lock:
                        _code_cache[src] = code
        funcs = {}
        for src, name in sources.items():
            mod = self.ctx.load_module(_code_cache[src])
            funcs[src] = (mod, self.ctx.function(mod, name))
        self.stats["unique_sources"] += len(sources)
        for pid, ps in plans.items():
            launches = []
            for p in ps:
                args = []
                for a in p.args:
                    if a[0] == "buf":
                        args.append(self.ctx.base + self.buffers[a[1]] + 4 * a[2])
                    elif a[0] == "scratch":
                        args.append(self.ctx.base + self.scratch_off + 4 * a[1])
                    else:
                        args.append(a[1])
                launches.append(self.ctx.launcher(funcs[p.source][1], p.grid, p.block, p.shared, args))
            self.kernels[pid] = ps
            self.stats["kernels"] += len(ps)
            if len(launches) == 1:
                self.funcs[pid] = launches[0]
            else:
                self.funcs[pid] = (lambda ls=launches: [f() for f in ls])

    # ------------------------------------------------------------------ run pass
    def run(self, cmd):
        if isinstance(cmd, (AllocEntry, DeallocEntry, ForNode)):
            return
        if isinstance(cmd, Feeder):
            if self._capturing:
                # inside a graph: copy this iteration's data from the staging slot
                dst = self.buffers[cmd.kres.id] + 4 * cmd.kres.offset
                self.ctx.copy(dst, self._feeder_slots[cmd.id], 4 * prod(cmd.shape))
                self._graph_feeders.append(cmd)
                return
            arr = self._feeder_value(cmd)
            self.ctx.write(self.buffers[cmd.kres.id] + 4 * cmd.kres.offset, arr)
            return
        if isinstance(cmd, Receiver):
            outs = []
            for bid, shape, off in zip(cmd.ids, cmd.shapes, cmd.offsets):
                out = np.empty(shape, dtype=np.float32)
                self.ctx.read(self.buffers[bid] + 4 * off, out)
                outs.append(out)
            cmd.func(*outs)
            return
        self.funcs[cmd.program_id]()

    @staticmethod
    def _feeder_value(cmd):
        arr = cmd.func()
        assert isinstance(arr, np.ndarray) and list(arr.shape) == list(cmd.shape), "Invalid function"
        return np.ascontiguousarray(arr, dtype=np.float32)

    def _capturable(self, proc):
        return not any(isinstance(c, (Receiver, ForNode)) for c in proc.procedure)

    def _run_loop(self, cmd, iterations=None):
        inner = cmd.get_proc()
        reps = len(cmd.r) if iterations is None else iterations
        if reps <= 0:
            return
        if not (self.use_graphs and self._capturable(inner)):
            for _ in range(reps):
                self._run_proc(inner, self.run, False)
            return
        g = self._graphs.get(cmd.id)
        if g is None:
            self._capturing = True
            self._graph_feeders = []
            self.ctx.graph_begin()
            try:
                self._run_proc(inner, self.run, False)
            finally:
                self._capturing = False
                g = self.ctx.graph_end()
            self._graphs[cmd.id] = (g, self._graph_feeders)
        else:
            g, feeders = g
            self._graph_feeders = feeders
        g = self._graphs[cmd.id][0]
        feeders = self._graphs[cmd.id][1]
        for _ in range(reps):
            for f in feeders:
                self.ctx.write(self._feeder_slots[f.id], self._feeder_value(f))
            self.ctx.graph_launch(g)

    def _run_proc(self, proc, func, init=False):
        for cmd in proc.procedure:
            if isinstance(cmd, ForNode):
                inner = cmd.get_proc()
                assert inner is not None, "Inner proc is None!"
                if init:
                    self._run_proc(inner, func, init)
                else:
                    self._run_loop(cmd)
            else:
                func(cmd)

    # ------------------------------------------------------------------ driver
    def prepare(self, proc):
        """Init pass: layout, upload, JIT."""
        self._capturing = False
        self._feeder_size = {}

        def note_feeders(c, _):
            if isinstance(c, Feeder):
                self._feeder_size[c.id] = prod(c.shape)
            return c
        proc.walk(note_feeders, step_fused=False, step_proc=True)
        self._run_proc(proc, self.init, init=True)
        self._finish_init()

    def execute(self, proc):
        self.prepare(proc)
        self._run_proc(proc, self.run, init=False)
        self.ctx.sync()
        self.refresh_tensors()

    # ------------------------------------------------------------------ timing hooks
    def loops(self, proc):
        """The ``ForNode`` commands of the top-level Proc, in order."""
        return [c for c in proc.procedure if isinstance(c, ForNode)]

    def replay(self, loop_cmd, iterations: int):
        """Run ``iterations`` more iterations of a prepared loop body (a graph
        replay each when the body is capturable)."""
        self._run_loop(loop_cmd, iterations)

    def launch(self, cmd):
        """Enqueue one prepared compute command."""
        self.funcs[cmd.program_id]()

    def refresh_tensors(self):
        """Copy every Tensor buffer back into its host array."""
        for bid, content in self._contents.items():
            out = np.empty(content.size, dtype=np.float32)
            self.ctx.read(self.buffers[bid], out)
            content.reshape(-1)[:] = out

    def close(self):
        for g, _ in self._graphs.values():
            self.ctx.graph_destroy(g)
        self._graphs = {}
        self.ctx.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
