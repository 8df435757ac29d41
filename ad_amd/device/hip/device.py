"""HIPDevice -- the reference's device protocol on an MI355X.

Mirrors ``OpenCLDevice`` (autodiff/device/opencl/device.py:16-146): ``init``
and ``run`` dispatch on the command kind, ``_run_proc`` walks a Proc and
replays loop bodies, ``execute`` runs both passes.  Differences by design:

* every buffer lives in ONE device allocation (the arena) at a 256-byte
  aligned offset; the tetris region keeps the allocator's float offsets;
  after the buffers come the Feeder staging slots, the scratch region of
  multi-pass commands and the kernel argument tables;
* kernels are generated per command (``codegen``), deduplicated by source
  text and compiled in parallel through hipRTC at the end of the init pass;
  every kernel reads its arguments from a row of an argument table;
* each stretch of commands between Feeders/Receivers/loops is scheduled
  (``schedule``): launches ordered by their memory conflicts, independent
  launches of one kernel merged into one launch; the groups can be spread
  over several streams with event edges only where they touch overlapping
  memory (``lanes``; one stream by default, see the class notes);
* a loop body without nested loops is captured once as a HIP graph and the
  graph is replayed ``len(r)`` times (short bodies without Receivers also as
  graphs of several iterations); a Feeder inside it copies from its staging
  slot, which the host refills on a transfer stream while the previous
  launch computes (two sets of slots and graphs); a Receiver inside
  it copies its data into one of two snapshot slots, which the transfer
  stream brings to pinned host memory after the iteration, and its
  callback runs before the next iteration is launched (``receiver_lag``
  0) or one iteration later (1);
* a Feeder writes at its arena offset (the reference OpenCL backend writes
  at offset 0, cl_helper.py:316,326; ``feeder_offset_zero`` does that);
* after the run, every Tensor's host array is refreshed from the device, as
  the reference's CL_MEM_USE_HOST_PTR buffers are on a CPU device.
"""
import os
import threading
from concurrent.futures import ThreadPoolExecutor
from math import prod

import numpy as np

from ...alloc import AllocEntry, DeallocEntry
from ...fusion import DPElwFuse, FuseBase, ReduceElwFuse
from ...graph import Feeder, ForNode, Receiver
from ...node import Node
from .. import Device
from . import codegen
from .runtime import HEADER_PATH, Context, compile_source
from .schedule import assign_lanes, schedule_dag

ALIGN = 256
SCRATCH_RING_FLOATS = 64 << 20     # 256 MiB of scratch slots for multi-pass commands
UNROLL_LAUNCHES = 256              # kernel commands per unrolled loop graph, at most
_code_cache = {}            # source text -> code object (process-wide)
_code_lock = threading.Lock()


def _align(n):
    return (n + ALIGN - 1) // ALIGN * ALIGN


def _header():
    with open(HEADER_PATH) as fh:
        return fh.read()


class _Launch:
    """One kernel launch: a plan of a command, its argument row, the
    ranges it reads and writes."""
    __slots__ = ("cmd", "plan", "args", "reads", "writes")

    def __init__(self, cmd, plan, args, reads, writes):
        self.cmd, self.plan, self.args, self.reads, self.writes = cmd, plan, args, reads, writes


def _transitive_reduction(deps):
    """The same order with the fewest edges: an edge j -> i is dropped when
    another dependency of i already follows j."""
    before, out = [], []
    for d in deps:
        reach = 0
        for j in d:
            reach |= before[j] | (1 << j)
        before.append(reach)
        out.append([j for j in d if not any(before[k] >> j & 1 for k in d if k != j)])
    return out


class HIPDevice(Device):
    """The reference's device protocol on one MI355X (see the module notes).

    Options (defaults give the reference's results):

    * ``use_graphs`` -- replay loop bodies as HIP graphs (else launch by launch);
    * ``group_launches`` -- run independent launches of one kernel as one
      launch (argument rows selected by ``blockIdx.z``);
    * ``lanes`` -- streams for independent launch groups in uncaptured runs.
      Capture always uses one: capturing the C4 training step on four lanes
      ended in a host segmentation fault inside
      hipStreamEndCapture/hipGraphInstantiate whose cause is not established;
    * ``loop_unroll`` -- a loop body without Receivers is also captured as a
      graph of up to this many consecutive iterations (at most
      ``UNROLL_LAUNCHES`` kernel commands per graph);
    * ``receiver_lag`` -- a Receiver inside a replayed loop calls back before
      the next iteration is launched (0, the reference's order) or one
      iteration later (1: the next iteration computes meanwhile, and its
      Feeders are called first);
    * ``exact_reduce`` -- reductions combine all R elements (the reference's
      work-group tree drops elements for non-power-of-two lengths and pads
      MAX with 0, reduce.py:33-43);
    * ``feeder_offset_zero`` -- a Feeder writes at offset 0 of its buffer, as
      the OpenCL backend does (cl_helper.py:316,326); by default it honours
      the arena offset, as the CUDA backend does (cuda_helper.py:117-119);
    * ``strict_temps`` -- raise on a fused temp read through a non-identity
      access, which the reference silently reads as the element's own value
      (karg.py:47-48);
    * ``dot_precision`` -- "bf16" (beyond the reference, which computes in
      fp32): the operands of DotProds of at least ``bf16_min_macs``
      multiply-adds (2^30 by default: smaller products gain less than their
      operand packing costs) rounded to bfloat16, products summed in fp32 on
      bf16 MFMA;
    * ``arena`` -- "packed" (the reference's layout: every tetris variable
      at its packed offset, variables with disjoint lifetimes sharing
      memory) or "unpacked" (beyond the reference: every tetris variable in
      storage of its own, so reuse of memory between variables orders no
      launches; costs the sum of the variables' sizes instead of the packed
      high-water mark);
    * ``graph_dag`` -- a captured loop body keeps only the dependencies the
      schedule found (launches touching overlapping memory, one writing, in
      Proc order; transitively reduced), so independent launches may run at
      the same time; off (the default), the graph is the captured chain.
      Measured on C5 (647 launches, critical path 11.3 of 16.8 ms of kernel
      time, at most 10 launches side by side): 16.74 against 16.68 ms per
      step, C4 1.631 against 1.620 ms -- the runtime gains nothing from the
      parallel branches;
    * ``stream_min_bytes`` -- float4 reads of a range of at least this many
      bytes that no other command reads (and no loop iteration reads again),
      and writes of such a range no command reads, bypass the caches
      (nontemporal), so they do not evict data that is read again (None:
      never).  Results are unchanged;
    * ``narrow_launches`` -- a launch group of 64 x 64-tile products too
      small to fill the device (at most ``codegen.NARROW_MAX_BLOCKS`` blocks)
      runs the ``dp_quad`` kernel instead: 32 x 32 tiles, each block's K
      panels split among its four waves.  Sums are grouped differently
      (within the fp32 tolerance of any K split).
    """

    def __init__(self, device_index: int = 0, use_graphs: bool = True, jit_threads: int = None,
                 group_launches: bool = True, lanes: int = 1, receiver_lag: int = 0,
                 exact_reduce: bool = False, feeder_offset_zero: bool = False,
                 strict_temps: bool = False, dot_precision: str = "fp32", bf16_min_macs: int = 1 << 30,
                 loop_unroll: int = 32, arena: str = "packed", stream_min_bytes: int = 32 << 20,
                 graph_dag: bool = False, narrow_launches: bool = True):
        super().__init__()
        self.narrow_launches = narrow_launches
        self.graph_dag = graph_dag
        assert arena in ("packed", "unpacked"), "arena must be packed or unpacked"
        assert not (arena == "unpacked" and feeder_offset_zero), \
            "feeder_offset_zero writes into the packed arena; it needs arena='packed'"
        self.arena = arena
        self.stream_min_bytes = stream_min_bytes
        assert dot_precision in ("fp32", "bf16"), "dot_precision must be fp32 or bf16"
        assert receiver_lag in (0, 1), "receiver_lag must be 0 or 1"
        self.use_graphs = use_graphs
        self.group_launches = group_launches
        self.lanes = max(1, lanes)
        self.loop_unroll = max(1, loop_unroll)
        self.receiver_lag = receiver_lag
        self.exact_reduce = exact_reduce
        self.feeder_offset_zero = feeder_offset_zero
        self.strict_temps = strict_temps
        self._plan_opts = codegen.PlanOptions(exact_reduce=exact_reduce, dot=dot_precision,
                                              bf16_min_macs=bf16_min_macs)
        self.jit_threads = jit_threads or min(16, (os.cpu_count() or 4))
        self.ctx = Context(device_index)
        self._graphs = {}
        self._reset_program()

    def _reset_program(self):
        """Forget every per-program structure: the graphs of an earlier
        program (destroyed here, after the stream has drained, since they
        point into the arena the next layout replaces), its layout, plans,
        slots and schedules.  ``prepare`` starts from here, so one device can
        run several programs in turn, as the reference's device does by
        overwriting its dictionaries (device.py:46-91)."""
        self._destroy_graphs()
        self.kernels = {}            # program_id -> [KernelPlan]
        self.funcs = {}              # program_id -> launch callable (ungrouped)
        self.buffers = {}            # buffer id -> arena byte offset
        self.buffers_size = {}       # buffer id -> floats
        self._vars = {}              # tetris variable id -> (packed float offset, floats)
        self._var_off = {}           # tetris variable id -> arena byte offset (unpacked arena)
        self._events = 0             # event pool entries used by the schedules
        self._allocs = []
        self._contents = {}
        self._pending = []
        self._feeder_slots = {}      # feeder id -> staging byte offsets, [parity * unroll + u]
        self._feeder_loop = {}       # feeder id -> ForNode id of its loop body
        self._unroll = {}            # ForNode id -> iterations per unrolled graph
        self._recv_slots = {}        # in-loop receiver id -> (slot byte offset per parity, bytes)
        self._graphs = {}            # ForNode id -> ([single-iteration graph per parity], [unrolled graph per parity] or None, feeders, receivers)
        self._launches = {}          # ForNode id -> graph launches so far
        self._parity = 0
        self._slot = 0
        self._schedules = {}         # Proc id -> one-lane items (captured into graphs)
        self.stretch_graphs = {}     # Proc id -> per stretch, per launch group: (kernel, instances, deps, reads, writes, flops)
        self._lane_schedules = {}    # Proc id -> items over self.lanes lanes (uncaptured runs)
        self._narrow_plans = {}      # kernel name -> dp_quad plan some launch group takes
        self._capturing = False
        self.stats = {"kernels": 0, "unique_sources": 0, "multipass_cmds": 0, "launches_per_iter": 0}

    # ------------------------------------------------------------------ init pass
    def init(self, cmd):
        if isinstance(cmd, Feeder):
            cmd.kres.calc_offset()
            self._note_vars(cmd.kres)
            self._feeder_slots[cmd.id] = None
            return
        if isinstance(cmd, Receiver):
            cmd.offsets, cmd.shapes, cmd.ids, cmd.vars = [], [], [], []
            for k in cmd.kargs:
                k.calc_offset()
                self._note_vars(k)
                cmd.vars.append(getattr(k, "tetris_var", None))
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
            for n in (cmd.nodes if isinstance(cmd, FuseBase) else [cmd]):
                if not isinstance(n, Node):
                    continue
                for k in n.kargs:
                    self._note_vars(k)
                self._note_vars(n.kres)
            self._pending.append(cmd)
            return
        raise AssertionError(f"Encountered unexpected cmd: {cmd}")

    def _note_vars(self, karg):
        for km in codegen.iter_kmatrix(karg):
            var = getattr(km, "tetris_var", None)
            if var is not None:
                self._vars[var[0]] = (var[1], var[2])

    def _layout(self):
        """Byte offset of every non-temp buffer, in AllocEntry order; with the
        unpacked arena, then one region per tetris variable, by variable id."""
        off = 0
        info = codegen.BufferInfo(unpacked=self.arena == "unpacked")
        for a in self._allocs:
            self.buffers[a.id] = off
            self.buffers_size[a.id] = a.size
            info.size[a.id] = a.size
            if a.content is not None:
                self._contents[a.id] = a.content
            off += _align(a.size * 4)
        if info.unpacked:
            # each variable starts at the same address modulo ALIGN as at its
            # packed offset, so every alignment a kernel was planned for holds
            for vid in sorted(self._vars):
                voff, size = self._vars[vid]
                self._var_off[vid] = off + 4 * voff % ALIGN
                off = _align(self._var_off[vid] + 4 * size)
        return off, info

    def _mark_streams(self, proc, info):
        """Mark the float4 accesses that bypass the caches (``km.stream``):
        a read of a range (arena variable or buffer) that no other command
        reads and, inside a loop body, that the body itself writes (a range
        the body only reads is read again by the next iteration); a write of
        a range no command reads.  Only ranges of at least
        ``stream_min_bytes``: the caches keep smaller ones to good effect.
        Marks of an earlier device on the same Proc are cleared first."""
        readers, reads, writes = {}, [], []

        def nodes(cmd):
            return [n for n in (cmd.nodes if isinstance(cmd, FuseBase) else [cmd]) if isinstance(n, Node)]

        def body_writes(body):
            out = set()
            for c in body.procedure:
                if isinstance(c, ForNode):
                    out |= body_writes(c.get_proc())
                elif isinstance(c, (Node, FuseBase)) and not isinstance(c, Receiver):
                    for n in ([c] if isinstance(c, Feeder) else nodes(c)):
                        if not n.kres.is_none() and not n.kres.is_temp:
                            out.add(codegen._region(n.kres, info, coarse=True)[0])
            return out

        def scan(body, own):
            for c in body.procedure:
                if isinstance(c, ForNode):
                    scan(c.get_proc(), body_writes(c.get_proc()))
                    continue
                if isinstance(c, (Feeder, Receiver)) or not isinstance(c, (Node, FuseBase)):
                    continue
                for n in nodes(c):
                    for k in n.kargs:
                        for km in codegen.iter_kmatrix(k):
                            if km.is_temp or getattr(km, "scratch_offset", None) is not None:
                                continue
                            r = codegen._region(km, info, coarse=True)[0]
                            readers.setdefault(r, set()).add(c.program_id)
                            if own is not None and r not in own:
                                readers[r].add(None)        # read again every iteration
                            reads.append((km, r))
                    if not n.kres.is_none() and not n.kres.is_temp:
                        writes.append((n.kres, codegen._region(n.kres, info, coarse=True)[0]))
        scan(proc, None)
        for km, _ in reads + writes:
            km.stream = False
        big = self.stream_min_bytes
        if big is None:
            return
        for km, r in reads:
            if len(readers[r]) == 1 and 4 * (r[2] - r[1]) >= big:
                km.stream = True
        for km, r in writes:
            if r not in readers and 4 * (r[2] - r[1]) >= big:
                km.stream = True

    def _addr(self, bid, off, var):
        """Arena byte offset of float ``off`` of buffer ``bid``; ``var`` is the
        tetris variable (id, packed offset, size) the access belongs to, or
        None."""
        if var is not None and self._var_off:
            return self._var_off[var[0]] + 4 * (off - var[1])
        return self.buffers[bid] + 4 * off

    def _finish_init(self, proc):
        off, info = self._layout()
        for loop in self._all_loops(proc):
            body = loop.get_proc()
            n_cmds = sum(1 for c in body.procedure if isinstance(c, (Node, FuseBase))
                         and not isinstance(c, (Feeder, Receiver, ForNode)))
            has_recv = any(isinstance(c, Receiver) for c in body.procedure)
            self._unroll[loop.id] = 1 if has_recv or not self._capturable(body) else \
                max(1, min(self.loop_unroll, UNROLL_LAUNCHES // max(1, n_cmds)))
            for c in body.procedure:
                if isinstance(c, Feeder):
                    self._feeder_loop[c.id] = loop.id
        # two sets of staging slots per Feeder (one per iteration of an
        # unrolled graph): a replayed loop fills one set while the graph of
        # the previous launch reads the other
        for fid in list(self._feeder_slots):
            size = _align(self._feeder_size.get(fid, 0) * 4)
            count = 2 * self._unroll.get(self._feeder_loop.get(fid), 1)
            self._feeder_slots[fid] = [off + i * size for i in range(count)]
            off += count * size
        # two snapshot slots per Receiver in a capturable loop body: the graph
        # copies the Receiver's data there; the transfer stream fetches it
        fetch_bytes = [0]
        for loop in self._all_loops(proc):
            body = loop.get_proc()
            if not self._capturable(body):
                continue
            per_loop = 0
            for c in body.procedure:
                if isinstance(c, Receiver):
                    size = sum(_align(4 * prod(shape)) for shape in c.shapes)
                    self._recv_slots[c.id] = ((off, off + size), size)
                    off += 2 * size
                    per_loop += size
            fetch_bytes[0] = max(fetch_bytes[0], per_loop)
        # kernel plans and the ranges each command touches; commands that need
        # scratch get consecutive slots of a ring, so neighbouring commands do
        # not share scratch and can run in one launch
        self._mark_streams(proc, info)
        plans, regions, needs = {}, {}, {}
        for cmd in self._pending:
            if self.strict_temps:
                self._check_temps(cmd)
            ps, need, multipass = codegen.command_plans(cmd, info, 0, self._plan_opts)
            plans[cmd.program_id] = ps
            needs[cmd.program_id] = (need + 63) // 64 * 64
            regions[cmd.program_id] = codegen.command_regions(cmd, info)
            self.stats["multipass_cmds"] += int(multipass)
        max_need = max(needs.values(), default=0)
        ring = max(max_need, min(sum(needs.values()), SCRATCH_RING_FLOATS))
        self._scratch_base = {}
        cursor = 0
        for cmd in self._pending:
            need = needs[cmd.program_id]
            if need == 0:
                continue
            if cursor + need > ring:
                cursor = 0
            self._scratch_base[cmd.program_id] = cursor
            cursor += need
        self.scratch_off = off
        off += _align(ring * 4)
        # schedule every stretch of every Proc, then lay out argument tables
        rows = []                      # (byte offset in table region, [u64 values])
        table_bytes = [0]

        def add_rows(values_list):
            start = table_bytes[0]
            for vals in values_list:
                rows.append((table_bytes[0], vals))
                table_bytes[0] += 8 * max(1, len(vals))
            return start

        self._plans = plans
        launch_rows = {}               # program_id -> [row offsets per plan]
        for pid, ps in plans.items():
            launch_rows[pid] = [add_rows([self._arg_values(p, pid)]) for p in ps]
        sched = self._build_schedules(proc, plans, regions, add_rows)
        self.table_off = off
        off += _align(max(table_bytes[0], 8))
        self.ctx.reserve(max(off, ALIGN))
        if fetch_bytes[0]:
            for fset in (0, 1):
                self.ctx.fetch_reserve(fset, fetch_bytes[0])
        for bid, content in self._contents.items():
            assert content.dtype == np.float32, "Content is not np.float32"
            self.ctx.write(self.buffers[bid], np.ascontiguousarray(content))
        table = np.zeros(max(table_bytes[0], 8) // 8, dtype=np.uint64)
        base = self.ctx.base
        for boff, vals in rows:
            for i, (is_ptr, v) in enumerate(vals):
                table[boff // 8 + i] = (base + v) if is_ptr else v
        self.ctx.write(self.table_off, table)
        funcs = self._compile({**plans, "narrow": list(self._narrow_plans.values())})
        self.stats["unique_sources"] += len(funcs)
        tbase = self.ctx.base + self.table_off
        for pid, ps in plans.items():
            launches = [self.ctx.launcher(funcs[p.name], p.grid, p.block, p.shared, [tbase + r])
                        for p, r in zip(ps, launch_rows[pid])]
            self.kernels[pid] = ps
            self.stats["kernels"] += len(ps)
            self.funcs[pid] = launches[0] if len(launches) == 1 else (lambda ls=launches: [f() for f in ls])
        self.ctx.lanes_reserve(self.lanes, self._events)
        launchers = {}

        def bind(items):
            out = []
            for item in items:
                if item[0] in ("cmd", "record", "wait"):
                    out.append(item)
                    continue
                _, plan, row, count, lane, g, deps = item
                if row not in launchers:
                    grid = (plan.grid[0], plan.grid[1], count)
                    launchers[row] = self.ctx.launcher_on(funcs[plan.name], grid, plan.block,
                                                          plan.shared, [tbase + row])
                # (kind, launcher, lane, index in its stretch, groups of the
                # stretch it follows, whether the launch makes a graph node)
                out.append(("launch", launchers[row], lane, g, deps, min(plan.grid[:2]) > 0 and count > 0))
            return out
        for pid_proc, (items, lane_items) in sched.items():
            self._schedules[pid_proc] = bind(items)
            self._lane_schedules[pid_proc] = bind(lane_items)
        self._pending = []

    @staticmethod
    def _check_temps(cmd):
        if not hasattr(cmd, "nodes"):
            return
        init = getattr(cmd, "init_node", None)
        if isinstance(cmd, DPElwFuse):
            kind, cols = "dp", init.shape[1]
        elif isinstance(cmd, ReduceElwFuse):
            kind, cols = "red", 1
        else:
            kind, cols = "global", 1
        bad = codegen.temp_access_violations(codegen.statements(cmd.nodes), kind, cols)
        if bad:
            si, tid, acc = bad[0]
            raise ValueError(f"fused command {type(cmd).__name__} (program {cmd.program_id}) reads temp "
                             f"{tid} through the access {acc}; the reference reads that element's own value")

    def _feeder_dst(self, cmd):
        if self.feeder_offset_zero:
            return self.buffers[cmd.kres.id]
        return self._addr(cmd.kres.id, cmd.kres.offset, getattr(cmd.kres, "tetris_var", None))

    def _arg_values(self, plan, pid):
        """Argument row of a plan of command ``pid``: ``(True, arena byte
        offset)`` for a pointer (resolved against the arena base once it
        exists), ``(False, v)`` for an integer."""
        vals = []
        for a in plan.args:
            if a[0] == "buf":
                vals.append((True, self.buffers[a[1]] + 4 * a[2]))
            elif a[0] == "var":
                bid, vid, voff, size = a[1]
                vals.append((True, self._addr(bid, voff + a[2], (vid, voff, size))))
            elif a[0] == "scratch":
                vals.append((True, self.scratch_off + 4 * (self._scratch_base[pid] + a[1])))
            else:
                vals.append((False, int(a[1]) & 0xFFFFFFFFFFFFFFFF))
        return vals

    def _build_schedules(self, proc, plans, regions, add_rows):
        """Per Proc: the launch order and grouping of each stretch of kernel
        commands between Feeders, Receivers and loops."""
        out = {}

        def visit(p):
            items = []          # one lane
            lane_items = []     # self.lanes lanes
            stretch = []

            def flush():
                if not stretch:
                    return
                launches = []
                for cmd in stretch:
                    c_reads, c_writes = regions[cmd.program_id]
                    base = self._scratch_base.get(cmd.program_id, 0)
                    for plan in plans[cmd.program_id]:
                        reads = list(c_reads if plan.reads is None else plan.reads)
                        writes = list(c_writes if plan.writes is None else plan.writes)
                        lo, hi = plan.scratch
                        if hi > lo:
                            reads.append(("scratch", base + lo, base + hi))
                            writes.append(("scratch", base + lo, base + hi))
                        launches.append(_Launch(cmd, plan, None, reads, writes))
                key = (lambda L: (L.plan.name, L.plan.grid, L.plan.block, L.plan.shared)) \
                    if self.group_launches else (lambda L: None)
                groups, deps = schedule_dag([(L, L.reads, L.writes) for L in launches], key)
                rows, plans_of = [], []
                for group in groups:
                    members = [launches[i] for i in group]
                    plan = members[0].plan
                    # a group too small to fill the device takes the plans'
                    # dp_quad alternative (same arguments and results layout)
                    narrow = self.narrow_launches and codegen.use_narrow(plan, len(members))
                    if narrow:
                        plan = plan.narrow
                        self._narrow_plans[plan.name] = plan
                    plans_of.append((plan, len(members)))
                    rows.append(add_rows([self._arg_values(m.plan.narrow if narrow else m.plan, m.cmd.program_id)
                                          for m in members]))
                # the launch groups of this stretch and the earlier groups each
                # must follow (kernel name, instances, dependencies)
                self.stretch_graphs.setdefault(p.id, []).append(
                    [(plans_of[g][0].name, plans_of[g][1], deps[g],
                      [r for i in groups[g] for r in launches[i].reads],
                      [w for i in groups[g] for w in launches[i].writes],
                      sum(launches[i].plan.flops for i in groups[g])) for g in range(len(groups))])
                # one lane: the groups in order (the form captured into graphs)
                one = [("launch", plans_of[g][0], rows[g], plans_of[g][1], 0, g, tuple(deps[g]))
                       for g in range(len(groups))]
                items.extend(one)
                if self.lanes == 1:
                    lane_items.extend(one)
                    stretch.clear()
                    return
                # several lanes (uncaptured runs): fork off stream 0, waits
                # only across lanes, join back at the end of the stretch
                lane_of, waits = assign_lanes(deps, self.lanes)
                used = sorted(set(lane_of) - {0})
                if used:
                    fork = self._new_event()
                    lane_items.append(("record", 0, fork))
                    lane_items.extend(("wait", lane, fork) for lane in used)
                recorded = {}
                needed = {d for w in waits for d in w}
                for g in range(len(groups)):
                    for d in waits[g]:
                        lane_items.append(("wait", lane_of[g], recorded[d]))
                    lane_items.append(("launch", plans_of[g][0], rows[g], plans_of[g][1], lane_of[g], g,
                                       tuple(deps[g])))
                    if g in needed:
                        recorded[g] = self._new_event()
                        lane_items.append(("record", lane_of[g], recorded[g]))
                for lane in used:
                    join = self._new_event()
                    lane_items.append(("record", lane, join))
                    lane_items.append(("wait", 0, join))
                stretch.clear()

            for cmd in p.procedure:
                if isinstance(cmd, (AllocEntry, DeallocEntry)):
                    continue
                if isinstance(cmd, (Feeder, Receiver, ForNode)):
                    flush()
                    items.append(("cmd", cmd))
                    lane_items.append(("cmd", cmd))
                    if isinstance(cmd, ForNode):
                        visit(cmd.get_proc())
                    continue
                stretch.append(cmd)
            flush()
            out[p.id] = (items, lane_items)

        visit(proc)
        return out

    def _new_event(self):
        self._events += 1
        return self._events - 1

    def _compile(self, plans):
        """hipRTC-compile every distinct kernel (in parallel) and load it."""
        header = _header()
        sources = {}
        for ps in plans.values():
            for p in ps:
                sources.setdefault(p.name, p.source)
        todo = [src for src in sources.values() if src not in _code_cache]

        def build(src):
            return src, compile_source(header + src)
        if todo:
            with ThreadPoolExecutor(self.jit_threads) as pool:
                for src, code in pool.map(build, todo):
                    with _code_lock:
                        _code_cache[src] = code
        funcs = {}
        for name, src in sources.items():
            mod = self.ctx.load_module(_code_cache[src])
            funcs[name] = self.ctx.function(mod, name)
        return funcs

    # ------------------------------------------------------------------ run pass
    def run(self, cmd):
        if isinstance(cmd, (AllocEntry, DeallocEntry, ForNode)):
            return
        if isinstance(cmd, Feeder):
            if self._capturing:
                # inside a graph: copy this iteration's data from the staging slot
                self.ctx.copy(self._feeder_dst(cmd), self._feeder_slots[cmd.id][self._slot], 4 * prod(cmd.shape))
                self._graph_feeders.append(cmd)
                return
            arr = self._feeder_value(cmd)
            self.ctx.write(self._feeder_dst(cmd), arr)
            return
        if isinstance(cmd, Receiver):
            if self._capturing:
                # inside a graph: snapshot the data into this iteration's slot
                dst = self._recv_slots[cmd.id][0][self._parity]
                for bid, shape, off, var in zip(cmd.ids, cmd.shapes, cmd.offsets, cmd.vars):
                    n = 4 * prod(shape)
                    self.ctx.copy(dst, self._addr(bid, off, var), n)
                    dst += _align(n)
                self._graph_receivers.append(cmd)
                return
            outs = []
            for bid, shape, off, var in zip(cmd.ids, cmd.shapes, cmd.offsets, cmd.vars):
                out = np.empty(shape, dtype=np.float32)
                self.ctx.read(self._addr(bid, off, var), out)
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
        """A loop body replays as a graph unless it holds a loop, or a Feeder
        after a Receiver (its function would run before the Receiver's
        callback of the same iteration)."""
        seen_receiver = False
        for c in proc.procedure:
            if isinstance(c, ForNode):
                return False
            if isinstance(c, Receiver):
                seen_receiver = True
            elif isinstance(c, Feeder) and seen_receiver:
                return False
        return True

    def _all_loops(self, proc):
        out = []
        for c in proc.procedure:
            if isinstance(c, ForNode):
                out.append(c)
                out.extend(self._all_loops(c.get_proc()))
        return out

    def _run_scheduled(self, proc):
        ctx = self.ctx
        items = self._schedules[proc.id] if (self._capturing or self.lanes == 1) \
            else self._lane_schedules[proc.id]
        for item in items:
            kind = item[0]
            if kind == "launch":
                item[1](item[2])
            elif kind == "record":
                ctx.record_on(item[1], item[2])
            elif kind == "wait":
                ctx.wait_on(item[1], item[2])
            elif isinstance(item[1], ForNode):
                self._run_loop(item[1])
            else:
                self.run(item[1])

    def _run_loop(self, cmd, iterations=None):
        inner = cmd.get_proc()
        assert inner is not None, "Inner proc is None!"
        reps = len(cmd.r) if iterations is None else iterations
        if reps <= 0:
            return
        if not (self.use_graphs and self._capturable(inner)):
            for _ in range(reps):
                self._run_scheduled(inner)
            return
        U = self._unroll.get(cmd.id, 1)
        if cmd.id not in self._graphs:
            singles = self._capture(inner, U, 1)
            feeders, receivers = self._graph_feeders, self._graph_receivers
            unrolled = self._capture(inner, U, U) if U > 1 else None
            self._graphs[cmd.id] = (singles, unrolled, feeders, receivers)
            self._launches[cmd.id] = 0
        singles, unrolled, feeders, receivers = self._graphs[cmd.id]
        waiting = []                         # fetched iterations whose callbacks are due
        done = 0
        while done < reps:
            n = U if unrolled is not None and reps - done >= U else 1
            graphs = unrolled if n > 1 else singles
            parity = self._launches[cmd.id] & 1
            if feeders:
                # the inputs of these iterations go up on the transfer stream
                # while the previous launch computes; the graph waits for them
                self.ctx.stage_begin(parity)
                for u in range(n):
                    for f in feeders:
                        self.ctx.stage_write(parity, self._feeder_slots[f.id][parity * U + u], self._feeder_value(f))
                self.ctx.stage_end(parity)
            self.ctx.graph_launch(graphs[parity if len(graphs) > 1 else 0])
            if feeders:
                self.ctx.stage_release(parity)
            if receivers:
                # the snapshots of this iteration come down on the transfer stream
                self.ctx.fetch_begin(parity)
                taken = [self._fetch_receiver(r, parity) for r in receivers]
                self.ctx.fetch_end(parity)
                waiting.append((parity, taken))
                if len(waiting) > self.receiver_lag:
                    self._deliver(*waiting.pop(0))
            self._launches[cmd.id] += 1
            done += n
        for item in waiting:
            self._deliver(*item)

    def _capture(self, inner, unroll, count):
        """Graphs of ``count`` consecutive iterations of a loop body, one per
        staging parity (one only when the body has no Feeder or Receiver);
        iteration u of parity p reads Feeder slot ``p * unroll + u``.  With
        ``graph_dag`` the captured chain is rewired to the schedule's
        dependencies (``_dag_deps``)."""
        graphs = []
        for parity in (0, 1):
            self._capturing, self._parity = True, parity
            self._graph_feeders = []
            self._graph_receivers = []
            self.ctx.graph_begin()
            try:
                for u in range(count):
                    self._slot = parity * unroll + u
                    self._run_scheduled(inner)
            except BaseException:
                self._capturing = False
                self.ctx.graph_end()          # close the capture; the error propagates
                raise
            self._capturing = False
            if self.graph_dag:
                graphs.append(self.ctx.graph_end_dag(self._dag_deps(inner, count)))
            else:
                graphs.append(self.ctx.graph_end())
            if not self._graph_feeders and not self._graph_receivers:
                break                    # one graph serves every launch
        return graphs

    def _dag_deps(self, inner, count):
        """For the nodes a capture of ``count`` iterations of ``inner`` made,
        in capture order: the earlier nodes each must follow.  A launch
        follows the launches of its stretch the schedule says it depends on
        (every pair touching overlapping memory, one writing, stays
        ordered); a launch with none follows everything before its stretch.
        A copy (a Feeder's staging slot, a Receiver's snapshot) follows
        everything before it, and everything after it follows the copy."""
        deps, frontier = [], []
        stretch_base, stretch_nodes = None, []

        def close_stretch():
            nonlocal frontier, stretch_base, stretch_nodes
            if stretch_base is None:
                return
            if stretch_nodes:
                used = {d for n in stretch_nodes for d in deps[n] if d >= stretch_base}
                frontier = [n for n in stretch_nodes if n not in used]
            stretch_base, stretch_nodes = None, []

        node_of = {}
        for _ in range(count):
            for item in self._schedules[inner.id]:
                if item[0] == "launch":
                    _, _, _, g, gdeps, makes_node = item
                    if g == 0:
                        close_stretch()
                        stretch_base, node_of = len(deps), {}
                    if not makes_node:
                        node_of[g] = None
                        continue
                    mine = sorted({node_of[d] for d in gdeps if node_of.get(d) is not None})
                    node_of[g] = len(deps)
                    deps.append(mine if mine else list(frontier))
                    stretch_nodes.append(node_of[g])
                    continue
                close_stretch()
                cmd = item[1]
                if isinstance(cmd, Receiver):
                    copies = sum(1 for shape in cmd.shapes if prod(shape) > 0)
                else:
                    copies = 1 if isinstance(cmd, Feeder) and prod(cmd.shape) > 0 else 0
                for _ in range(copies):
                    deps.append(list(frontier))
                    frontier = [len(deps) - 1]
            close_stretch()
        return _transitive_reduction(deps)

    def _fetch_receiver(self, r, parity):
        src = self._recv_slots[r.id][0][parity]
        parts = []
        for shape in r.shapes:
            n = 4 * prod(shape)
            parts.append((self.ctx.fetch_copy(parity, src, n), shape))
            src += _align(n)
        return r, parts

    def _deliver(self, parity, taken):
        """Receiver callbacks of one fetched iteration, in body order."""
        for r, parts in taken:
            outs = []
            for host_off, shape in parts:
                out = np.empty(shape, dtype=np.float32)
                self.ctx.fetch_take(parity, host_off, out)
                outs.append(out)
            r.func(*outs)

    def _run_proc(self, proc, func, init=False):
        """The reference's command walk (device.py:114-124), used for the init
        pass; the run pass goes through the schedules."""
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
        """Init pass: layout, upload, JIT, schedules.  Anything an earlier
        ``prepare`` of this device built is released first."""
        self._reset_program()
        self._feeder_size = {}

        def note_feeders(c, _):
            if isinstance(c, Feeder):
                self._feeder_size[c.id] = prod(c.shape)
            return c
        proc.walk(note_feeders, step_fused=False, step_proc=True)
        codegen.annotate_spans(proc)
        self._run_proc(proc, self.init, init=True)
        self._finish_init(proc)
        for loop in self.loops(proc):
            items = self._schedules[loop.get_proc().id]
            self.stats["launches_per_iter"] = sum(1 for it in items if it[0] == "launch")
            lane_items = self._lane_schedules[loop.get_proc().id]
            self.stats["lanes_used"] = len({it[2] for it in lane_items if it[0] == "launch"})

    def execute(self, proc):
        self.prepare(proc)
        self._run_scheduled(proc)
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
        """Enqueue one prepared compute command (its own launches, ungrouped)."""
        self.funcs[cmd.program_id]()

    def refresh_tensors(self):
        """Copy every Tensor buffer back into its host array."""
        for bid, content in self._contents.items():
            out = np.empty(content.size, dtype=np.float32)
            self.ctx.read(self.buffers[bid], out)
            content.reshape(-1)[:] = out

    def _destroy_graphs(self):
        """Destroy the loop graphs once nothing queued can still be running
        them (a replay returns without waiting)."""
        if not self._graphs:
            return
        self.ctx.sync()
        for singles, unrolled, _, _ in self._graphs.values():
            for g in singles + (unrolled or []):
                self.ctx.graph_destroy(g)
        self._graphs = {}

    def close(self):
        if getattr(self.ctx, "h", None) is None:
            return
        try:
            self.ctx.sync()
        finally:
            try:
                self._destroy_graphs()
            finally:
                self.ctx.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
