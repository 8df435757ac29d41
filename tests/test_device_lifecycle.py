"""Device lifecycle on the CPU, against a context that records calls instead
of making them: a second program on one device starts from a clean slate
(no graph, allocation or slot of the first survives), and ``close`` waits
for queued work before it destroys graphs and the context."""
import numpy as np

import ad_amd as ad
from ad_amd import workloads
from ad_amd.device.hip import device as devmod


class GraphRecordingContext:
    """The calls ``HIPDevice`` makes, recorded; graphs are numbered handles."""

    def __init__(self):
        self.h = 1
        self.base = 1 << 40
        self.log = []
        self.size = None
        self.live_graphs = set()
        self._next = 0

    def reserve(self, n):
        self.size = n
        self.log.append(("reserve", n))

    def write(self, off, arr): self.log.append(("write", off))
    def read(self, off, out): self.log.append(("read", off))
    def copy(self, dst, src, n): self.log.append(("copy", dst, src, n))
    def load_module(self, code): return code
    def function(self, mod, name): return name

    def launcher(self, func, grid, block, shared, args):
        return lambda *_: self.log.append(("launch", func))
    launcher_on = launcher

    def lanes_reserve(self, *a): pass
    def fetch_reserve(self, *a): pass
    def fetch_begin(self, s): self.log.append(("fetch_begin", s))
    def fetch_copy(self, s, off, n): return 0
    def fetch_end(self, s): self.log.append(("fetch_end", s))
    def fetch_take(self, s, off, out): out[...] = 0
    def stage_begin(self, t): pass
    def stage_write(self, t, off, arr): pass
    def stage_end(self, t): pass
    def stage_release(self, t): pass
    def record_on(self, *a): pass
    def wait_on(self, *a): pass

    def graph_begin(self):
        self.log.append(("graph_begin",))

    def graph_end(self):
        self._next += 1
        self.live_graphs.add(self._next)
        self.log.append(("graph_end", self._next))
        return self._next

    def graph_end_dag(self, deps):
        self.last_dag = [list(d) for d in deps]
        return self.graph_end()

    def graph_launch(self, g):
        assert g in self.live_graphs, f"launch of destroyed graph {g}"
        self.log.append(("graph_launch", g))

    def graph_destroy(self, g):
        assert g in self.live_graphs, f"graph {g} destroyed twice"
        self.live_graphs.discard(g)
        self.log.append(("graph_destroy", g))

    def sync(self): self.log.append(("sync",))

    def close(self):
        self.log.append(("close",))
        self.h = None


def _device(**kw):
    real = devmod.Context
    devmod.Context = lambda index: GraphRecordingContext()
    try:
        dev = devmod.HIPDevice(**kw)
    finally:
        devmod.Context = real
    dev._compile = lambda plans: {p.name: p.name for ps in plans.values() for p in ps}
    return dev


def _layernorm():
    workloads.layernorm_train(rows=64, cols=128, steps=3, receive=True)


def _mlp():
    workloads.mlp(steps=5, din=16, dh=24, dout=8, receive=True)


def test_second_program_starts_clean():
    dev = _device()
    ctx = dev.ctx
    _mlp()
    ad.execute(device=dev)
    first_graphs = set(ctx.live_graphs)
    first_buffers = set(dev.buffers)
    assert first_graphs, "the loop body should have been captured"
    ad.reset()
    _layernorm()
    proc = ad.compile_proc()
    mark = len(ctx.log)
    dev.execute(proc)
    later = ctx.log[mark:]
    # every graph of the first program is destroyed after a sync and before
    # the second program lays out its arena
    kinds = [e[0] for e in later]
    first_reserve = kinds.index("reserve")
    destroyed = {e[1] for e in later[:first_reserve] if e[0] == "graph_destroy"}
    assert destroyed == first_graphs
    assert "sync" in kinds[:kinds.index("graph_destroy")]
    # nothing replayed belongs to the first program
    launched = {e[1] for e in later if e[0] == "graph_launch"}
    assert launched and not (launched & first_graphs)
    # the layout holds exactly the second program's buffers, sized as a
    # fresh device sizes them
    fresh = _device()
    ad.reset()
    _layernorm()
    fresh.execute(ad.compile_proc())
    assert sorted(dev.buffers.values()) == sorted(fresh.buffers.values())
    assert ctx.size == fresh.ctx.size
    assert not (set(dev.buffers) & first_buffers - set(fresh.buffers))


def test_close_syncs_before_destroying():
    dev = _device()
    ctx = dev.ctx
    _mlp()
    ad.execute(device=dev)
    mark = len(ctx.log)
    dev.close()
    tail = [e[0] for e in ctx.log[mark:]]
    assert tail[0] == "sync"
    assert tail[-1] == "close"
    assert "graph_destroy" in tail and tail.index("sync") < tail.index("graph_destroy")
    assert not ctx.live_graphs
    n = len(ctx.log)
    dev.close()        # a second close does nothing
    assert len(ctx.log) == n


def test_replay_then_close_waits():
    """``replay`` returns without waiting; ``close`` right after it must
    still sync first."""
    dev = _device()
    ctx = dev.ctx
    workloads.mlp(steps=2, din=16, dh=24, dout=8, receive=False)
    proc = ad.compile_proc()
    dev.prepare(proc)
    loop = dev.loops(proc)[0]
    dev.replay(loop, 3)
    assert ctx.log[-1][0] == "graph_launch"
    dev.close()
    tail = [e[0] for e in ctx.log]
    last_launch = max(i for i, k in enumerate(tail) if k == "graph_launch")
    first_destroy = tail.index("graph_destroy")
    assert "sync" in tail[last_launch:first_destroy]
    assert np.all([k != "graph_launch" for k in tail[first_destroy:]])
