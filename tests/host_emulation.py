"""Host emulation of a whole ``HIPDevice`` run, for bounds checking on the
CPU: the device plans, lays out its arena, writes its argument tables and
schedules its (grouped) launches against a recording context; every launch
then runs on the host over one arena of the device's size, compiled with
AddressSanitizer, so any global or LDS access outside its allocation is
reported with the kernel that made it.

By default only addresses are checked: every kernel's addresses are
functions of its indices alone, so cross-lane exchanges and matrix products
return their own input, barriers do nothing, and the threads of a block run
one after another (elementwise passes still compute their real values,
``host_values``).  With ``lockstep`` the threads of a block run together with
real barriers, shuffles and fp32 and bf16 MFMAs (``LOCKSTEP_SHIM``), so DotProd
kernels compute their real values too.  Loop bodies replay as recorded
graphs (with their Feeder staging and Receiver snapshot copies), and the
argument-table rows each launch reads are checked against the table the
device wrote.  A bounds check runs each distinct launch once; a value run
(``host_values``) replays the device's whole sequence in call order --
every iteration, the Feeder data staged for it, every host read and
Receiver fetch -- so whole training loops can be compared with the oracle.
Test infrastructure; nothing in the package imports it."""
import hashlib
import os
import re
import subprocess

import numpy as np

from ad_amd.device.hip import device as devmod
from ad_amd.device.hip.runtime import HEADER_PATH

CLANG = "/opt/rocm/llvm/bin/clang++"
FAKE_BASE = 1 << 46            # arena base the recorded tables are written against

SHIM = r"""
#include <cstdint>
#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <cmath>
#include <cstring>
#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __shared__ static
struct adhip_dim3 { unsigned x, y, z; };
static adhip_dim3 threadIdx, blockIdx, blockDim, gridDim;
struct float4 { float x, y, z, w; };
static inline float4 make_float4(float a, float b, float c, float d) { float4 r; r.x = a; r.y = b; r.z = c; r.w = d; return r; }
struct uint4 { unsigned x, y, z, w; };
#define __syncthreads() ((void)0)
template <class T> static inline T __shfl_xor(T v, int, int = 64) { return v; }
#define __builtin_amdgcn_fence(...) ((void)0)
#define __builtin_amdgcn_iglp_opt(...) ((void)0)
#define __builtin_amdgcn_s_setprio(...) ((void)0)
#define __builtin_amdgcn_sched_barrier(...) ((void)0)
#define __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, ...) (c)
#define __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, ...) (c)
using std::exp2; using std::log2; using std::sin; using std::sqrt; using std::fabs;
template <class F> static void adhip_launch(F f, const unsigned long long* t, unsigned gx, unsigned gy,
                                            unsigned gz, unsigned bx) {
  gridDim = {gx, gy, gz}; blockDim = {bx, 1, 1};
  for (unsigned z = 0; z < gz; ++z) for (unsigned y = 0; y < gy; ++y) for (unsigned x = 0; x < gx; ++x) {
    blockIdx = {x, y, z};
    for (unsigned t2 = 0; t2 < bx; ++t2) { threadIdx = {t2, 0, 0}; f(t); }
  }
}
"""


# The same kernels with real values: every thread of a block runs as a fiber
# of its own; __syncthreads is a block barrier; a wavefront-scope fence is a
# wave barrier; a shuffle or an MFMA exchanges the wave's values between two
# wave barriers.  v_mfma_f32_32x32x2f32 takes A[i][k] from lane i + 32k and
# B[k][j] from lane j + 32k and returns, in lane l's element r, row
# 8*(r/4) + 4*(l/32) + r%4 of column l%32 of C + A*B;
# v_mfma_f32_32x32x16_bf16 takes eight k per lane (k = 8*(l/32) + v) and
# returns the same layout.  A barrier that no thread can pass (a divergent
# barrier) aborts the run.  Blocks run one after another.
LOCKSTEP_SHIM = r"""
#include <cstdint>
#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <cmath>
#include <cstring>
#include <vector>
#include <ucontext.h>
#include <sys/mman.h>
#include <sanitizer/common_interface_defs.h>
#include <sanitizer/asan_interface.h>
#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __shared__ static
struct adhip_dim3 { unsigned x, y, z; };
static adhip_dim3 threadIdx, blockIdx, blockDim, gridDim;
struct float4 { float x, y, z, w; };
static inline float4 make_float4(float a, float b, float c, float d) { float4 r; r.x = a; r.y = b; r.z = c; r.w = d; return r; }
struct uint4 { unsigned x, y, z, w; };
typedef float adhip_v16 __attribute__((ext_vector_type(16)));
// Every thread of a block is a fiber (ucontext) of the one OS thread: a
// fiber runs until it waits at a barrier or ends, then the next fiber of the
// block that may go on resumes, in ascending thread order (descending with
// ADHIP_DESCENDING: data shared between threads without a barrier between
// the write and the read then gives other results).  The stack switches are
// announced to AddressSanitizer.  A barrier no fiber can pass aborts the run.
struct adhip_barrier;
struct adhip_fiber {
  ucontext_t ctx;
  char* stack;
  void* fake;
  unsigned tid;
  bool done;
  adhip_barrier* bar;
  unsigned gen;
};
static const size_t ADHIP_STACK = 256 * 1024;
static ucontext_t adhip_sched;
static const void* adhip_main_bottom = nullptr;
static size_t adhip_main_size = 0;
static std::vector<adhip_fiber> adhip_fibers;
static adhip_fiber* adhip_cur = nullptr;
static void (*adhip_kernel)(const unsigned long long*) = nullptr;
static const unsigned long long* adhip_table = nullptr;
static void adhip_yield() {
  adhip_fiber* f = adhip_cur;
  __sanitizer_start_switch_fiber(&f->fake, adhip_main_bottom, adhip_main_size);
  swapcontext(&f->ctx, &adhip_sched);
  __sanitizer_finish_switch_fiber(f->fake, nullptr, nullptr);
}
static void adhip_fiber_main() {
  __sanitizer_finish_switch_fiber(nullptr, &adhip_main_bottom, &adhip_main_size);
  adhip_kernel(adhip_table);
  adhip_cur->done = true;
  __sanitizer_start_switch_fiber(nullptr, adhip_main_bottom, adhip_main_size);
}   // returns to adhip_sched (uc_link)
struct adhip_barrier {
  unsigned n = 0, count = 0, gen = 0;
  void wait() {
    if (++count == n) { count = 0; ++gen; return; }
    adhip_cur->bar = this;
    adhip_cur->gen = gen;
    adhip_yield();
  }
};
static void adhip_run_block(unsigned bx) {
  while (adhip_fibers.size() < bx) {
    adhip_fiber f{};
    void* st = mmap(nullptr, ADHIP_STACK, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
    if (st == MAP_FAILED) { fprintf(stderr, "fiber stack\n"); abort(); }
    f.stack = (char*)st;
    f.tid = adhip_fibers.size();
    adhip_fibers.push_back(f);
  }
  for (unsigned i = 0; i < bx; ++i) {
    adhip_fiber& f = adhip_fibers[i];
    f.done = false; f.bar = nullptr; f.fake = nullptr;
    __asan_unpoison_memory_region(f.stack, ADHIP_STACK);
    getcontext(&f.ctx);
    f.ctx.uc_stack.ss_sp = f.stack;
    f.ctx.uc_stack.ss_size = ADHIP_STACK;
    f.ctx.uc_link = &adhip_sched;
    makecontext(&f.ctx, adhip_fiber_main, 0);
  }
#ifdef ADHIP_DESCENDING
  unsigned left = bx, i = bx - 1, stuck = 0;
#else
  unsigned left = bx, i = 0, stuck = 0;
#endif
  while (left) {
    adhip_fiber& f = adhip_fibers[i];
    if (!f.done && (!f.bar || f.bar->gen != f.gen)) {
      f.bar = nullptr;
      adhip_cur = &f;
      threadIdx = {f.tid, 0, 0};
      void* fake = nullptr;
      __sanitizer_start_switch_fiber(&fake, f.stack, ADHIP_STACK);
      swapcontext(&adhip_sched, &f.ctx);
      __sanitizer_finish_switch_fiber(fake, nullptr, nullptr);
      if (f.done) --left;
      stuck = 0;
    } else if (++stuck > bx) {
      fprintf(stderr, "barrier deadlock\n");
      abort();
    }
#ifdef ADHIP_DESCENDING
    i = i == 0 ? bx - 1 : i - 1;
#else
    i = i + 1 == bx ? 0 : i + 1;
#endif
  }
}
static adhip_barrier adhip_block_bar;
static adhip_barrier adhip_wave_bar[16];
static float adhip_wave_a[16][64], adhip_wave_b[16][64];
static inline unsigned adhip_lane() { return threadIdx.x & 63u; }
static inline unsigned adhip_wave() { return threadIdx.x >> 6; }
#define __syncthreads() adhip_block_bar.wait()
template <class T> static inline T __shfl_xor(T v, int off, int width = 64) {
  const unsigned l = adhip_lane(), w = adhip_wave();
  float* buf = adhip_wave_a[w];
  T out;
  memcpy(&buf[l], &v, sizeof(float));
  adhip_wave_bar[w].wait();
  const unsigned src = (l & ~(unsigned)(width - 1)) | ((l ^ (unsigned)off) & (unsigned)(width - 1));
  memcpy(&out, &buf[src], sizeof(float));
  adhip_wave_bar[w].wait();
  return out;
}
static inline adhip_v16 adhip_mfma_32x32x2(float a, float b, adhip_v16 c) {
  const unsigned l = adhip_lane(), w = adhip_wave();
  adhip_wave_a[w][l] = a; adhip_wave_b[w][l] = b;
  adhip_wave_bar[w].wait();
  adhip_v16 d = c;
  const unsigned col = l & 31u;
  for (int r = 0; r < 16; ++r) {
    const unsigned row = 8u * (r >> 2) + 4u * (l >> 5) + (r & 3);
    d[r] = c[r] + (adhip_wave_a[w][row] * adhip_wave_b[w][col] + adhip_wave_a[w][row + 32] * adhip_wave_b[w][col + 32]);
  }
  adhip_wave_bar[w].wait();
  return d;
}
// v_mfma_f32_32x32x16_bf16: lane l holds A[l%32][8*(l/32) + v] and
// B[k][l%32] with k = 8*(l/32) + v in element v of its operands; the
// results layout is the fp32 MFMA's
static float adhip_wave_a8[16][64][8], adhip_wave_b8[16][64][8];
template <class V> static inline adhip_v16 adhip_mfma_32x32x16_bf16(V a, V b, adhip_v16 c) {
  const unsigned l = adhip_lane(), w = adhip_wave();
  for (int v = 0; v < 8; ++v) { adhip_wave_a8[w][l][v] = (float)a[v]; adhip_wave_b8[w][l][v] = (float)b[v]; }
  adhip_wave_bar[w].wait();
  adhip_v16 d = c;
  const unsigned col = l & 31u;
  for (int r = 0; r < 16; ++r) {
    const unsigned row = 8u * (r >> 2) + 4u * (l >> 5) + (r & 3);
    float sum = 0.f;
    for (int h = 0; h < 2; ++h)
      for (int v = 0; v < 8; ++v) sum += adhip_wave_a8[w][row + 32 * h][v] * adhip_wave_b8[w][col + 32 * h][v];
    d[r] = c[r] + sum;
  }
  adhip_wave_bar[w].wait();
  return d;
}
// a wave executes in lockstep on the GPU: the kernels order LDS traffic
// between the lanes of a wave with wavefront-scope fences alone
#define __builtin_amdgcn_fence(...) adhip_wave_bar[adhip_wave()].wait()
#define __builtin_amdgcn_iglp_opt(...) ((void)0)
#define __builtin_amdgcn_s_setprio(...) ((void)0)
#define __builtin_amdgcn_sched_barrier(...) ((void)0)
#define __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, ...) adhip_mfma_32x32x2((a), (b), (c))
#define __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, ...) adhip_mfma_32x32x16_bf16((a), (b), (c))
using std::exp2; using std::log2; using std::sin; using std::sqrt; using std::fabs;
template <class F> static void adhip_launch(F f, const unsigned long long* t, unsigned gx, unsigned gy,
                                            unsigned gz, unsigned bx) {
  gridDim = {gx, gy, gz}; blockDim = {bx, 1, 1};
  adhip_block_bar.n = bx;
  for (unsigned w = 0; w < 16; ++w) adhip_wave_bar[w].n = (bx - 64 * w) < 64 ? (bx > 64 * w ? bx - 64 * w : 0) : 64;
  adhip_kernel = f;
  adhip_table = t;
  for (unsigned z = 0; z < gz; ++z) for (unsigned y = 0; y < gy; ++y) for (unsigned x = 0; x < gx; ++x) {
#ifdef ADHIP_DESCENDING
    blockIdx = {gx - 1 - x, gy - 1 - y, gz - 1 - z};
#else
    blockIdx = {x, y, z};
#endif
    adhip_run_block(bx);
  }
}
"""


class RecordingContext:
    """The ``Context`` calls a device makes while it prepares and runs a
    Proc, recorded instead of executed.  Transfers (writes, reads, in-arena
    copies, staged Feeder copies, Receiver fetches) are checked against the
    arena; launches are recorded with their grid and argument-table row.
    Loop bodies are captured into recorded graphs, and every replay of a
    graph records its launches again, so a loop of n iterations yields n
    copies of its body's launches, in order."""

    def __init__(self):
        self.size = None
        self.base = FAKE_BASE
        self.h = 1
        self.writes, self.launches, self.errors = [], [], []
        self.reads = []                # (arena offset, bytes) of every host read, in order
        self._capture = None           # launches of the graph being captured
        self.dag_late = False          # replay dependency graphs latest-node first
        self._late = {}                # graph -> its nodes in that order
        self._graphs = {}
        self._staging = {}             # tag -> open
        self._fetch = {}               # set -> (capacity, used, open, pending)

    def _check(self, off, n, what):
        if self.size is None or off < 0 or n < 0 or off + n > self.size:
            self.errors.append((what, off, n, self.size))

    def _sink(self):
        return self.launches if self._capture is None else self._capture

    def reserve(self, n):
        self.size = n

    def write(self, off, arr):
        arr = np.ascontiguousarray(arr)
        self._check(off, arr.nbytes, "write")
        if self._capture is not None:
            self.errors.append(("host write during capture", off, arr.nbytes, self.size))
        self.writes.append((off, arr.tobytes()))
        self.launches.append(("write", off, arr.tobytes()))

    def read(self, off, out):
        self._check(off, out.nbytes, "read")
        self.reads.append((off, out.nbytes))
        self.launches.append(("read", off, out.nbytes))

    def copy(self, dst, src, n):
        self._check(dst, n, "copy to")
        self._check(src, n, "copy from")
        if max(dst, src) < min(dst, src) + n:
            self.errors.append(("overlapping copy", dst, src, n))
        self._sink().append(("copy", dst, src, n))

    def launcher(self, func, grid, block, shared, args):
        return lambda *_: self._sink().append(("launch", func, tuple(grid), tuple(block), shared, args[0]))

    def launcher_on(self, func, grid, block, shared, args):
        """As ``launcher``; a launch on another stream than 0 is preceded by
        a ``("lane", stream)`` mark."""
        def go(stream=0):
            if stream:
                self._sink().append(("lane", stream))
            self._sink().append(("launch", func, tuple(grid), tuple(block), shared, args[0]))
        return go

    def graph_begin(self):
        if self._capture is not None:
            self.errors.append(("nested capture", 0, 0, self.size))
        self._capture = []

    def graph_end(self):
        g = len(self._graphs) + 1
        self._graphs[g] = self._capture
        self._capture = None
        return g

    def graph_end_dag(self, deps):
        """As ``graph_end``; the dependency lists are checked against the
        captured nodes (one per launch with a non-empty grid, one per copy)
        and kept in ``dags``."""
        captured = [op for op in self._capture
                    if op[0] == "copy" and op[3] > 0 or op[0] == "launch" and min(op[2]) > 0]
        if len(deps) != len(captured):
            self.errors.append(("dependency lists do not match the capture", len(deps), len(captured), 0))
        for i, d in enumerate(deps):
            if any(not 0 <= j < i for j in d):
                self.errors.append(("dependency on a later node", i, list(d), 0))
        self.dags = getattr(self, "dags", []) + [[list(d) for d in deps]]
        nodes = [op for op in self._capture if not any(op is c for c in captured)] + \
            _latest_ready_first(captured, deps)
        g = self.graph_end()
        self._late[g] = nodes
        return g

    def graph_launch(self, g):
        self.launches.extend(self._late[g] if self.dag_late and g in self._late else self._graphs[g])

    def graph_destroy(self, g):
        self._graphs.pop(g, None)

    def stage_begin(self, tag):
        if self._staging.get(tag):
            self.errors.append(("staging set opened twice", tag, 0, self.size))
        self._staging[tag] = True

    def stage_write(self, tag, off, arr):
        if not self._staging.get(tag):
            self.errors.append(("staged write to a closed set", tag, off, self.size))
        arr = np.ascontiguousarray(arr, dtype=np.float32)
        self._check(off, arr.nbytes, "staged write")
        self.launches.append(("write", off, arr.tobytes()))

    def stage_end(self, tag):
        self._staging[tag] = False

    def stage_release(self, tag):
        pass

    def fetch_reserve(self, fset, nbytes):
        self._fetch[fset] = [nbytes, 0, False, False]

    def fetch_begin(self, fset):
        f = self._fetch.get(fset)
        if f is None or f[2] or f[3]:
            self.errors.append(("fetch set begun before it was taken", fset, 0, self.size))
            return
        f[1], f[2] = 0, True

    def fetch_copy(self, fset, off, nbytes):
        f = self._fetch[fset]
        self._check(off, nbytes, "fetch from")
        self._sink().append(("read", off, nbytes))
        host = f[1]
        f[1] += (nbytes + 255) // 256 * 256
        if f[1] > f[0]:
            self.errors.append(("fetch set overflow", fset, f[1], f[0]))
        return host

    def fetch_end(self, fset):
        f = self._fetch[fset]
        f[2], f[3] = False, True

    def fetch_take(self, fset, host_off, out):
        f = self._fetch[fset]
        if host_off + out.nbytes > f[1]:
            self.errors.append(("fetch take out of range", fset, host_off, f[1]))
        f[3] = False
        out[...] = 0

    def load_module(self, code):
        return code

    def function(self, mod, name):
        return name

    def lanes_reserve(self, *a): pass
    def sync(self): pass
    def record_on(self, stream, event):
        self._sink().append(("record", stream, event))

    def wait_on(self, stream, event):
        self._sink().append(("wait", stream, event))

    def close(self):
        self.h = None


_NARGS_RE = re.compile(r"blockIdx\.z \* (\d+)u")


def _latest_ready_first(nodes, deps):
    """The nodes of a dependency graph in the order that always runs the
    highest-numbered node whose dependencies have all run."""
    done, order = set(), []
    while len(order) < len(nodes):
        i = max(j for j in range(len(nodes)) if j not in done and all(d in done for d in deps[j]))
        done.add(i)
        order.append(nodes[i])
    return order


def lanes_late_first(ops):
    """The recorded operations in another order the streams allow: at each
    step the highest-numbered stream whose next operation may start runs
    it (a wait may start once the latest earlier record of its event has
    run).  Host transfers (writes, reads) keep their place: everything
    issued before one runs before it.  Launches, copies, records and waits
    of stream 0 keep their order, as do those of each other stream."""
    out, segment = [], []

    def drain():
        seq, queues, last_record = [], {}, {}
        lane = 0
        for op in segment:
            if op[0] == "lane":
                lane = op[1]
                continue
            on = op[1] if op[0] in ("record", "wait") else (lane if op[0] == "launch" else 0)
            lane = 0 if op[0] == "launch" else lane
            dep = last_record.get(op[2]) if op[0] == "wait" else None
            if op[0] == "record":
                last_record[op[2]] = len(seq)
            queues.setdefault(on, []).append(len(seq))
            seq.append((op, dep))
        done, heads = set(), {q: 0 for q in queues}
        while len(done) < len(seq):
            for q in sorted(queues, reverse=True):
                if heads[q] < len(queues[q]):
                    i = queues[q][heads[q]]
                    if seq[i][1] is None or seq[i][1] in done:
                        break
            else:
                raise AssertionError("the streams' waits admit no order")
            heads[q] += 1
            done.add(i)
            out.append(seq[i][0])
        segment.clear()

    for op in ops:
        if op[0] in ("write", "read"):
            drain()
            out.append(op)
        else:
            segment.append(op)
    drain()
    return out


def check_tables(dev, ctx, sources):
    """Every launch's argument rows lie inside the argument table the device
    wrote: rows ``row + z * nargs`` for z < grid.z (the kernel's own stride),
    and every pointer in those rows points into the arena.  No launch asks
    for dynamic LDS: the kernels declare only static LDS."""
    errors = []
    table = [w for w in ctx.writes if w[0] == dev.table_off]
    if not table:
        return ["no argument table written"]
    t_lo, t_hi = dev.table_off, dev.table_off + len(table[-1][1])
    words = np.frombuffer(table[-1][1], dtype=np.uint64)
    for op in ctx.launches:
        if op[0] != "launch":
            continue
        _, func, grid, block, shared, row = op
        m = _NARGS_RE.search(sources[func])
        nargs = int(m.group(1)) if m else None
        off = row - FAKE_BASE
        if nargs is None:
            errors.append((func, "no table stride in source"))
            continue
        if off < t_lo or off + 8 * nargs * grid[2] > t_hi:
            errors.append((func, "rows outside the table", off, nargs, grid))
            continue
        vals = words[(off - t_lo) // 8:(off - t_lo) // 8 + nargs * grid[2]]
        ptrs = vals[vals >= FAKE_BASE]
        if ptrs.size and int(ptrs.max()) > FAKE_BASE + ctx.size:
            errors.append((func, "pointer past the arena", int(ptrs.max()) - FAKE_BASE, ctx.size))
        if shared and "extern __shared__" not in sources[func]:
            errors.append((func, "dynamic LDS requested of a kernel without any", shared))
    return errors


def recording_device(**device_options):
    """A ``HIPDevice`` whose context records (``RecordingContext``) and
    whose compile step only collects the kernel sources
    (``dev.recorded_sources``)."""
    real = devmod.Context
    devmod.Context = lambda index: RecordingContext()
    try:
        dev = devmod.HIPDevice(**device_options)
    finally:
        devmod.Context = real
    dev.recorded_sources = {}

    def record_compile(plans):
        for ps in plans.values():
            for p in ps:
                dev.recorded_sources[p.name] = p.source
        return {n: n for n in dev.recorded_sources}
    dev._compile = record_compile
    return dev


def _host_source(src):
    return re.sub(r"__attribute__\(\(address_space\(\d\)\)\)", "", src)


def check_run(proc, workdir, shrink=None, device=None, dump=None, lockstep=False, full=False,
              descending=False, **device_options):
    """Run ``proc`` through a recording HIPDevice (loops replayed as
    recorded graphs), then check transfers and argument tables
    (``check_tables``) and run every launch on the host under
    AddressSanitizer.  ``device`` reuses a recording device (a second
    program on one device); ``shrink`` (bytes) cuts the host arena short, to
    show the check catches an access past it; ``dump`` (a path) receives the
    arena after the last launch.

    By default each distinct launch runs once (a graph replay repeats the
    same addresses) over an arena holding every host write from the start.
    With ``full`` the run is the device's own, in call order: every replay's
    launches and copies, host writes and staged Feeder data applied when
    they were made, and every host read and Receiver fetch saved when it was
    made (to ``reads.bin`` in ``workdir``, in order).  ``descending`` runs
    the operations of several streams late stream first
    (``lanes_late_first``), the nodes of dependency-graph replays latest
    ready node first, and, with ``lockstep``, a launch's blocks and a
    block's threads in descending order.  Returns ``(ok, log)``."""
    dev = device or recording_device(**device_options)
    dev.ctx.dag_late = descending
    mark = len(dev.ctx.launches)
    dev.ctx.writes = []
    dev.ctx.reads = []
    dev.execute(proc)
    ctx = dev.ctx
    sources = dev.recorded_sources
    if ctx.errors:
        return False, f"transfers outside the arena: {ctx.errors}"
    launches = ctx.launches[mark:]
    saved, ctx.launches = ctx.launches, launches
    try:
        bad = check_tables(dev, ctx, sources)
    finally:
        ctx.launches = saved
    if bad:
        return False, f"argument tables: {bad[:5]}"
    if descending:
        launches = lanes_late_first(launches)
    os.makedirs(workdir, exist_ok=True)
    blob = bytearray(ctx.size)
    for off, data in ctx.writes:
        blob[off:off + len(data)] = data
    size = ctx.size - (shrink or 0)
    used = {op[1] for op in launches if op[0] == "launch"}
    text = [("#define ADHIP_DESCENDING 1\n" if descending else "") + (LOCKSTEP_SHIM if lockstep else SHIM),
            _host_source(open(HEADER_PATH).read())]
    for i, (name, src) in enumerate(sources.items()):
        if name in used:
            text.append(f"namespace k{i} {{\n{_host_source(src)}\n}}\nusing k{i}::{name};")
    digest = hashlib.sha1(bytes(blob) + "".join(sources).encode()).hexdigest()[:12]
    blob_path = os.path.join(workdir, f"arena_{digest}.bin")
    with open(blob_path, "wb") as fh:
        fh.write(bytes(blob[:size]))
    text.append("int main() {")
    text.append(f"  const size_t n = {size}ull; unsigned char* a = (unsigned char*)malloc(n);")
    text.append(f'  FILE* fh = fopen("{blob_path}", "rb"); if (!fh || fread(a, 1, n, fh) != n) return 3; fclose(fh);')
    table_words = max(0, (size - dev.table_off) // 8)
    text.append(f"  unsigned long long* tab = (unsigned long long*)(a + {dev.table_off}ull);")
    text.append(f"  for (size_t i = 0; i < {table_words}ull; ++i)"
                f" if (tab[i] >= {FAKE_BASE}ull) tab[i] = (unsigned long long)(a + (tab[i] - {FAKE_BASE}ull));")
    if full:
        # host data of the writes made after set-up, applied in call order
        # (the argument table keeps its rewritten pointers)
        data = b"".join(op[2] for op in launches if op[0] == "write" and op[1] != dev.table_off)
        data_path = os.path.join(workdir, f"writes_{hashlib.sha1(data).hexdigest()[:12]}.bin")
        with open(data_path, "wb") as fh:
            fh.write(data)
        text.append(f"  unsigned char* wd = (unsigned char*)malloc({len(data)}ull + 1);")
        text.append(f'  fh = fopen("{data_path}", "rb"); if (!fh || fread(wd, 1, {len(data)}ull, fh) != {len(data)}ull) return 5; fclose(fh);')
        text.append(f'  FILE* rd = fopen("{os.path.join(workdir, "reads.bin")}", "wb"); if (!rd) return 6;')
    # without ``full``, one call per distinct launch: replays of a graph
    # repeat the same addresses, so each (kernel, grid, row) is checked once
    seen = set()
    pos = 0
    for k, op in enumerate(launches):
        if op[0] == "copy":
            _, dst, src, nb = op
            text.append(f"  memmove(a + {dst}ull, a + {src}ull, {nb}ull);")
            continue
        if op[0] == "write":
            if full and op[1] != dev.table_off:
                text.append(f"  memcpy(a + {op[1]}ull, wd + {pos}ull, {len(op[2])}ull);")
                pos += len(op[2])
            continue
        if op[0] == "read":
            if full:
                text.append(f"  if (fwrite(a + {op[1]}ull, 1, {op[2]}ull, rd) != {op[2]}ull) return 7;")
            continue
        if op[0] in ("lane", "record", "wait"):
            continue
        _, func, grid, block, shared, row = op
        if not full and (func, grid, row) in seen:
            continue
        seen.add((func, grid, row))
        text.append(f'  fprintf(stderr, "launch {k} {func}\\n"); adhip_launch({func}, '
                    f"(const unsigned long long*)(a + {row - FAKE_BASE}ull), {grid[0]}, {grid[1]}, {grid[2]}, {block[0]});")
    if full:
        text.append("  fclose(rd);")
    if dump:
        text.append(f'  {{ FILE* out = fopen("{dump}", "wb"); if (!out || fwrite(a, 1, n, out) != n) return 4; fclose(out); }}')
    text.append('  fprintf(stderr, "all launches in bounds\\n");\n  return 0;\n}')
    code = "\n".join(text)
    exe = os.path.join(workdir, "run_" + hashlib.sha1(code.encode()).hexdigest()[:12])
    with open(exe + ".cpp", "w") as fh:
        fh.write(code)
    r = subprocess.run([CLANG, "-std=c++17", "-O1", "-g", "-fsanitize=address", "-fno-omit-frame-pointer",
                        "-Wno-everything", *(["-pthread"] if lockstep else []), exe + ".cpp", "-o", exe],
                       capture_output=True, text=True)
    if r.returncode != 0:
        return False, "host build failed:\n" + r.stderr[-3000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=600, env=env)
    return r.returncode == 0 and "all launches in bounds" in r.stderr, r.stderr[-4000:]


def host_arena(proc, workdir, lockstep=False, full=False, descending=False, **device_options):
    """Run ``proc``'s launches on the host (``check_run``) and return the
    recording device and the arena bytes after the last launch (None if a
    launch leaves the arena)."""
    dump = os.path.join(workdir, "arena_after.bin")
    dev = recording_device(**device_options)
    ok, log = check_run(proc, workdir, device=dev, dump=dump, lockstep=lockstep, full=full,
                        descending=descending)
    if not ok:
        print(log[-2000:])
    return dev, (np.fromfile(dump, dtype=np.uint8) if ok else None)


def host_values(proc, workdir, lockstep=False, descending=False, **device_options):
    """Values of every host read of a Proc (top-level Receivers, Receivers
    inside loops once per iteration, the final Tensor read-back) computed
    by running the device's whole run on the host (``check_run`` with
    ``full``), in the order the device made them; None if a launch leaves
    the arena.  Without ``lockstep`` only kernels whose lanes do not
    exchange data (elementwise passes, operand gathers, copies) compute
    real values: cross-lane and MFMA builtins return their inputs and a
    block's threads run one after another."""
    dev, arena = host_arena(proc, workdir, lockstep=lockstep, full=True, descending=descending,
                            **device_options)
    if arena is None:
        return None
    blob = np.fromfile(os.path.join(workdir, "reads.bin"), dtype=np.uint8)
    out, at = [], 0
    for op in dev.ctx.launches:
        if op[0] == "read":
            out.append(blob[at:at + op[2]].view(np.float32).copy())
            at += op[2]
    assert at == blob.size
    return out
