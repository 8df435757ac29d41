"""Host emulation of a whole ``HIPDevice`` run, for bounds checking on the
CPU: the device plans, lays out its arena, writes its argument tables and
schedules its (grouped) launches against a recording context; every launch
then runs on the host over one arena of the device's size, compiled with
AddressSanitizer, so any global or LDS access outside its allocation is
reported with the kernel that made it.

Only addresses are checked: every kernel's addresses are functions of its
indices alone, so cross-lane exchanges and matrix products return their own
input, barriers do nothing, and the threads of a block run one after
another.  Loop bodies replay as recorded graphs (with their Feeder staging
and Receiver snapshot copies), and the argument-table rows each launch
reads are checked against the table the device wrote.  Test
infrastructure; nothing in the package imports it."""
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

    def read(self, off, out):
        self._check(off, out.nbytes, "read")
        self.reads.append((off, out.nbytes))

    def copy(self, dst, src, n):
        self._check(dst, n, "copy to")
        self._check(src, n, "copy from")
        if max(dst, src) < min(dst, src) + n:
            self.errors.append(("overlapping copy", dst, src, n))
        self._sink().append(("copy", dst, src, n))

    def launcher(self, func, grid, block, shared, args):
        return lambda *_: self._sink().append(("launch", func, tuple(grid), tuple(block), shared, args[0]))
    launcher_on = launcher

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
        return self.graph_end()

    def graph_launch(self, g):
        self.launches.extend(self._graphs[g])

    def graph_destroy(self, g):
        self._graphs.pop(g, None)

    def stage_begin(self, tag):
        if self._staging.get(tag):
            self.errors.append(("staging set opened twice", tag, 0, self.size))
        self._staging[tag] = True

    def stage_write(self, tag, off, arr):
        if not self._staging.get(tag):
            self.errors.append(("staged write to a closed set", tag, off, self.size))
        self._check(off, np.asarray(arr).nbytes, "staged write")

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
    def record_on(self, *a): pass
    def wait_on(self, *a): pass

    def close(self):
        self.h = None


_NARGS_RE = re.compile(r"blockIdx\.z \* (\d+)u")


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


def check_run(proc, workdir, shrink=None, device=None, dump=None, **device_options):
    """Run ``proc`` through a recording HIPDevice (loops replayed as
    recorded graphs), then check transfers and argument tables
    (``check_tables``) and run every launch on the host under
    AddressSanitizer.  ``device`` reuses a recording device (a second
    program on one device); ``shrink`` (bytes) cuts the host arena short, to
    show the check catches an access past it; ``dump`` (a path) receives the
    arena after the last launch.  Returns ``(ok, log)``."""
    dev = device or recording_device(**device_options)
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
    os.makedirs(workdir, exist_ok=True)
    blob = bytearray(ctx.size)
    for off, data in ctx.writes:
        blob[off:off + len(data)] = data
    size = ctx.size - (shrink or 0)
    used = {op[1] for op in launches if op[0] == "launch"}
    text = [SHIM, _host_source(open(HEADER_PATH).read())]
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
    # one call per distinct launch: replays of a graph repeat the same
    # addresses, so each (kernel, grid, row) is checked once
    seen = set()
    for k, op in enumerate(launches):
        if op[0] == "copy":
            _, dst, src, nb = op
            text.append(f"  memmove(a + {dst}ull, a + {src}ull, {nb}ull);")
            continue
        _, func, grid, block, shared, row = op
        if (func, grid, row) in seen:
            continue
        seen.add((func, grid, row))
        text.append(f'  fprintf(stderr, "launch {k} {func}\\n"); adhip_launch({func}, '
                    f"(const unsigned long long*)(a + {row - FAKE_BASE}ull), {grid[0]}, {grid[1]}, {grid[2]}, {block[0]});")
    if dump:
        text.append(f'  {{ FILE* out = fopen("{dump}", "wb"); if (!out || fwrite(a, 1, n, out) != n) return 4; fclose(out); }}')
    text.append('  fprintf(stderr, "all launches in bounds\\n");\n  return 0;\n}')
    code = "\n".join(text)
    exe = os.path.join(workdir, "run_" + hashlib.sha1(code.encode()).hexdigest()[:12])
    with open(exe + ".cpp", "w") as fh:
        fh.write(code)
    r = subprocess.run([CLANG, "-std=c++17", "-O1", "-g", "-fsanitize=address", "-fno-omit-frame-pointer",
                        "-Wno-everything", exe + ".cpp", "-o", exe], capture_output=True, text=True)
    if r.returncode != 0:
        return False, "host build failed:\n" + r.stderr[-3000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=600, env=env)
    return r.returncode == 0 and "all launches in bounds" in r.stderr, r.stderr[-4000:]


def host_arena(proc, workdir, **device_options):
    """Run ``proc``'s launches on the host (``check_run``) and return the
    recording device and the arena bytes after the last launch (None if a
    launch leaves the arena)."""
    dump = os.path.join(workdir, "arena_after.bin")
    dev = recording_device(**device_options)
    ok, log = check_run(proc, workdir, device=dev, dump=dump)
    return dev, (np.fromfile(dump, dtype=np.uint8) if ok else None)


def host_values(proc, workdir, **device_options):
    """Values of every host read (Receiver) of a Proc computed by running its
    launches on the host, in read order; None if a launch leaves the arena.
    Only kernels whose lanes do not exchange data (elementwise passes,
    operand gathers, copies) compute real values here: cross-lane and MFMA
    builtins return their inputs and a block's threads run one after
    another.  Each distinct launch runs once, so a Proc with loops gives
    the values of one pass through each body."""
    dev, arena = host_arena(proc, workdir, **device_options)
    if arena is None:
        return None
    return [arena[off:off + nb].view(np.float32).copy() for off, nb in dev.ctx.reads]
