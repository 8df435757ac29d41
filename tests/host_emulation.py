"""Host emulation of a whole ``HIPDevice`` run, for bounds checking on the
CPU: the device plans, lays out its arena, writes its argument tables and
schedules its (grouped) launches against a recording context; every launch
then runs on the host over one arena of the device's size, compiled with
AddressSanitizer, so any global or LDS access outside its allocation is
reported with the kernel that made it.

Only addresses are checked: every kernel's addresses are functions of its
indices alone, so cross-lane exchanges and matrix products return their own
input, barriers do nothing, and the threads of a block run one after
another.  Test infrastructure; nothing in the package imports it."""
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
    """The ``Context`` calls a device makes before and while it runs a Proc
    without loops, recorded instead of executed; transfers are checked
    against the arena."""

    def __init__(self):
        self.size = None
        self.base = FAKE_BASE
        self.writes, self.launches, self.errors = [], [], []

    def _check(self, off, n, what):
        if self.size is None or off < 0 or off + n > self.size:
            self.errors.append((what, off, n, self.size))

    def reserve(self, n):
        self.size = n

    def write(self, off, arr):
        arr = np.ascontiguousarray(arr)
        self._check(off, arr.nbytes, "write")
        self.writes.append((off, arr.tobytes()))

    def read(self, off, out):
        self._check(off, out.nbytes, "read")

    def copy(self, dst, src, n):
        self._check(dst, n, "copy to")
        self._check(src, n, "copy from")

    def launcher(self, func, grid, block, shared, args):
        return lambda *_: self.launches.append((func, tuple(grid), tuple(block), args[0]))
    launcher_on = launcher

    def load_module(self, code):
        return code

    def function(self, mod, name):
        return name

    def fetch_reserve(self, *a): pass
    def lanes_reserve(self, *a): pass
    def sync(self): pass
    def close(self): pass
    def record_on(self, *a): pass
    def wait_on(self, *a): pass


def _host_source(src):
    return re.sub(r"__attribute__\(\(address_space\(\d\)\)\)", "", src)


def check_run(proc, workdir, shrink=None, **device_options):
    """Run ``proc`` (no loops) through a recording HIPDevice, then every
    launch on the host under AddressSanitizer.  ``shrink`` (bytes) cuts the
    host arena short, to show the check catches an access past it.  Returns
    ``(ok, log)``."""
    real = devmod.Context
    devmod.Context = lambda index: RecordingContext()
    try:
        dev = devmod.HIPDevice(use_graphs=False, **device_options)
    finally:
        devmod.Context = real
    sources = {}

    def record_compile(plans):
        for ps in plans.values():
            for p in ps:
                sources[p.name] = p.source
        return {n: n for n in sources}
    dev._compile = record_compile
    dev.execute(proc)
    ctx = dev.ctx
    if ctx.errors:
        return False, f"transfers outside the arena: {ctx.errors}"
    os.makedirs(workdir, exist_ok=True)
    blob = bytearray(ctx.size)
    for off, data in ctx.writes:
        blob[off:off + len(data)] = data
    size = ctx.size - (shrink or 0)
    text = [SHIM, _host_source(open(HEADER_PATH).read())]
    for i, (name, src) in enumerate(sources.items()):
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
    for k, (func, grid, block, row) in enumerate(ctx.launches):
        text.append(f'  fprintf(stderr, "launch {k} {func}\\n"); adhip_launch({func}, '
                    f"(const unsigned long long*)(a + {row - FAKE_BASE}ull), {grid[0]}, {grid[1]}, {grid[2]}, {block[0]});")
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
