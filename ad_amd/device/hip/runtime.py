"""ctypes binding of libadhip.so (include/adhip.h).

The library is built in-tree (``python -m ad_amd.build`` or
``__graft_entry__.build()``) next to this file.  There is no fallback: if
the library or a GPU is missing, creating a context raises.
"""
import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libadhip.so")
HEADER_PATH = os.path.join(os.path.dirname(os.path.dirname(_HERE)), "csrc", "adhip_kernels.h")

_lib = None
_lock = threading.Lock()

EXPORTS = [
    "adhip_create", "adhip_destroy", "adhip_last_error", "adhip_device_info", "adhip_arena_reserve",
    "adhip_write", "adhip_stage_begin", "adhip_stage_write", "adhip_stage_end", "adhip_stage_release",
    "adhip_fetch_reserve", "adhip_fetch_begin", "adhip_fetch_copy", "adhip_fetch_end", "adhip_fetch_take",
    "adhip_read", "adhip_copy", "adhip_compile", "adhip_free", "adhip_module_load",
    "adhip_module_function", "adhip_launch", "adhip_graph_begin", "adhip_graph_end",
    "adhip_graph_launch", "adhip_graph_destroy", "adhip_sync", "adhip_event_record",
    "adhip_event_elapsed", "adhip_lanes_reserve", "adhip_launch_on", "adhip_record_on", "adhip_wait_on",
    "adhip_reduce_cols", "adhip_reduce_cols_noalloc", "adhip_graph_end_dag",
]


class HipError(RuntimeError):
    pass


def load_library(path=LIB_PATH):
    """Load libadhip.so and declare every exported signature."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise HipError(f"{path} is not built; run __graft_entry__.build() first")
        lib = ctypes.CDLL(path)
        c = ctypes
        vp, sz, u64, i32, u32 = c.c_void_p, c.c_size_t, c.c_uint64, c.c_int, c.c_uint32
        sigs = {
            "adhip_create": (i32, [i32, c.POINTER(vp)]),
            "adhip_destroy": (None, [vp]),
            "adhip_last_error": (c.c_char_p, [vp]),
            "adhip_device_info": (i32, [vp, c.POINTER(i32), c.c_char_p, sz]),
            "adhip_arena_reserve": (i32, [vp, sz, c.POINTER(u64)]),
            "adhip_write": (i32, [vp, u64, vp, sz]),
            "adhip_stage_begin": (i32, [vp, i32]),
            "adhip_stage_write": (i32, [vp, i32, u64, vp, sz]),
            "adhip_stage_end": (i32, [vp, i32]),
            "adhip_stage_release": (i32, [vp, i32]),
            "adhip_fetch_reserve": (i32, [vp, i32, sz]),
            "adhip_fetch_begin": (i32, [vp, i32]),
            "adhip_fetch_copy": (i32, [vp, i32, u64, sz, ctypes.POINTER(ctypes.c_size_t)]),
            "adhip_fetch_end": (i32, [vp, i32]),
            "adhip_fetch_take": (i32, [vp, i32, sz, vp, sz]),
            "adhip_read": (i32, [vp, u64, vp, sz]),
            "adhip_copy": (i32, [vp, u64, u64, sz]),
            "adhip_compile": (i32, [c.c_char_p, c.c_char_p, c.POINTER(vp), c.POINTER(sz), c.c_char_p, sz]),
            "adhip_free": (None, [vp]),
            "adhip_module_load": (i32, [vp, vp, sz, c.POINTER(vp)]),
            "adhip_module_function": (i32, [vp, c.c_char_p, c.POINTER(vp)]),
            "adhip_launch": (i32, [vp, vp, c.POINTER(u32), c.POINTER(u32), u32, c.POINTER(u64), sz]),
            "adhip_graph_begin": (i32, [vp]),
            "adhip_graph_end": (i32, [vp, c.POINTER(vp)]),
            "adhip_graph_launch": (i32, [vp, vp]),
            "adhip_graph_end_dag": (i32, [vp, i32, c.POINTER(i32), c.POINTER(i32), c.POINTER(vp)]),
            "adhip_graph_destroy": (None, [vp]),
            "adhip_sync": (i32, [vp]),
            "adhip_event_record": (i32, [vp, i32]),
            "adhip_event_elapsed": (i32, [vp, i32, i32, c.POINTER(c.c_float)]),
            "adhip_lanes_reserve": (i32, [vp, i32, i32]),
            "adhip_launch_on": (i32, [vp, i32, vp, c.POINTER(u32), c.POINTER(u32), u32, c.POINTER(u64), sz]),
            "adhip_record_on": (i32, [vp, i32, i32]),
            "adhip_wait_on": (i32, [vp, i32, i32]),
            "adhip_reduce_cols": (i32, [vp, u64, u64, u32, u32, i32]),
            "adhip_reduce_cols_noalloc": (i32, [vp, u64, u64, u32, u32, i32]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def compile_options():
    """hipRTC options: gfx950, no FP contraction (statements round one at a
    time, as the reference's OpenCL statements do), packed-FP32 ops off."""
    return ("--offload-arch=gfx950 -O3 -std=c++17 -ffp-contract=off "
            "-Xclang -target-feature -Xclang -packed-fp32-ops")


def compile_source(src: str, options: str = None):
    """hipRTC-compile ``src``; returns the code object bytes.  Thread-safe."""
    lib = load_library()
    code = ctypes.c_void_p()
    size = ctypes.c_size_t()
    log = ctypes.create_string_buffer(1 << 16)
    rc = lib.adhip_compile(src.encode(), (options or compile_options()).encode(),
                           ctypes.byref(code), ctypes.byref(size), log, len(log))
    if rc != 0:
        msg = lib.adhip_last_error(None).decode(errors="replace")
        raise HipError(f"{msg}\n{log.value.decode(errors='replace')}\n--- source ---\n{src}")
    try:
        return ctypes.string_at(code, size.value)
    finally:
        lib.adhip_free(code)


class Context:
    """One device context: stream, arena, staging, modules, graphs."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        h = ctypes.c_void_p()
        rc = self.lib.adhip_create(int(device), ctypes.byref(h))
        if rc != 0:
            raise HipError(f"adhip_create({device}) failed ({rc}): "
                           f"{self.lib.adhip_last_error(None).decode(errors='replace')}")
        self.h = h
        self.base = 0
        self.arena_bytes = 0
        self._images = []        # code objects stay alive while modules are loaded

    def check(self, rc, what):
        if rc != 0:
            raise HipError(f"{what} failed ({rc}): {self.lib.adhip_last_error(self.h).decode(errors='replace')}")

    def info(self):
        n = ctypes.c_int()
        name = ctypes.create_string_buffer(256)
        self.check(self.lib.adhip_device_info(self.h, ctypes.byref(n), name, 256), "adhip_device_info")
        return n.value, name.value.decode(errors="replace")

    def reserve(self, nbytes: int) -> int:
        base = ctypes.c_uint64()
        self.check(self.lib.adhip_arena_reserve(self.h, nbytes, ctypes.byref(base)), "adhip_arena_reserve")
        self.base = base.value
        self.arena_bytes = nbytes
        return self.base

    def write(self, byte_off: int, arr):
        self.check(self.lib.adhip_write(self.h, byte_off, arr.ctypes.data, arr.nbytes), "adhip_write")

    def stage_begin(self, tag: int):
        self.check(self.lib.adhip_stage_begin(self.h, tag), "adhip_stage_begin")

    def stage_write(self, tag: int, byte_off: int, arr):
        self.check(self.lib.adhip_stage_write(self.h, tag, byte_off, arr.ctypes.data, arr.nbytes),
                   "adhip_stage_write")

    def stage_end(self, tag: int):
        self.check(self.lib.adhip_stage_end(self.h, tag), "adhip_stage_end")

    def stage_release(self, tag: int):
        self.check(self.lib.adhip_stage_release(self.h, tag), "adhip_stage_release")

    def fetch_reserve(self, fset: int, nbytes: int):
        self.check(self.lib.adhip_fetch_reserve(self.h, fset, nbytes), "adhip_fetch_reserve")

    def fetch_begin(self, fset: int):
        self.check(self.lib.adhip_fetch_begin(self.h, fset), "adhip_fetch_begin")

    def fetch_copy(self, fset: int, byte_off: int, nbytes: int) -> int:
        host_off = ctypes.c_size_t()
        self.check(self.lib.adhip_fetch_copy(self.h, fset, byte_off, nbytes, ctypes.byref(host_off)),
                   "adhip_fetch_copy")
        return host_off.value

    def fetch_end(self, fset: int):
        self.check(self.lib.adhip_fetch_end(self.h, fset), "adhip_fetch_end")

    def fetch_take(self, fset: int, host_off: int, arr):
        self.check(self.lib.adhip_fetch_take(self.h, fset, host_off, arr.ctypes.data, arr.nbytes),
                   "adhip_fetch_take")

    def read(self, byte_off: int, arr):
        self.check(self.lib.adhip_read(self.h, byte_off, arr.ctypes.data, arr.nbytes), "adhip_read")

    def copy(self, dst_off: int, src_off: int, nbytes: int):
        self.check(self.lib.adhip_copy(self.h, dst_off, src_off, nbytes), "adhip_copy")

    def load_module(self, code: bytes):
        mod = ctypes.c_void_p()
        buf = ctypes.create_string_buffer(code, len(code))
        self._images.append(buf)
        self.check(self.lib.adhip_module_load(self.h, buf, len(code), ctypes.byref(mod)), "adhip_module_load")
        return mod

    def function(self, mod, name: str):
        fn = ctypes.c_void_p()
        rc = self.lib.adhip_module_function(mod, name.encode(), ctypes.byref(fn))
        if rc != 0:
            raise HipError(f"kernel {name}: {self.lib.adhip_last_error(None).decode(errors='replace')}")
        return fn

    def launcher(self, fn, grid, block, shared, args):
        """A zero-argument callable launching ``fn`` with fixed arguments."""
        g = (ctypes.c_uint32 * 3)(*grid)
        b = (ctypes.c_uint32 * 3)(*block)
        a = (ctypes.c_uint64 * max(1, len(args)))(*[int(v) & 0xFFFFFFFFFFFFFFFF for v in args])
        n = len(args)
        launch = self.lib.adhip_launch
        h = self.h
        check = self.check

        def go():
            rc = launch(h, fn, g, b, shared, a, n)
            if rc != 0:
                check(rc, "adhip_launch")
        return go

    def lanes_reserve(self, streams: int, events: int):
        self.check(self.lib.adhip_lanes_reserve(self.h, streams, events), "adhip_lanes_reserve")

    def launcher_on(self, fn, grid, block, shared, args):
        """A callable ``go(stream)`` launching ``fn`` on a lane with fixed
        arguments."""
        g = (ctypes.c_uint32 * 3)(*grid)
        b = (ctypes.c_uint32 * 3)(*block)
        a = (ctypes.c_uint64 * max(1, len(args)))(*[int(v) & 0xFFFFFFFFFFFFFFFF for v in args])
        n = len(args)
        launch = self.lib.adhip_launch_on
        h = self.h
        check = self.check

        def go(stream=0):
            rc = launch(h, stream, fn, g, b, shared, a, n)
            if rc != 0:
                check(rc, "adhip_launch_on")
        return go

    def record_on(self, stream: int, event: int):
        self.check(self.lib.adhip_record_on(self.h, stream, event), "adhip_record_on")

    def wait_on(self, stream: int, event: int):
        self.check(self.lib.adhip_wait_on(self.h, stream, event), "adhip_wait_on")

    def graph_begin(self):
        self.check(self.lib.adhip_graph_begin(self.h), "adhip_graph_begin")

    def graph_end(self):
        g = ctypes.c_void_p()
        self.check(self.lib.adhip_graph_end(self.h, ctypes.byref(g)), "adhip_graph_end")
        return g

    def graph_end_dag(self, deps):
        """End the capture; ``deps[i]`` lists the earlier captured nodes node
        ``i`` must follow (the chain's own edges are dropped)."""
        offs = [0]
        flat = []
        for d in deps:
            flat.extend(int(x) for x in d)
            offs.append(len(flat))
        o = (ctypes.c_int32 * len(offs))(*offs)
        f = (ctypes.c_int32 * max(1, len(flat)))(*flat)
        g = ctypes.c_void_p()
        self.check(self.lib.adhip_graph_end_dag(self.h, len(deps), o, f, ctypes.byref(g)), "adhip_graph_end_dag")
        return g

    def graph_launch(self, g):
        self.check(self.lib.adhip_graph_launch(self.h, g), "adhip_graph_launch")

    def graph_destroy(self, g):
        self.lib.adhip_graph_destroy(g)

    def sync(self):
        self.check(self.lib.adhip_sync(self.h), "adhip_sync")

    def event(self, slot: int):
        self.check(self.lib.adhip_event_record(self.h, slot), "adhip_event_record")

    def elapsed_ms(self, a: int, b: int) -> float:
        ms = ctypes.c_float()
        self.check(self.lib.adhip_event_elapsed(self.h, a, b, ctypes.byref(ms)), "adhip_event_elapsed")
        return ms.value

    def reduce_cols(self, x_off: int, out_off: int, rows: int, cols: int, op: int = 0):
        """Column SUM (op 0) or MAX (op 1) of the [rows, cols] matrix at arena
        byte offset ``x_off`` into ``cols`` floats at ``out_off``."""
        self.check(self.lib.adhip_reduce_cols(self.h, self.base + x_off, self.base + out_off, rows, cols, op),
                   "adhip_reduce_cols")

    def reduce_cols_noalloc(self, x_off: int, out_off: int, rows: int, cols: int, op: int = 0):
        """``reduce_cols`` with its scratch in the library's static device
        array: allocates nothing (usable under graph capture)."""
        self.check(self.lib.adhip_reduce_cols_noalloc(self.h, self.base + x_off, self.base + out_off, rows, cols,
                                                      op), "adhip_reduce_cols_noalloc")

    def close(self):
        if self.h:
            self.lib.adhip_destroy(self.h)
            self.h = None
