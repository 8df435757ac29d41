"""CPU restatement of the OpenCL backend -- test infrastructure only.

Each function names the reference code it follows.  See ``oracle/__init__``.
"""
import ctypes
import hashlib
import math
import os
import subprocess
import tempfile
from math import ceil, prod

import numpy as np

from ad_amd.alloc import AllocEntry, DeallocEntry
from ad_amd.expr import (Add, BitwiseAnd, Constant, Div, Global, LessThan, Minus, MoreThan,
                         Mult, Remainder, ShiftLeft, ShiftRight, Val, X, Y)
from ad_amd.fusion import DPElwFuse, ElwFuse, FuseBase, ReduceElwFuse
from ad_amd.graph import (BinaryNode, BinaryOp, ContigiousNode, DotProdNode, Feeder, ForNode,
                          Receiver, ReduceNode, ReduceOp, UnaryNode, UnaryOp)
from ad_amd.kernalize import KConcat, KConstant, KMatrix
from ad_amd.node import Node

_HERE = os.path.dirname(os.path.abspath(__file__))
_CACHE = os.environ.get("AD_ORACLE_CACHE", os.path.join(tempfile.gettempdir(), "ad_oracle_cache"))

_OPS = {Add: "+", Minus: "-", Mult: "*", Div: "/", Remainder: "%", ShiftRight: ">>",
        ShiftLeft: "<<", BitwiseAnd: "&", MoreThan: ">", LessThan: "<"}


# ---------------------------------------------------------------- lowering (karg.py)
def lower_expr(e) -> str:
    """autodiff/device/opencl/karg.py:8-43"""
    if isinstance(e, Constant):
        return str(e.val)
    if isinstance(e, Global):
        return "_global_id"
    if isinstance(e, X):
        return "_x"
    if isinstance(e, Y):
        return "_y"
    if isinstance(e, Val):
        return lower_expr(e.v)
    op = _OPS.get(type(e))
    if op is None:
        raise Exception(f"Invalid expr at lower: {e}")
    return f"({lower_expr(e.a)} {op} {lower_expr(e.b)})"


def lower_karg(k) -> str:
    """autodiff/device/opencl/karg.py:45-54: temps ignore their access."""
    if isinstance(k, KMatrix):
        return f"temp_{k.id}" if k.is_temp else f"buf_{k.id}[{lower_expr(k.access)}]"
    if isinstance(k, KConcat):
        return f"({lower_expr(k.condition)} ? ({lower_karg(k.karg_two)}) : ({lower_karg(k.karg_one)}))"
    if isinstance(k, KConstant):
        return str(k.constant)
    raise TypeError(k)


def lower_args(cmd):
    """Buffer ids a kernel binds (karg.py:56-85)."""
    args = []
    if isinstance(cmd, Node):
        args = cmd.kargs_child_ids(filter_temp=True)
        ids = cmd.kres.get_ids(filter_temp=True)
        if len(ids) == 1 and ids[0] not in args:
            args.append(ids[0])
    else:
        for n in cmd.nodes:
            if isinstance(n, Node):
                args.extend(n.kargs_child_ids(filter_temp=True))
                ids = n.kres.get_ids(filter_temp=True)
                if len(ids) == 1:
                    args.append(ids[0])
        args = list(set(args))
    return args


def _statements(nodes, init_kind):
    """Ordered statements of a command: ``(kind, node)`` with kind one of
    ``bin``/``un``/``tmp``/``init`` (the DotProd/Reduce result line)."""
    out = []
    for n in nodes:
        if isinstance(n, BinaryNode):
            out.append(("bin", n))
        elif isinstance(n, UnaryNode):
            out.append(("un", n))
        elif isinstance(n, ContigiousNode):
            out.append(("copy", n))
        elif isinstance(n, AllocEntry):
            assert n.is_temp, "not temp alloc entry in fused op"
            out.append(("tmp", n))
        elif isinstance(n, (DotProdNode, ReduceNode)):
            out.append(("init", n))
    return out


def _rhs(kind, n, init_value):
    """Right-hand side of one statement (binary.py:8-16, unary.py:8-33,
    contigious.py:9-10, dp_elw_fuse.py:21-22, reduce_elw_fuse.py:22-23)."""
    if kind == "bin":
        op = "+" if n.op == BinaryOp.ADD else "*"
        return f"{lower_karg(n.kargs[0])} {op} {lower_karg(n.kargs[1])}"
    if kind == "copy":
        return lower_karg(n.kargs[0])
    if kind == "init":
        return init_value
    a = lower_karg(n.kargs[0])
    op = n.op
    if op == UnaryOp.EXP2:
        return f"exp2({a})"
    if op == UnaryOp.LOG2:
        return f"log2({a})"
    if op == UnaryOp.SIN:
        return f"sin({a})"
    if op == UnaryOp.RECIP:
        return f"1.0/{a}"
    if op == UnaryOp.SQRT:
        return f"sqrt(fabs({a}))"
    cmp = {UnaryOp.EQUAL: "==", UnaryOp.MORE_ZERO: ">", UnaryOp.LESS_ZERO: "<",
           UnaryOp.MORE_OR_EQ_ZERO: ">=", UnaryOp.LESS_OR_EQ_ZERO: "<="}[op]
    return f"({a} {cmp} 0.0f) ? 1.0 : 0.0"


def _bind(args) -> str:
    return "".join(f"    float* buf_{a} = B[{i}];\n" for i, a in enumerate(args))


def _lockstep_body(stmts, n, index_setup, init_value, init_compute):
    """The kernel as an ideal SIMD machine runs it: statement by statement
    over the whole index space; within a statement every element reads
    before any element writes (values staged in ``_st``).  Temps are arrays
    indexed by element.  ``init_compute`` fills ``_init[e]`` first."""
    lines = [f"    const long long _n = {n}LL;",
             "    std::vector<float> _st_v(_n > 0 ? _n : 1); float* _st = _st_v.data();"]
    temps = [s[1].id for s in stmts if s[0] == "tmp"]
    for t in temps:
        lines.append(f"    std::vector<float> _tv_{t}(_n > 0 ? _n : 1, 0.0f); float* _tp_{t} = _tv_{t}.data();")
    if init_compute:
        lines.append("    std::vector<float> _init_v(_n > 0 ? _n : 1); float* _init = _init_v.data();")
        lines.append(init_compute)
    tdefs = "".join(f"float& temp_{t} = _tp_{t}[_e]; " for t in temps)
    for kind, node in stmts:
        if kind == "tmp":
            continue
        rhs = _rhs(kind, node, init_value)
        dst = lower_karg(node.kres)
        lines.append(f"""    #pragma omp parallel for schedule(static)
    for (long long _e = 0; _e < _n; ++_e) {{ {index_setup} {tdefs}(void)0; _st[_e] = {rhs}; }}
    #pragma omp parallel for schedule(static)
    for (long long _e = 0; _e < _n; ++_e) {{ {index_setup} {tdefs}(void)0; {dst} = _st[_e]; }}""")
    return "\n".join(lines)


def _fused_body(stmts, init_value):
    out = []
    for kind, node in stmts:
        if kind == "tmp":
            out.append(f"float temp_{node.id} = 0.0;")
        else:
            out.append(f"{lower_karg(node.kres)} = {_rhs(kind, node, init_value)};")
    return "\n            ".join(out)


def _elementwise_kernel(name, args, stmts, n) -> str:
    """1-D NDRange kernels (binary.py:18-33, unary.py:35-52,
    contigious.py:12-29, elw_fuse.py:27-44).  ``<name>`` runs lockstep
    semantics; ``<name>_wi`` runs one work-item at a time (the timed CPU
    baseline; identical when no element reads what another element writes)."""
    setup = "const size_t _global_id = (size_t)_e; (void)_global_id;"
    return f"""
extern "C" void {name}(float** B) {{
{_bind(args)}{_lockstep_body(stmts, n, setup, None, None)}
}}
extern "C" void {name}_wi(float** B) {{
{_bind(args)}    #pragma omp parallel for schedule(static)
    for (long long _gid = 0; _gid < {n}LL; ++_gid) {{
        const size_t _global_id = (size_t)_gid; (void)_global_id;
        {_fused_body(stmts, None)}
    }}
}}
"""


def _dotprod_kernel(name, args, dp, stmts, fused) -> str:
    """kernels/dotprod.py:7-43 and dp_elw_fuse.py:26-65.  Every output element
    accumulates ``A(_ty,k)*B(k,_tx)`` for k = 0..K-1 in order in fp32; the
    loop nest walks columns innermost (as a vectorising OpenCL CPU runtime
    would) without changing any element's accumulation order."""
    M, N = dp.shape
    K = dp.children_shapes[0][1]
    a_expr = lower_karg(dp.kargs[0])
    b_expr = lower_karg(dp.kargs[1])
    gid = f"int _global_id = _ty * {N} + _tx; (void)_global_id;" if fused else \
        "const size_t _global_id = _tx; (void)_global_id;"
    compute = f"""    #pragma omp parallel for collapse(2) schedule(static)
    for (int _ty = 0; _ty < {M}; ++_ty) {{
      for (int _tb = 0; _tb < {N}; _tb += 256) {{
        const int _te = (_tb + 256 < {N}) ? _tb + 256 : {N};
        float _acc[256];
        for (int _tx = _tb; _tx < _te; ++_tx) _acc[_tx - _tb] = 0.0f;
        for (int _k = 0; _k < {K}; ++_k) {{
            float _elementA;
            {{ int _x = _ty; int _y = _k; (void)_x; (void)_y; _elementA = {a_expr}; }}
            for (int _tx = _tb; _tx < _te; ++_tx) {{
                int _x = _k; int _y = _tx; (void)_x; (void)_y;
                float _elementB = {b_expr};
                _acc[_tx - _tb] += _elementA * _elementB;
            }}
        }}
        for (int _tx = _tb; _tx < _te; ++_tx) _init[(long long)_ty * {N} + _tx] = _acc[_tx - _tb];
      }}
    }}"""
    setup = (f"const int _ty = (int)(_e / {N}); const int _tx = (int)(_e % {N}); "
             f"int _x = _ty; int _y = _tx; (void)_x; (void)_y; {gid}")
    wi_body = _fused_body(stmts, "_value")
    return f"""
extern "C" void {name}(float** B) {{
{_bind(args)}{_lockstep_body(stmts, M * N, setup, "_init[_e]", compute)}
}}
extern "C" void {name}_wi(float** B) {{
{_bind(args)}    const long long _n = {M * N}LL;
    std::vector<float> _init_v(_n); float* _init = _init_v.data();
{compute}
    #pragma omp parallel for schedule(static)
    for (long long _e = 0; _e < _n; ++_e) {{
        {setup}
        float _value = _init[_e];
        {wi_body}
    }}
}}
"""


def _reduce_kernel(name, args, red, stmts, fused, exact=False) -> str:
    """kernels/reduce.py:8-66 and reduce_elw_fuse.py:12-80: one work-group of
    ``L = ceil(R/2)*2`` items per row; ``scratch[y] = y < R ? A(x,y) : 0``;
    tree ``off = L/2, L/4, ... > 0``; item 0 writes and runs the epilogue.
    ``exact`` (not the reference: the fix of its tree) combines all R
    elements in order, SUM from 0 and MAX from -inf."""
    V, R = red.children_shapes[0]
    L = ceil(R / 2) * 2
    a_expr = lower_karg(red.kargs[0])
    if red.op == ReduceOp.SUM:
        step = "scratch[_y] += scratch[_y + _offset];"
    else:
        step = "scratch[_y] = std::fmax(scratch[_y], scratch[_y + _offset]);"
    if exact:
        ident, comb = ("0.0f", "_a += v;") if red.op == ReduceOp.SUM else ("-INFINITY", "_a = std::fmax(_a, v);")
        compute = f"""    #pragma omp parallel for schedule(static)
    for (int _x = 0; _x < {V}; ++_x) {{
        float _a = {ident};
        for (int _y = 0; _y < {R}; ++_y) {{ const float v = {a_expr}; {comb} }}
        _init[_x] = _a;
    }}"""
    else:
        compute = None
    compute = compute or f"""    #pragma omp parallel
    {{
    std::vector<float> scratch_v({L});
    float* scratch = scratch_v.data();
    #pragma omp for schedule(static)
    for (int _x = 0; _x < {V}; ++_x) {{
        for (int _y = 0; _y < {L}; ++_y)
            scratch[_y] = (_y < {R}) ? {a_expr} : 0.0f;
        for (int _offset = {L} / 2; _offset > 0; _offset >>= 1)
            for (int _y = 0; _y < _offset; ++_y) {{ {step} }}
        _init[_x] = scratch[0];
    }}
    }}"""
    gid = "int _global_id = _x; (void)_global_id;" if fused else ""
    setup = f"const int _x = (int)_e; const int _y = 0; (void)_x; (void)_y; {gid}"
    wi_body = _fused_body(stmts, "_init[_e]")
    return f"""
extern "C" void {name}(float** B) {{
{_bind(args)}{_lockstep_body(stmts, V, setup, "_init[_e]", compute)}
}}
extern "C" void {name}_wi(float** B) {{
{_bind(args)}    const long long _n = {V}LL;
    std::vector<float> _init_v(_n); float* _init = _init_v.data();
{compute}
    #pragma omp parallel for schedule(static)
    for (long long _e = 0; _e < _n; ++_e) {{
        {setup}
        {wi_body}
    }}
}}
"""


_PRELUDE = """
#include <cmath>
#include <cstddef>
#include <vector>
using std::exp2; using std::log2; using std::sin; using std::sqrt; using std::fabs;
"""


def kernel_source(cmd, name, exact_reduce=False):
    """C++ text for one command (the restated ``init_<kind>``)."""
    args = lower_args(cmd)
    if isinstance(cmd, (BinaryNode, UnaryNode, ContigiousNode)):
        return args, _elementwise_kernel(name, args, _statements([cmd], None), prod(cmd.shape))
    if isinstance(cmd, ElwFuse):
        return args, _elementwise_kernel(name, args, _statements(cmd.nodes, None),
                                         prod(cmd.init_node.shape))
    if isinstance(cmd, DotProdNode):
        return args, _dotprod_kernel(name, args, cmd, _statements([cmd], None), fused=False)
    if isinstance(cmd, DPElwFuse):
        return args, _dotprod_kernel(name, args, cmd.init_node, _statements(cmd.nodes, None), fused=True)
    if isinstance(cmd, ReduceNode):
        return args, _reduce_kernel(name, args, cmd, _statements([cmd], None), fused=False, exact=exact_reduce)
    if isinstance(cmd, ReduceElwFuse):
        return args, _reduce_kernel(name, args, cmd.init_node, _statements(cmd.nodes, None), fused=True,
                                    exact=exact_reduce)
    raise TypeError(f"Encountered unexpected cmd: {cmd}")


def work_item_only(source: str, name: str) -> str:
    """The ``<name>_wi`` function of a command's source (each generator
    emits the lockstep function ``<name>`` first, then ``<name>_wi``)."""
    i = source.index(f'extern "C" void {name}_wi(')
    return source[i:]


def compile_cpp_parallel(sources, jobs: int) -> str:
    """Compile the functions ``sources`` (texts without the prelude) in
    ``jobs`` translation units at once and link them into one cached shared
    object; returns its path.  For the work-item kernels of whole training
    steps (thousands of commands), which one g++ run takes minutes over."""
    os.makedirs(_CACHE, exist_ok=True)
    flags = ["-O3", "-march=native", "-ffp-contract=off", "-fno-math-errno", "-fPIC", "-w", "-fopenmp"]
    key = hashlib.sha256(("".join(sources) + " ".join(flags)).encode()).hexdigest()[:24]
    so = os.path.join(_CACHE, f"p_{key}.so")
    if os.path.exists(so):
        return so
    jobs = max(1, min(jobs, len(sources)))
    parts, sizes = [[] for _ in range(jobs)], [0] * jobs
    for src in sorted(sources, key=len, reverse=True):
        j = sizes.index(min(sizes))
        parts[j].append(src)
        sizes[j] += len(src)
    procs, objs = [], []
    for j, part in enumerate(parts):
        path = os.path.join(_CACHE, f"p_{key}_{j}.cpp")
        with open(path, "w") as fh:
            fh.write(_PRELUDE + "".join(part))
        objs.append(path + f".o{os.getpid()}")
        procs.append(subprocess.Popen(["g++", *flags, "-c", path, "-o", objs[-1]]))
    bad = [p.wait() for p in procs]
    if any(bad):
        raise RuntimeError(f"g++ failed on {sum(1 for b in bad if b)} of {jobs} parts")
    tmp = so + f".tmp{os.getpid()}"
    subprocess.run(["g++", "-shared", "-fopenmp", *objs, "-o", tmp], check=True)
    os.replace(tmp, so)
    for o in objs:
        os.remove(o)
    return so


def compile_cpp(source: str, threads_flag=True) -> str:
    """Compile ``source`` into a cached shared object and return its path."""
    os.makedirs(_CACHE, exist_ok=True)
    flags = ["-O3", "-march=native", "-ffp-contract=off", "-fno-math-errno", "-shared", "-fPIC", "-w"]
    if threads_flag:
        flags.append("-fopenmp")
    key = hashlib.sha256((source + " ".join(flags)).encode()).hexdigest()[:24]
    so = os.path.join(_CACHE, f"k_{key}.so")
    if not os.path.exists(so):
        src = os.path.join(_CACHE, f"k_{key}.cpp")
        with open(src, "w") as fh:
            fh.write(source)
        tmp = so + f".tmp{os.getpid()}"
        subprocess.run(["g++", *flags, src, "-o", tmp], check=True)
        os.replace(tmp, so)
    return so


class OracleDevice:
    """The reference's device protocol (device/opencl/device.py:16-146) on
    the CPU.  Buffers are numpy float32 arrays; a Tensor's buffer IS its
    ``arr`` (the reference uses CL_MEM_USE_HOST_PTR on a CPU device)."""

    def __init__(self, feeder_offset_zero=False, threads=None, lockstep=True, exact_reduce=False, jobs=None):
        self.jobs = jobs
        self.kernels = {}
        self.exact_reduce = exact_reduce
        self.funcs = {}
        self.buffers = {}
        self.buffers_size = {}
        self.feeder_offset_zero = feeder_offset_zero
        self.lockstep = lockstep
        self._pending = []
        self._lib = None
        if threads is not None:
            os.environ["OMP_NUM_THREADS"] = str(threads)

    # -- init pass
    def init(self, cmd):
        if isinstance(cmd, Feeder):
            cmd.kres.calc_offset()
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
                if cmd.content is not None:
                    assert cmd.content.dtype == np.float32, "Content is not np.float32"
                    self.buffers[cmd.id] = cmd.content.reshape(-1)
                else:
                    self.buffers[cmd.id] = np.zeros(cmd.size, dtype=np.float32)
                self.buffers_size[cmd.id] = cmd.size
            return
        if isinstance(cmd, (DeallocEntry, ForNode)):
            return
        if isinstance(cmd, (Node, FuseBase)):
            name = f"k_{cmd.program_id}"
            args, src = kernel_source(cmd, name, self.exact_reduce)
            self._pending.append((cmd.program_id, name, args, src))
            return
        raise AssertionError(f"Encountered unexpected cmd: {cmd}")

    def _finish_init(self):
        if not self._pending:
            return
        if self.lockstep:
            self._lib = ctypes.CDLL(compile_cpp(_PRELUDE + "".join(p[3] for p in self._pending)))
        else:
            # work-item kernels only, compiled in parallel (the timed CPU
            # baseline of whole training steps)
            jobs = self.jobs or len(os.sched_getaffinity(0))
            self._lib = ctypes.CDLL(compile_cpp_parallel(
                [work_item_only(p[3], p[1]) for p in self._pending], jobs))
        for pid, name, args, _ in self._pending:
            fn = getattr(self._lib, name if self.lockstep else name + "_wi")
            fn.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
            fn.restype = None
            ptrs = (ctypes.c_void_p * max(1, len(args)))(*[self.buffers[a].ctypes.data for a in args])
            self.kernels[pid] = (fn, ptrs)
            self.funcs[pid] = (lambda f=fn, p=ptrs: f(p))
        self._pending = []

    # -- run pass
    def run(self, cmd):
        if isinstance(cmd, (AllocEntry, DeallocEntry, ForNode)):
            return
        if isinstance(cmd, Feeder):
            arr = cmd.func()
            assert isinstance(arr, np.ndarray) and list(arr.shape) == list(cmd.shape), "Invalid function"
            off = 0 if self.feeder_offset_zero else cmd.kres.offset
            flat = np.ascontiguousarray(arr, dtype=np.float32).reshape(-1)
            self.buffers[cmd.kres.id][off:off + flat.size] = flat
            return
        if isinstance(cmd, Receiver):
            outs = []
            for bid, shape, off in zip(cmd.ids, cmd.shapes, cmd.offsets):
                n = prod(shape)
                outs.append(self.buffers[bid][off:off + n].copy().reshape(shape))
            cmd.func(*outs)
            return
        self.funcs[cmd.program_id]()

    def _run_proc(self, proc, func, init=False):
        for cmd in proc.procedure:
            if isinstance(cmd, ForNode):
                inner = cmd.get_proc()
                assert inner is not None, "Inner proc is None!"
                if init:
                    self._run_proc(inner, func, init)
                else:
                    for _ in cmd.r:
                        self._run_proc(inner, func, init)
            else:
                func(cmd)

    def execute(self, proc):
        self._run_proc(proc, self.init, init=True)
        self._finish_init()
        self._run_proc(proc, self.run, init=False)
