"""Lowering of procedural-IR commands to specialised HIP kernels.

For every command this module produces one or more ``KernelPlan``s: a
canonical HIP source (compiled through hipRTC, deduplicated by text), a
launch geometry and an argument list of arena byte offsets and integers.

Statement semantics follow the reference kernel templates
(autodiff/device/opencl/kernels/*.py): a fused command is an ordered list of
statements ``kres = f(kargs)`` evaluated per element; temps are registers;
constants are double literals (``str(float)``), so ``x * c`` is computed in
double and rounded to float, exactly as the OpenCL source does.

Where a statement writes a location another element of the same command
still reads (the tetris allocator places a value born inside a fused group
over one that dies there), the reference's single kernel races; the result
kept here is the statement-by-statement one.  ``conflict_pairs`` finds those
statement pairs, ``split_phases`` cuts the command into the fewest passes
with no conflict inside a pass (temps carried through scratch), and a
statement that conflicts with itself falls back to one staged kernel per
statement (``lockstep_plans``).  A DotProd or Reduce runs in the first pass
that needs it, with the epilogue in registers or, split over K / rows, as
partial results combined by an elementwise pass (``first_pass_plans``).
"""
import hashlib
import math
import re
from dataclasses import dataclass, field
from math import ceil, prod
from typing import Dict, List, Optional, Tuple

from ...alloc import AllocEntry
from ...expr import (Add, BitwiseAnd, Constant, Div, Global, LessThan, Minus, MoreThan, Mult,
                     Remainder, ShiftLeft, ShiftRight, Val, X, Y)
from ...fusion import DPElwFuse, ElwFuse, ReduceElwFuse
from ...graph import (BinaryNode, BinaryOp, ContigiousNode, DotProdNode, Receiver, ReduceNode, ReduceOp,
                      UnaryNode, UnaryOp)
from ...kernalize import KConcat, KConstant, KMatrix
from ...node import Node
from .analysis import AFF, INV, const_of, interval, split_const, upper_bound, vec_class

BLOCK = 256
_TEMP_RE = re.compile(r"\btemp_\d+\b")
_HEADER = []


def _header_text() -> str:
    """Text of the device template header every kernel is compiled with."""
    if not _HEADER:
        from .runtime import HEADER_PATH
        with open(HEADER_PATH) as fh:
            _HEADER.append(fh.read())
    return _HEADER[0]

_OPS = {Add: "+", Minus: "-", Mult: "*", Div: "/", Remainder: "%", ShiftRight: ">>",
        ShiftLeft: "<<", BitwiseAnd: "&", MoreThan: ">", LessThan: "<"}


# ------------------------------------------------------------------ plans
@dataclass
class KernelPlan:
    source: str                   # full source; the kernel symbol is ``name``
    grid: Tuple[int, int, int]
    block: Tuple[int, int, int]
    args: List[tuple]             # ("buf", buffer_id, float_offset) | ("var", (buffer_id, var_id, var_offset, size), float_offset) | ("scratch", float_offset) | ("int", v)
    shared: int = 0
    family: str = ""              # "elw" | "reduce" | "dotprod" | "copy"
    flops: int = 0                # algorithmic flops (dotprod) for reporting
    bytes: int = 0                # algorithmic bytes for reporting

    name: str = ""                # kernel symbol: adhip_<family>_<hash of the source>
    reads: Optional[list] = None  # ranges read / written, when narrower than the command's
    writes: Optional[list] = None
    scratch: Tuple[int, int] = (0, 0)   # [lo, hi) of the command's scratch floats it touches
    # the same work on the ``dp_quad`` kernel (same arguments, ranges and
    # results layout), taken by launches too small to fill the device
    narrow: Optional["KernelPlan"] = None

    def __post_init__(self):
        # register temps are named after node ids; number them by first use
        # so commands that differ only in ids share one compiled kernel
        names = {}
        self.source = _TEMP_RE.sub(lambda m: names.setdefault(m.group(0), f"t{len(names)}_"), self.source)
        # every template emits the symbol KNAME; give each distinct source its
        # own symbol so profiles tell kernels apart
        tag = {"dotprod": "dp", "reduce": "red", "elw": "elw", "copy": "copy"}.get(self.family, "k")
        self.source = _table_entry(self.source, len(self.args))
        # the symbol hashes the template header too, so a changed template
        # gives new symbols (profiles name the kernel that was measured)
        self.name = f"adhip_{tag}_{hashlib.sha1((_header_text() + self.source).encode()).hexdigest()[:12]}"
        self.source = self.source.replace(KNAME, self.name)

    @property
    def key(self):
        return self.name


_ENTRY_RE = re.compile(r'extern "C" __global__ void __launch_bounds__\(([\d, ]+)\) ' + "adhip_kernel" + r"\(([^)]*)\) \{")


LAZY_ARGS = 24


def _table_entry(src: str, nargs: int) -> str:
    """Turn the generated kernel (the last function of ``src``) into a device
    function plus an entry point whose only parameter is an argument table
    in device memory: row ``blockIdx.z`` holds the 8-byte arguments (pointers
    and integers) of one instance, so one launch can run several independent
    commands that share the kernel."""
    m = _ENTRY_RE.search(src)
    assert m is not None, "generated kernel entry not found"
    bounds, params = m.group(1), m.group(2)
    plist = [q.strip() for q in params.split(",") if q.strip()]
    assert len(plist) == nargs, (plist, nargs)
    end = src.rindex("}")
    body = src[m.end():end]
    casts = []
    for i, q in enumerate(plist):
        ty = q.rsplit(" ", 1)[0]
        if ty.endswith("*"):
            # a pointer read from memory is generic (flat loads, which also
            # count against the LDS wait counter); it points to global
            # memory, and saying so gives global loads and stores
            casts.append(f"({ty})({ty[:-1].strip()} __attribute__((address_space(1)))*)a_[{i}]")
        else:
            casts.append(f"({ty})a_[{i}]")
    if nargs > LAZY_ARGS:
        # many arguments (a concat of many pieces): read each one from the
        # table where it is used, so a wave loads only the pieces its
        # elements take instead of holding (and spilling) all of them
        for i, q in enumerate(plist):
            name = q.rsplit(" ", 1)[1]
            body = re.sub(rf"\b{re.escape(name)}\b", f"({casts[i]})", body)
        return (src[:m.start()] +
                f'extern "C" __global__ void __launch_bounds__({bounds}) {KNAME}('
                f"const unsigned long long* __restrict__ tbl_) {{\n"
                f"  const unsigned long long* a_ = tbl_ + (unsigned long long)blockIdx.z * {nargs}u;\n"
                f"{body}}}\n")
    return (src[:m.start()] +
            f"static __device__ __forceinline__ void {KNAME}_body({params}) {{{body}}}\n"
            f'extern "C" __global__ void __launch_bounds__({bounds}) {KNAME}('
            f"const unsigned long long* __restrict__ tbl_) {{\n"
            f"  const unsigned long long* a_ = tbl_ + (unsigned long long)blockIdx.z * {max(nargs, 1)}u;\n"
            f"  (void)a_;\n  {KNAME}_body({', '.join(casts)});\n}}\n")


# ------------------------------------------------------------------ statements
def statements(nodes):
    """``[(kind, node)]`` with kind ``bin``/``un``/``copy``/``tmp``/``init``."""
    out = []
    for n in nodes:
        if isinstance(n, BinaryNode):
            out.append(("bin", n))
        elif isinstance(n, UnaryNode):
            out.append(("un", n))
        elif isinstance(n, ContigiousNode):
            out.append(("copy", n))
        elif isinstance(n, AllocEntry):
            assert n.is_temp, "non-temp alloc entry inside a fused command"
            out.append(("tmp", n))
        elif isinstance(n, (DotProdNode, ReduceNode)):
            out.append(("init", n))
    return out


def _iter_kmatrix(karg):
    if isinstance(karg, KMatrix):
        yield karg
    elif isinstance(karg, KConcat):
        yield from _iter_kmatrix(karg.karg_one)
        yield from _iter_kmatrix(karg.karg_two)


iter_kmatrix = _iter_kmatrix


# ------------------------------------------------------------------ hazards
class BufferInfo:
    """Per buffer id: total floats.  ``unpacked``: every tetris variable has
    storage of its own (no two variables share memory), instead of its
    packed offset in the tetris region."""

    def __init__(self, unpacked: bool = False):
        self.size: Dict[int, int] = {}
        self.unpacked = unpacked


def access_span(km: KMatrix, domain):
    """Floats ``[lo, hi)`` of its buffer that an access can touch, given
    the index space ``domain`` of the operand's role (Global below
    prod(domain); X, Y below its first and second extent): interval bounds
    of the access expression.  A subtraction that could go below zero is
    bounded below by 0: a concat piece is read only where its condition
    holds, and there its index is a valid one."""
    n = 1
    for d in domain:
        n *= int(d)
    if n <= 0:
        return None
    xmax = int(domain[0]) - 1
    ymax = int(domain[1]) - 1 if len(domain) > 1 else 0
    lo, hi = interval(km.access, n - 1, xmax, ymax)
    return lo, hi + 1


def _note_span(karg, domain):
    for km in _iter_kmatrix(karg):
        if km.is_temp:
            continue
        sp = access_span(km, domain)
        if sp is None:
            continue
        old = getattr(km, "span", None)
        km.span = sp if old is None else (min(old[0], sp[0]), max(old[1], sp[1]))


def annotate_spans(proc):
    """Record on every buffer access of a Proc (``km.span``) the floats it
    can touch, from its access expression and the index space of its role:
    a DotProd's operands range over [M, K] and [K, N] and its result over
    [M, N] (X, Y); a Reduce's operand over [V, R] and its result over [V];
    an elementwise statement, Feeder or Receiver over its shape (Global).

    This is what the reference's tetris pass leaves to go on
    (alloc/tetris_opt.py:159-188 rewrites every access of an arena variable
    to ``expr + offset`` on the shared region without recording which
    variable it was): every float an access touches lies in its span, so
    accesses whose spans do not overlap cannot conflict, and scheduling and
    hazard analysis stay as fine as the accesses themselves.  Spans are
    cleared and recomputed on every call."""
    from ...graph import ForNode
    todo = []

    def walk(p):
        for c in p.procedure:
            if isinstance(c, ForNode):
                walk(c.get_proc())
            elif hasattr(c, "nodes"):
                todo.extend(n for n in c.nodes if isinstance(n, Node))
            elif isinstance(c, Node):
                todo.append(c)
    walk(proc)
    for n in todo:
        for k in list(n.kargs) + ([n.kres] if n.kres is not None and not n.kres.is_none() else []):
            for km in _iter_kmatrix(k):
                km.span = None
    for n in todo:
        if isinstance(n, DotProdNode):
            _note_span(n.kargs[0], n.children_shapes[0])
            _note_span(n.kargs[1], n.children_shapes[1])
            if not n.kres.is_none():
                _note_span(n.kres, n.shape)
        elif isinstance(n, ReduceNode):
            _note_span(n.kargs[0], n.children_shapes[0])
            if not n.kres.is_none():
                _note_span(n.kres, n.shape)
        elif isinstance(n, Receiver):
            for k in n.kargs:
                _note_span(k, k.shape)
        else:                       # elementwise statements, copies, Feeders
            for k in n.kargs:
                _note_span(k, n.shape)
            if n.kres is not None and not n.kres.is_none():
                _note_span(n.kres, n.shape)


def _region(km: KMatrix, buffers: BufferInfo, coarse: bool = False):
    """``((key, lo, hi), var)``: the floats ``[lo, hi)`` of memory ``key``
    an access can touch.  An access of a tetris variable is bounded by the
    variable and, unless ``coarse``, by its span as well (a slice of the
    variable, such as one head's block of a concatenated result); with an
    unpacked arena the key is the variable and the range relative to it."""
    var = getattr(km, "tetris_var", None)
    span = getattr(km, "span", None)
    if var is not None:
        vid, off, size = var
        lo, hi = off, off + size
        if span is not None and not coarse and max(lo, span[0]) < min(hi, span[1]):
            lo, hi = max(lo, span[0]), min(hi, span[1])
        if buffers.unpacked:
            return (("tv", vid), lo - off, hi - off), vid
        return (km.id, lo, hi), vid
    if span is not None:
        return (km.id, span[0], span[1]), ("buf", km.id)
    return (km.id, 0, buffers.size.get(km.id, 1 << 62)), ("buf", km.id)


def _km_ptr(params, km: KMatrix, c: int) -> str:
    """The pointer parameter of a buffer access with folded offset ``c``: a
    tetris variable is addressed relative to its own start (its storage is
    placed by the device), any other buffer relative to the buffer."""
    var = getattr(km, "tetris_var", None)
    if var is not None:
        return params.ptr("var", (km.id,) + tuple(var), c - var[1])
    return params.ptr("buf", km.id, c)


def _unval(e):
    while type(e) is Val:
        e = e.v
    return e


def _loc_sig(km: KMatrix, index_kind: str, n_cols: int):
    """Location of an access as a function of the element index ``g``:
    ``("g", c)`` when it is ``g + c`` (then distinct elements touch distinct
    locations), otherwise ``("e", text, c)``.  Elements are ``Global`` for
    elementwise commands, ``X * n_cols + Y`` for a DotProd and ``X`` for a
    Reduce."""
    core, c = split_const(km.access)
    core = _unval(core)
    if isinstance(core, Global):
        return ("g", c)
    if index_kind == "red" and isinstance(core, X):
        return ("g", c)
    if index_kind == "dp" and type(core) is Add:
        a, b = _unval(core.a), _unval(core.b)
        if isinstance(a, Y):
            a, b = b, a
        if isinstance(b, Y):
            if n_cols == 1 and isinstance(a, X):
                return ("g", c)
            if type(a) in (ShiftLeft, Mult) and isinstance(_unval(a.a), X):
                k = const_of(a.b)
                if k is not None and (1 << int(k) if type(a) is ShiftLeft else int(k)) == n_cols:
                    return ("g", c)
    return ("e", repr(core), c)


def temp_access_violations(stmts, index_kind: str, n_cols: int = 1):
    """Temps read through an access that is not the element's own location,
    as ``(statement index, temp id, access text)``.  The reference lowers a
    temp operand to its register whatever the access (karg.py:47-48), so a
    fused node reading an in-group temp through, e.g., a permute silently
    reads its own element's value instead."""
    out = []
    for si, (kind, n) in enumerate(stmts):
        if kind in ("tmp", "load", "store", "sum", "init"):
            continue
        for k in n.kargs:
            for km in _iter_kmatrix(k):
                if km.is_temp and _loc_sig(km, index_kind, n_cols) != ("g", 0):
                    out.append((si, km.id, repr(km.access)))
    return out


def conflict_pairs(stmts, buffers: BufferInfo, index_kind: str, n_cols: int = 1):
    """Pairs ``(i, j)``, ``i <= j``, of statement indices that must not run
    in the same pass over the elements: some element's access in one may
    touch a location that another element accesses in the other, with at
    least one of them a write.  Under the reference's statement-by-statement
    semantics, ``i`` must then finish for every element before ``j`` starts
    (``i == j``: the statement's reads must all precede its writes).

    Accesses on disjoint regions never conflict; two accesses whose location
    is ``g + c`` with the same ``c`` touch, for every element, a location no
    other element touches.  A DotProd/Reduce operand is read for whole
    rows/columns, so any write overlapping it conflicts."""
    reads, writes = [], []
    for si, (kind, n) in enumerate(stmts):
        if kind in ("tmp", "load", "store"):
            continue
        whole = kind == "init"
        for k in n.kargs:
            for km in _iter_kmatrix(k):
                if not km.is_temp:
                    reads.append((km, whole, si))
        if not n.kres.is_none() and not n.kres.is_temp:
            writes.append((n.kres, False, si))
    out = set()
    for w, _, wi in writes:
        wr, _ = _region(w, buffers)
        wsig = _loc_sig(w, index_kind, n_cols)
        for r, whole, ri in reads + [(x, False, xi) for x, _, xi in writes if x is not w]:
            rr, _ = _region(r, buffers)
            if rr[0] != wr[0] or rr[2] <= wr[1] or wr[2] <= rr[1]:
                continue
            if not whole and wsig[0] == "g" and _loc_sig(r, index_kind, n_cols) == wsig:
                continue
            out.add((min(wi, ri), max(wi, ri)))
    return sorted(out)


def stmt_regions(stmts, buffers: BufferInfo):
    """Buffer ranges ``(buffer, lo, hi)`` (floats) a statement list may read
    and may write: the packed region of each arena variable it addresses, or
    the whole buffer otherwise."""
    reads, writes = set(), set()
    for kind, n in stmts:
        if kind in ("tmp", "load", "store", "sum"):
            continue
        for k in n.kargs:
            for km in _iter_kmatrix(k):
                if not km.is_temp:
                    reads.add(_region(km, buffers)[0])
        if not n.kres.is_none() and not n.kres.is_temp:
            writes.add(_region(n.kres, buffers)[0])
    return sorted(reads, key=repr), sorted(writes, key=repr)


def command_regions(cmd, buffers: BufferInfo):
    nodes = cmd.nodes if hasattr(cmd, "nodes") else [cmd]
    return stmt_regions(statements(nodes), buffers)


def components(stmts, buffers: BufferInfo):
    """Split an elementwise statement list into groups that share no temp
    and no memory range one of them writes; each group keeps its statements
    in order.  Groups are independent: any order of running them (or running
    them at once) gives the result of the whole list."""
    parent = list(range(len(stmts)))

    def find(i):
        while parent[i] != i:
            parent[i] = parent[parent[i]]
            i = parent[i]
        return i

    def union(i, j):
        ri, rj = find(i), find(j)
        if ri != rj:
            parent[max(ri, rj)] = min(ri, rj)

    defined, decl = {}, {}
    accesses = {}
    for i, (kind, n) in enumerate(stmts):
        if kind == "tmp":
            decl[n.id] = i
            continue
        if not n.kres.is_none() and n.kres.is_temp:
            defined[n.kres.id] = i
    for i, (kind, n) in enumerate(stmts):
        if kind == "tmp":
            continue
        for k in n.kargs:
            for km in _iter_kmatrix(k):
                if km.is_temp:
                    j = defined.get(km.id, decl.get(km.id))
                    if j is not None:
                        union(i, j)
                else:
                    (buf, lo, hi), _ = _region(km, buffers)
                    accesses.setdefault(buf, []).append((lo, hi, i, False))
        if not n.kres.is_none():
            if n.kres.is_temp:
                if n.kres.id in decl:
                    union(i, decl[n.kres.id])
            else:
                (buf, lo, hi), _ = _region(n.kres, buffers)
                accesses.setdefault(buf, []).append((lo, hi, i, True))
    # sweep each buffer's accesses by start: a write joins every live access
    # it overlaps.  All live writes are already joined, so the one reaching
    # furthest stands for them; reads since the last write are kept until the
    # next write joins (and so merges) the live ones.
    for buf, acc in accesses.items():
        acc.sort(key=lambda a: (a[0], a[1]))
        write_rep = None           # (hi, stmt) of the furthest-reaching live write
        reads = []                 # reads not yet merged by a write: (hi, stmt)
        for lo, hi, i, is_write in acc:
            if hi <= lo:
                continue
            if write_rep is not None and write_rep[0] <= lo:
                write_rep = None
            if write_rep is not None:
                union(i, write_rep[1])
            if is_write:
                live = [r for r in reads if r[0] > lo]
                for _, j in live:
                    union(i, j)
                reads = [max(live)] if live else []
                write_rep = (hi, i) if write_rep is None or hi > write_rep[0] else write_rep
            else:
                reads.append((hi, i))
    groups = {}
    for i in range(len(stmts)):
        groups.setdefault(find(i), []).append(stmts[i])
    return [groups[r] for r in sorted(groups)]


# ------------------------------------------------------------------ lowering helpers
MAX_PTR_PARAMS = 48


class Params:
    """Kernel pointer parameters keyed by (buffer id, folded offset).  Past
    ``MAX_PTR_PARAMS`` distinct pointers, further offsets are added to the
    buffer's base pointer in the source instead (a command that touches
    hundreds of arena slots compiles to its own kernel either way)."""

    def __init__(self):
        self.slots: List[tuple] = []
        self.index: Dict[tuple, int] = {}

    def _slot(self, key) -> int:
        if key not in self.index:
            self.index[key] = len(self.slots)
            self.slots.append(key)
        return self.index[key]

    def ptr(self, kind, ident, offset) -> str:
        key = (kind, ident, offset)
        if key in self.index or len(self.slots) < MAX_PTR_PARAMS or offset == 0:
            return f"p{self._slot(key)}"
        return f"(p{self._slot((kind, ident, 0))} + {offset}LL)"


def lower_index(e, ity) -> str:
    c = const_of(e)
    if c is not None:
        return f"(({ity}){int(c)})"
    if isinstance(e, Global):
        return "_global_id"
    if isinstance(e, X):
        return "_x"
    if isinstance(e, Y):
        return "_y"
    if type(e) is Val:
        return lower_index(e.v, ity)
    op = _OPS[type(e)]
    return f"({lower_index(e.a, ity)} {op} {lower_index(e.b, ity)})"


def const_literal(c) -> str:
    """The reference emits ``str(constant)``: a double literal for floats."""
    if isinstance(c, float):
        if math.isinf(c) or math.isnan(c):
            return "(__builtin_huge_val())" if c > 0 else ("(-__builtin_huge_val())" if c < 0 else "(__builtin_nan(\"\"))")
        return repr(c)
    return str(c)


def _scratch_km(off, access=None):
    km = KMatrix(-1, access if access is not None else Global(), [1])
    km.scratch_offset = off
    return km


HOIST_MAX = 8


def _stream_arg(km) -> str:
    """Template argument of ``adhip::ld4`` / ``st4`` for an access: true for
    a KMatrix the device marked ``stream`` (data no other command reads)."""
    return "true" if getattr(km, "stream", False) else "false"

_NO_SIZES = BufferInfo()


@dataclass(frozen=True)
class PlanOptions:
    """Choices that change results, all off by default (the reference's):
    ``exact_reduce`` -- reductions combine every element (``kept_elements``);
    ``dot`` -- "bf16" rounds the operands of DotProds of at least
    ``bf16_min_macs`` multiply-adds to bfloat16 and sums in fp32 on bf16 MFMA
    (``pack_plan``, ``dotprod_bf16_plan``); smaller ones stay fp32."""
    exact_reduce: bool = False
    dot: str = "fp32"
    bf16_min_macs: int = 1 << 30


DEFAULT_OPTIONS = PlanOptions()


class _StoreTracker:
    """The regions one element has stored to so far, and the operand reads
    hoisted ahead of every store (``_l[k]``, up to ``limit`` of them)."""

    def __init__(self, limit, slot="_l[{}]"):
        self.limit = limit
        self.slot = slot                # how a hoisted read is named (its index filled in)
        self.stored: List[tuple] = []
        self.scratch_stored = False
        self.loads: List[str] = []
        self._idx: Dict[str, int] = {}

    def free(self, karg) -> bool:
        """True if no store so far may have written what ``karg`` reads."""
        if isinstance(karg, KConcat):
            return self.free(karg.karg_one) and self.free(karg.karg_two)
        if isinstance(karg, KConstant):
            return True                 # reads nothing
        if not isinstance(karg, KMatrix) or karg.is_temp:
            return False
        if getattr(karg, "scratch_offset", None) is not None:
            return not self.scratch_stored
        buf, lo, hi = _region(karg, _NO_SIZES)[0]
        return not any(b == buf and lo < h and l < hi for b, l, h in self.stored)

    def hoisted(self, expr):
        """``_l[k]`` for ``expr`` (one slot per distinct expression), or None
        when the slots are used up."""
        if expr not in self._idx:
            if len(self.loads) >= self.limit:
                return None
            self._idx[expr] = len(self.loads)
            self.loads.append(expr)
        return self.slot.format(self._idx[expr])

    def note(self, km):
        if getattr(km, "scratch_offset", None) is not None:
            self.scratch_stored = True
        else:
            self.stored.append(_region(km, _NO_SIZES)[0])


# a left-nested chain of at least this many concat pieces along one index
# is selected by a balanced tree of comparisons
CONCAT_BALANCE_MIN = 4


def balance_concat(k):
    """The same operand with every left-nested chain of concats along one
    index expression (``Concat(Concat(Concat(a, b), c), d)``: conditions
    ``e > t`` with the same ``e`` and falling thresholds ``t``, as
    kernalize.make_karg builds them) rebuilt as a balanced tree of
    comparisons against the same thresholds: each element still reads
    only the piece whose range holds it, after about log2(n) comparisons
    instead of up to n.  The concat of a head-by-sample result (128 pieces)
    otherwise costs up to 128 dependent selects per element.  Operands that
    are no such chain come back with their pieces balanced."""
    if not isinstance(k, KConcat) or getattr(k, "balanced", False):
        return k

    def split(cond):
        if type(cond) is MoreThan:
            t = const_of(cond.b)
            if t is not None:
                return repr(cond.a), int(t)
        return None, None

    key, _ = split(k.condition)
    chain, node = [], k
    if key is not None:
        while isinstance(node, KConcat):
            kk, t = split(node.condition)
            if kk != key or (chain and t >= chain[-1][0]):
                break
            chain.append((t, node.karg_two))
            node = node.karg_one
    if len(chain) < CONCAT_BALANCE_MIN:
        out = KConcat(balance_concat(k.karg_one), balance_concat(k.karg_two), k.condition, k.shape)
        out.balanced = True
        return out
    asc = sorted(chain, key=lambda x: x[0])
    pieces = [balance_concat(node)] + [balance_concat(p) for _, p in asc]
    thresholds = [None] + [t for t, _ in asc]
    e = k.condition.a

    def build(lo, hi):
        # pieces[j] serves e in (thresholds[j], thresholds[j + 1]]; pieces[0] e <= thresholds[1]
        if lo == hi:
            return pieces[lo]
        mid = (lo + hi + 1) // 2
        out = KConcat(build(lo, mid - 1), build(mid, hi), MoreThan(e, Val(Constant(thresholds[mid]))), k.shape)
        out.balanced = True
        return out
    return build(0, len(pieces) - 1)


class Lowerer:
    """Emits scalar C++ for operands and statements of one kernel.

    With ``hoist`` the operand reads that no earlier store of the same
    element can reach (no store so far overlaps their region) become
    ``_l[k]``, and ``loads`` lists the expressions that fill ``_l``: the
    caller evaluates them for a batch of elements before running any of
    their statements, so the loads are in flight together instead of each
    waiting behind the previous element's stores (which may alias them as
    far as the compiler knows).  Elements never touch each other's
    locations within one pass (cross-element conflicts split passes), so
    only the element's own earlier stores matter."""

    def __init__(self, ity, params: Params, hoist=False, stream=False):
        self.ity = ity
        self.params = params
        self.stream = stream                  # nontemporal operand loads
        self.forward: Dict[tuple, str] = {}   # location key -> register holding its value
        self.nreg = 0
        self.hoist = hoist
        self.stores = _StoreTracker(HOIST_MAX)

    @property
    def loads(self) -> List[str]:
        return self.stores.loads

    def _free(self, karg) -> bool:
        return self.stores.free(karg)

    def _hoisted(self, expr) -> str:
        return self.stores.hoisted(expr)

    def _note_store(self, km):
        self.stores.note(km)

    @property
    def _scratch_stored(self):
        return self.stores.scratch_stored

    @_scratch_stored.setter
    def _scratch_stored(self, v):
        self.stores.scratch_stored = v

    def _loc(self, km: KMatrix):
        core, c = split_const(km.access)
        if getattr(km, "scratch_offset", None) is not None:
            p = self.params.ptr("scratch", 0, km.scratch_offset + c)
        else:
            p = _km_ptr(self.params, km, c)
        idx = lower_index(core, self.ity)
        return p, idx, (p, repr(core))

    def operand(self, karg) -> str:
        if isinstance(karg, KConstant):
            return const_literal(karg.constant)
        if self.hoist and self._free(karg):
            self.hoist = False
            try:
                expr = self.operand(karg)
            finally:
                self.hoist = True
            return self._hoisted(expr) or expr
        if isinstance(karg, KConcat):
            # each piece is read only where the condition selects it: its
            # access may point outside its buffer for the elements the other
            # piece serves (a slice read as ``(g % n) - c`` underflows below
            # c), so no piece's load is hoisted out of the conditional
            karg = balance_concat(karg)
            cond = lower_index(karg.condition, self.ity)
            hoist, self.hoist = self.hoist, False
            try:
                return f"({cond} ? ({self.operand(karg.karg_two)}) : ({self.operand(karg.karg_one)}))"
            finally:
                self.hoist = hoist
        if karg.is_temp:
            return f"temp_{karg.id}"
        p, idx, key = self._loc(karg)
        if key in self.forward:
            return self.forward[key]
        if self.stream:
            return f"__builtin_nontemporal_load({p} + {idx})"
        return f"{p}[{idx}]"

    def rhs(self, kind, n, init_value) -> str:
        if kind == "bin":
            op = "+" if n.op == BinaryOp.ADD else "*"
            return f"{self.operand(n.kargs[0])} {op} {self.operand(n.kargs[1])}"
        if kind == "copy":
            return self.operand(n.kargs[0])
        if kind == "init":
            return init_value
        a = self.operand(n.kargs[0])
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

    def statements(self, stmts, init_value) -> List[str]:
        """Per-element statement list with store-to-load forwarding; stores of
        non-temp results are emitted in program order (a later store to the
        same location wins)."""
        lines = []
        for kind, n in stmts:
            if kind == "tmp":
                lines.append(f"float temp_{n.id} = 0.0f;")
                continue
            if kind == "load":          # temp carried in from an earlier pass
                tid, off = n
                expr = f"{self.params.ptr('scratch', 0, off)}[_global_id]"
                if self.hoist and not self._scratch_stored:
                    expr = self._hoisted(expr) or expr
                lines.append(f"float temp_{tid} = {expr};")
                continue
            if kind == "store":         # temp carried out to a later pass
                tid, off = n
                lines.append(f"{self.params.ptr('scratch', 0, off)}[_global_id] = temp_{tid};")
                self._scratch_stored = True
                continue
            if kind == "sum":           # combine the chunk results of a split pass, in order
                off, chunks, count, op, pad_zero = n
                pp = self.params.ptr("scratch", 0, off)
                lines.append(f"float _value = {pp}[_global_id];")
                for c in range(1, chunks):
                    nxt = f"{pp}[(unsigned long long)_global_id + {c * count}ull]"
                    lines.append(f"_value = fmaxf(_value, {nxt});" if op else f"_value = _value + {nxt};")
                if op and pad_zero:
                    lines.append("_value = fmaxf(_value, 0.0f);")
                continue
            value = self.rhs(kind, n, init_value)
            if n.kres.is_temp:
                lines.append(f"temp_{n.kres.id} = {value};")
                continue
            r = f"r{self.nreg}"
            self.nreg += 1
            lines.append(f"const float {r} = {value};")
            p, idx, key = self._loc(n.kres)
            lines.append(f"{p}[{idx}] = {r};")
            self.forward[key] = r
            self._note_store(n.kres)
        return lines

    def prefetched_statements(self, stmts, init_value, batch) -> List[str]:
        """``statements`` with every operand read that no earlier store of
        the element can reach issued ahead of the statements, ``batch``
        distinct reads at a time: a batch's reads (``_pK``), a scheduling
        barrier, then the statements up to the one that completed the
        batch.  Without the barrier the compiler may keep the loads next to
        their uses and wait for each in turn (a pass of 58 scaled copies
        compiled to 174 loads, 167 of them followed by a wait for all
        memory operations).  A read is hoisted only past stores that cannot reach
        it (``_StoreTracker.free``); a concat read moves whole, condition
        included."""
        self.hoist = True
        self.stores = _StoreTracker(1 << 30, slot="_p{}")
        out, body, first = [], [], 0

        def flush():
            nonlocal body, first
            new = self.stores.loads[first:]
            out.extend(f"const float _p{first + i} = {e};" for i, e in enumerate(new))
            if new:
                out.append("__builtin_amdgcn_sched_barrier(0);")
            out.extend(body)
            body, first = [], len(self.stores.loads)
        for st in stmts:
            body.extend(self.statements([st], init_value))
            if len(self.stores.loads) - first >= batch:
                flush()
        flush()
        return out


def _ity(bound) -> str:
    return "unsigned" if bound < (1 << 31) else "unsigned long long"


def _expr_bound(stmts, gmax, xmax, ymax):
    b = max(gmax, xmax, ymax, 1)
    for kind, n in stmts:
        if kind in ("tmp", "load", "store", "sum"):
            continue
        ks = list(n.kargs) + ([n.kres] if not n.kres.is_none() else [])
        for k in ks:
            for km in _iter_kmatrix(k):
                b = max(b, upper_bound(km.access, gmax, xmax, ymax))
            if isinstance(k, KConcat):
                b = max(b, upper_bound(k.condition, gmax, xmax, ymax))
    return b


def _params_decl(params: Params) -> str:
    return ", ".join(f"float* p{i}" for i in range(len(params.slots)))


def _plan_args(params: Params, extra_ints=()) -> List[tuple]:
    out = []
    for kind, ident, off in params.slots:
        out.append(("scratch", off) if kind == "scratch" else (kind, ident, off))
    out.extend(("int", v) for v in extra_ints)
    return out


KNAME = "adhip_kernel"


# ------------------------------------------------------------------ ElwFuse family
def _moving(index_kind):
    """Index variables that advance with the element index inside an aligned
    group of 4 elements, and those that are 0, per element space."""
    if index_kind == "dp":
        return (Global, Y), ()            # valid when the row length is a multiple of 4
    if index_kind == "dpT":
        return (Global, X), ()            # valid when the column length is a multiple of 4
    if index_kind == "red":
        return (Global, X), (Y,)
    return (Global,), ()


def _vec_access_ok(km, index_kind, write):
    core, c = split_const(km.access)
    moving, zero = _moving(index_kind)
    vc = vec_class(core, moving, zero)
    if vc.kind == AFF and vc.al and c % 4 == 0:
        return True
    return vc.kind == INV and not write


def _vec_operand_ok(k, index_kind):
    if isinstance(k, KConstant):
        return True
    if isinstance(k, KConcat):
        moving, zero = _moving(index_kind)
        return (vec_class(k.condition, moving, zero).kind == INV
                and _vec_operand_ok(k.karg_one, index_kind) and _vec_operand_ok(k.karg_two, index_kind))
    return k.is_temp or _vec_access_ok(k, index_kind, False)


def _vector_plan(stmts, n, index_kind="global", n_cols=1):
    """Lane layout for 4 elements per thread: every read must be contiguous
    and 4-aligned, or constant over aligned groups of 4 (a concat's condition
    too), and every write contiguous and aligned, with folded offsets that
    are multiples of 4 floats."""
    if n % 4 != 0 or (index_kind in ("dp", "dpT") and n_cols % 4 != 0):
        return False
    for kind, node in stmts:
        if kind in ("tmp", "load", "store", "sum"):
            continue
        # an init statement's value is the product or reduction (never its
        # operands, which are read in their own kernel)
        if kind != "init":
            for k in node.kargs:
                if not _vec_operand_ok(k, index_kind):
                    return False
        if not node.kres.is_temp and not _vec_access_ok(node.kres, index_kind, True):
            return False
    return True


def _index_setup(index_kind, ity, n_cols):
    if index_kind == "dp":
        return (f"const {ity} _x = _global_id / ({ity}){n_cols}; "
                f"const {ity} _y = _global_id % ({ity}){n_cols}; (void)_x; (void)_y;")
    if index_kind == "dpT":                 # elements in column order; n_cols = rows
        return (f"const {ity} _x = _global_id % ({ity}){n_cols}; "
                f"const {ity} _y = _global_id / ({ity}){n_cols}; (void)_x; (void)_y;")
    if index_kind == "red":
        return f"const {ity} _x = _global_id; const {ity} _y = 0; (void)_x; (void)_y;"
    return ""


SCALAR_MAX_N, SCALAR_MIN_STMTS = 1 << 18, 8
# a longer pass runs one element per thread too when it reads many distinct
# operands (sums of per-head gradients): measured at 2^22 elements, 16
# inputs 50 -> 43 us, 48 inputs 173 -> 141 us
SCALAR_WIDE_MAX_N, SCALAR_WIDE_MIN_LOADS = 1 << 23, 16
STREAM_PASS_BYTES = 256 << 20


def _distinct_loads(stmts) -> int:
    """Distinct memory operands (buffer, access) the statements read."""
    seen = set()
    for kind, node in stmts:
        if kind == "tmp" or not hasattr(node, "kargs"):
            continue
        for k in node.kargs:
            for km in _iter_kmatrix(k):
                if not km.is_temp:
                    seen.add((km.id, repr(km.access)))
    return len(seen)


# operand reads issued together ahead of the statements of a heavy
# one-element-per-thread pass (``Lowerer.prefetched_statements``)
PREFETCH_BATCH = 64


def elementwise_plan(stmts, n, index_kind="global", n_cols=1, flops=0, init_value=None) -> KernelPlan:
    """One thread per element (or per 4 elements when every access allows a
    float4), statements in order.  ``index_kind`` defines ``_x``/``_y`` for
    statements lifted out of a DotProd (``dp``: row = g / n_cols) or Reduce
    (``red``: row = g) command."""
    params = Params()
    bound = _expr_bound(stmts, max(n - 1, 0), max(n - 1, 0), max(n_cols - 1, 0))
    ity = _ity(bound)
    setup = _index_setup(index_kind, ity, n_cols)
    # a short pass with long statement chains runs one element per thread:
    # at 4 per thread it would leave about one wave per SIMD to hide the
    # latency of every dependent load (measured on the C5 gradient sums:
    # 196 us vector, 80 us scalar for 2^18 elements and ~75 statements)
    heavy = sum(1 for k, _ in stmts if k != "tmp") > SCALAR_MIN_STMTS and (
        n <= SCALAR_MAX_N or (n <= SCALAR_WIDE_MAX_N and _distinct_loads(stmts) >= SCALAR_WIDE_MIN_LOADS))
    if heavy or not _vector_plan(stmts, n, index_kind, n_cols):
        block = BLOCK
        # a wide pass that reads more than the 256 MB last-level cache holds
        # loads every operand nontemporally: none of it stays cached for a
        # later command anyway (measured on a 48-operand sum of 2^22
        # elements: 141 -> 125 us)
        low = Lowerer(ity, params, stream=heavy and n > SCALAR_MAX_N and
                      4 * n * _distinct_loads(stmts) > STREAM_PASS_BYTES)
        lines = low.prefetched_statements(stmts, init_value, PREFETCH_BATCH) if heavy else \
            low.statements(stmts, init_value)
        body = "\n    ".join(lines)
        src = f"""extern "C" __global__ void __launch_bounds__({block}) {KNAME}({_params_decl(params)}{', ' if params.slots else ''}unsigned long long n_) {{
  const {ity} _global_id = ({ity})blockIdx.x * {block}u + threadIdx.x;
  if (_global_id >= ({ity})n_) return;
  {setup}
  {body}
}}
"""
        grid = (max(1, ceil(n / block)), 1, 1)
    else:
        block = BLOCK
        src = _vector_source(stmts, ity, params, setup, index_kind)
        grid = (max(1, ceil(n / (4 * BLOCK))), 1, 1)
    return KernelPlan(src, grid, (block, 1, 1), _plan_args(params, (n,)), family="elw", flops=flops)


def _vector_source(stmts, ity, params: Params, setup="", index_kind="global") -> str:
    """Four consecutive elements per thread: float4 loads/stores for aligned
    contiguous accesses, one scalar load for group-constant accesses, a
    concat evaluated once per group (its condition is group-constant)."""
    body = "\n  ".join(_vector_lines(stmts, ity, params, index_kind))
    return f"""extern "C" __global__ void __launch_bounds__({BLOCK}) {KNAME}({_params_decl(params)}{', ' if params.slots else ''}unsigned long long n_) {{
  const {ity} _global_id = (({ity})blockIdx.x * {BLOCK}u + threadIdx.x) * 4u;
  if (_global_id >= ({ity})n_) return;
  {setup}
  {body}
}}
"""


def _vector_lines(stmts, ity, params: Params, index_kind="global", hoist=None) -> List[str]:
    """Statement lines for four consecutive elements ``_global_id`` ..
    ``_global_id + 3`` (``_global_id`` a multiple of 4).  With ``hoist`` (a
    ``_StoreTracker``) the reads no earlier store of the group can reach
    become float4 slots ``_l[k]`` whose expressions go to ``hoist.loads``."""
    lines = []
    loaded: Dict[tuple, List[str]] = {}
    written: Dict[tuple, str] = {}
    cnt = [0]

    def fresh(prefix):
        cnt[0] += 1
        return f"{prefix}{cnt[0]}"

    def loc(km):
        core, c = split_const(km.access)
        if getattr(km, "scratch_offset", None) is not None:
            p = params.ptr("scratch", 0, km.scratch_offset + c)
        else:
            p = _km_ptr(params, km, c)
        return p, core, (p, repr(core))

    def vec_expr(k):
        """A float4-valued expression for an operand (lazy for concats)."""
        if isinstance(k, KConstant):
            lit = f"(float)({const_literal(k.constant)})"
            return f"make_float4({lit}, {lit}, {lit}, {lit})"
        if isinstance(k, KConcat):
            k = balance_concat(k)
            cond = lower_index(k.condition, ity)
            return f"(({cond}) ? {vec_expr(k.karg_two)} : {vec_expr(k.karg_one)})"
        if k.is_temp:
            return f"make_float4(temp_{k.id}[0], temp_{k.id}[1], temp_{k.id}[2], temp_{k.id}[3])"
        p, core, key = loc(k)
        if key in written:
            return written[key]
        idx = lower_index(core, ity)
        moving, zero = _moving(index_kind)
        if vec_class(core, moving, zero).kind == AFF:
            return f"adhip::ld4<{_stream_arg(k)}>({p} + {idx})"
        v = f"{p}[{idx}]"
        return f"make_float4({v}, {v}, {v}, {v})"

    def operand(k):
        """Per-lane expressions of an operand; loads are hoisted into locals
        in program order (a location read twice is loaded once)."""
        if isinstance(k, KConstant):
            return [const_literal(k.constant)] * 4
        if isinstance(k, KMatrix) and k.is_temp:
            return [f"temp_{k.id}[{i}]" for i in range(4)]
        if isinstance(k, KMatrix):
            p, core, key = loc(k)
            if key in written:
                return [f"{written[key]}.{c}" for c in "xyzw"]
            if key in loaded:
                return loaded[key]
        expr = vec_expr(k)
        slot = hoist.hoisted(expr) if hoist is not None and hoist.free(k) else None
        if slot is not None:
            vals = [f"{slot}.{c}" for c in "xyzw"]
            if isinstance(k, KMatrix):
                loaded[loc(k)[2]] = vals
            return vals
        v = fresh("v")
        lines.append(f"const float4 {v} = {expr};")
        vals = [f"{v}.{c}" for c in "xyzw"]
        if isinstance(k, KMatrix):
            loaded[loc(k)[2]] = vals
        return vals

    def rhs(kind, n, lane):
        def op(k):
            return operand(k)[lane]
        if kind == "bin":
            o = "+" if n.op == BinaryOp.ADD else "*"
            return f"{op(n.kargs[0])} {o} {op(n.kargs[1])}"
        if kind == "copy":
            return op(n.kargs[0])
        if kind == "init":
            return f"_value.{'xyzw'[lane]}"
        a = op(n.kargs[0])
        u = n.op
        if u == UnaryOp.EXP2:
            return f"exp2({a})"
        if u == UnaryOp.LOG2:
            return f"log2({a})"
        if u == UnaryOp.SIN:
            return f"sin({a})"
        if u == UnaryOp.RECIP:
            return f"1.0/{a}"
        if u == UnaryOp.SQRT:
            return f"sqrt(fabs({a}))"
        cmp = {UnaryOp.EQUAL: "==", UnaryOp.MORE_ZERO: ">", UnaryOp.LESS_ZERO: "<",
               UnaryOp.MORE_OR_EQ_ZERO: ">=", UnaryOp.LESS_OR_EQ_ZERO: "<="}[u]
        return f"({a} {cmp} 0.0f) ? 1.0 : 0.0"

    for kind, n in stmts:
        if kind == "tmp":
            lines.append(f"float temp_{n.id}[4] = {{0.0f, 0.0f, 0.0f, 0.0f}};")
            continue
        if kind == "load":
            tid, off = n
            expr = f"(*reinterpret_cast<const float4*>({params.ptr('scratch', 0, off)} + _global_id))"
            v = hoist.hoisted(expr) if hoist is not None and not hoist.scratch_stored else None
            if v is None:
                v = fresh("v")
                lines.append(f"const float4 {v} = {expr};")
            lines.append(f"float temp_{tid}[4] = {{{v}.x, {v}.y, {v}.z, {v}.w}};")
            continue
        if kind == "store":
            tid, off = n
            lines.append(f"*reinterpret_cast<float4*>({params.ptr('scratch', 0, off)} + _global_id) = "
                         f"make_float4(temp_{tid}[0], temp_{tid}[1], temp_{tid}[2], temp_{tid}[3]);")
            if hoist is not None:
                hoist.scratch_stored = True
            continue
        if kind == "sum":
            off, chunks, count, op, pad_zero = n
            pp = params.ptr("scratch", 0, off)
            lines.append(f"float4 _value = *reinterpret_cast<const float4*>({pp} + _global_id);")
            for c in range(1, chunks):
                v = fresh("v")
                lines.append(f"const float4 {v} = *reinterpret_cast<const float4*>({pp} + "
                             f"(unsigned long long)_global_id + {c * count}ull);")
                for lane in "xyzw":
                    lines.append(f"_value.{lane} = fmaxf(_value.{lane}, {v}.{lane});" if op
                                 else f"_value.{lane} = _value.{lane} + {v}.{lane};")
            if op and pad_zero:
                for lane in "xyzw":
                    lines.append(f"_value.{lane} = fmaxf(_value.{lane}, 0.0f);")
            continue
        # operands are loaded before the statement computes (program order);
        # an init statement's value is the product or reduction itself
        if kind != "init":
            for k in n.kargs:
                operand(k)
        vals = [rhs(kind, n, i) for i in range(4)]
        if n.kres.is_temp:
            for i in range(4):
                lines.append(f"temp_{n.kres.id}[{i}] = {vals[i]};")
            continue
        p, core, key = loc(n.kres)
        r = fresh("w")
        lines.append(f"float4 {r}; {r}.x = {vals[0]}; {r}.y = {vals[1]}; {r}.z = {vals[2]}; {r}.w = {vals[3]};")
        lines.append(f"adhip::st4<{_stream_arg(n.kres)}>({p} + {lower_index(core, ity)}, {r});")
        written[key] = r
        loaded.pop(key, None)
        if hoist is not None:
            hoist.note(n.kres)
    return lines


# ------------------------------------------------------------------ DotProd+Elw family
def _loader_struct(name, karg, role, params: Params, ity, dims) -> Tuple[str, bool]:
    """Functor ``name`` with ``at(_x, _y)`` for a DotProd operand.  ``role``
    'A': (_x, _y) = (m, k); 'B': (_x, _y) = (k, n).  Returns (source, vec)."""
    M_or_K, second = dims
    if isinstance(karg, KConstant):
        return (f"struct {name} {{ static constexpr int kMode = 0; static constexpr bool kVec = false; @FIELDS@\n"
                f"  __device__ float at({ity} _x, {ity} _y) const {{ (void)_x; (void)_y; return (float)({const_literal(karg.constant)}); }}\n"
                f"  __device__ float4 at4({ity}, {ity}) const {{ return make_float4(0.f, 0.f, 0.f, 0.f); }} }};\n"), False
    low = Lowerer(ity, params)
    if isinstance(karg, KConcat):
        expr = low.operand(karg)
        return (f"struct {name} {{ static constexpr int kMode = 0; static constexpr bool kVec = false; @FIELDS@\n"
                f"  __device__ float at({ity} _x, {ity} _y) const {{ (void)_x; (void)_y; return (float)({expr}); }}\n"
                f"  __device__ float4 at4({ity}, {ity}) const {{ return make_float4(0.f, 0.f, 0.f, 0.f); }} }};\n"), False
    assert isinstance(karg, KMatrix) and not karg.is_temp, "DotProd operand must be a buffer or constant"
    core, c = split_const(karg.access)
    if getattr(karg, "scratch_offset", None) is not None:
        p = params.ptr("scratch", 0, karg.scratch_offset + c)
    else:
        p = _km_ptr(params, karg, c)
    idx = lower_index(core, ity)
    # A: mode 0 contiguous along k (= _y); B: mode 0 contiguous along n (= _y)
    vy = vec_class(core, Y)
    vx = vec_class(core, X)
    if vy.kind == AFF:
        mode = 0
        vec = vy.al and c % 4 == 0 and second % 4 == 0
    elif vx.kind == AFF:
        mode = 1
        vec = vx.al and c % 4 == 0 and M_or_K % 4 == 0
    else:
        mode, vec = 0, False
    if role == "B":
        mode = 0 if mode == 0 else 1
    src = (f"struct {name} {{ static constexpr int kMode = {mode}; static constexpr bool kVec = {'true' if vec else 'false'}; @FIELDS@\n"
           f"  __device__ float at({ity} _x, {ity} _y) const {{ return {p}[{idx}]; }}\n"
           f"  __device__ float4 at4({ity} _x, {ity} _y) const {{ return *reinterpret_cast<const float4*>({p} + {idx}); }} }};\n")
    return src, vec


def _fields(params: Params) -> str:
    return " ".join(f"float* p{i};" for i in range(len(params.slots)))


def _init_list(params: Params) -> str:
    return ", ".join(f"p{i}" for i in range(len(params.slots)))


def dp_config(M, N, K):
    """Block tile and K split of a DotProd: 64-wide tiles on a narrow side,
    128 otherwise (256 x 128 measured slower at 4096^3 and in the C5 step),
    and 64 x 64 for a short K (<= 128), where the epilogue's HBM traffic
    dominates and more, smaller blocks keep more of it in flight, and for
    products of at most 512 x 512 outputs (the per-head attention products,
    launched many at a time: more blocks per compute unit hide latency);
    K is split (up to 16 chunks of at least 256; of at least 512 for a
    K of 1024 or more once the product has 128 blocks: C5 62.0 -> 62.4
    steps/s, C4 unchanged) while the
    tiles alone would not give one block per compute unit, and a long K
    (chunks of at least 1024) is split once more until two blocks share
    each compute unit (one block's barriers then hide behind the other's
    products).  Those attention products with at most 512 terms are not
    split: the scheduler launches them dozens at a time, and a split's
    combine pass costs more than its shorter chains save (measured on the
    C5 step: 649 -> 554 launches, the same step time; C4 +0.8 %)."""
    small = K <= 128 or M * N <= (1 << 18)
    BM = 64 if M <= 64 or small else 128
    BN = 64 if N <= 64 or small else 128
    tiles = ceil(M / BM) * ceil(N / BN)
    split = 1
    if M * N <= (1 << 18) and K <= 512:
        return BM, BN, split, dp_panel(M, N, K, BM, BN, split)
    while tiles * split < 256 and split < 16 and \
            K // (2 * split) >= (512 if tiles * split >= 128 and K >= 1024 else 256):
        split *= 2
    while tiles * split < 512 and split < 16 and K // (2 * split) >= 1024:
        split *= 2
    return BM, BN, split, dp_panel(M, N, K, BM, BN, split)


def dp_buffers(M, N, K, BM, BN, split, BK):
    """LDS buffers of the K panels: one for 128 x 128 and 64 x 64 tiles (the
    next panel, already in registers, stored after a second barrier; three
    alternating runs on one box: 4096^3 DotProd+Elw 112.0 -> 114.4
    TFLOP/s, C5 60.36 -> 60.91 steps/s for the 128 x 128 tiles; with 64-deep
    panels for the 64 x 64 tiles, two runs each: C5 61.0 -> 62.1, C4 643 ->
    652 steps/s), two for the mixed 128 x 64 tiles (the next panel stored
    while the current one is read)."""
    return 1 if BM == BN else 2


def dp_panel(M, N, K, BM, BN, split):
    """Depth of the K panels staged in LDS: 32 for 128-wide tiles (measured
    against 16, 48 and 64 at 4096^3 and on the C5 step: 32 halves the
    barriers per product of 16 and still leaves two blocks per compute
    unit), 64 for 64 x 64 tiles in one buffer (35 KB per block; 16- and
    32-deep panels measured slower on the C5 step: 59.5 and 61.7 against
    62.1 steps/s)."""
    return 64 if BM == 64 and BN == 64 else 32


VEC_HOIST_MAX = 4


def epilogue_vec_ok(stmts, M, N) -> bool:
    """The in-kernel epilogue of an M x N DotProd can run on groups of 4
    consecutive columns: every access it makes (the product's own store
    included) is contiguous and 4-aligned along the row, or constant over
    the group."""
    return N % 4 == 0 and bool(stmts) and _vector_plan(stmts, M * N, "dp", N)


def _dp_epi_struct(stmts, params: Params, ity, M, N, partial_off=None, allow_vec=True) -> str:
    """The ``EPI`` functor of a DotProd kernel: the epilogue statements on
    the product (four consecutive columns per call with float4 accesses when
    every access allows it, else one element per call), or the store of a
    partial product to scratch at ``partial_off`` ([chunk][M][N])."""
    gid = f"const {ity} _global_id = _x * ({ity}){N} + _y; (void)_global_id;"
    if partial_off is not None:
        assert not stmts, "a DotProd storing partial products runs no epilogue"
    vec4 = allow_vec and N % 4 == 0 and (partial_off is not None or epilogue_vec_ok(stmts, M, N))
    if vec4:
        if partial_off is not None:
            pp = params.ptr("scratch", 0, partial_off)
            lines, loads = [f"*reinterpret_cast<float4*>({pp} + ((unsigned long long)_chunk * {M}ull + _x) * "
                            f"{N}ull + _y) = _value;"], []
        else:
            tracker = _StoreTracker(VEC_HOIST_MAX)
            lines = _vector_lines(stmts, ity, params, "dp", hoist=tracker)
            loads = tracker.loads
        body = "\n    ".join(lines)
        fill = "".join(f"\n    _l[{i}] = {e};" for i, e in enumerate(loads))
        return (f"struct EPI {{ @FIELDS@\n"
                f"  static constexpr bool kVec4 = true;\n"
                f"  static constexpr int kLoads = {len(loads)};\n"
                f"  __device__ void load4({ity} _x, {ity} _y, float4* _l) const {{\n"
                f"    {gid} (void)_l;{fill}\n  }}\n"
                f"  __device__ void vec(float4 _value, {ity} _x, {ity} _y, int _chunk, const float4* _l) const {{\n"
                f"    {gid} (void)_chunk; (void)_l;\n    {body}\n  }} }};\n")
    loads = []
    if partial_off is not None:
        pp = params.ptr("scratch", 0, partial_off)
        body = (f"{pp}[((unsigned long long)_chunk * {M}ull + _x) * {N}ull + _y] = _value;")
    else:
        low = Lowerer(ity, params, hoist=True)
        body = "\n    ".join(low.statements(stmts, "_value"))
        loads = low.loads
    fill = "".join(f"\n    _l[{i}] = {e};" for i, e in enumerate(loads))
    return (f"struct EPI {{ @FIELDS@\n"
            f"  static constexpr bool kVec4 = false;\n"
            f"  static constexpr int kLoads = {len(loads)};\n"
            f"  __device__ void load({ity} _x, {ity} _y, float* _l) const {{\n"
            f"    {gid} (void)_l;{fill}\n  }}\n"
            f"  __device__ void operator()(float _value, {ity} _x, {ity} _y, int _chunk, const float* _l) const {{\n"
            f"    {gid} (void)_chunk; (void)_l;\n    {body}\n  }} }};\n")


# products with at most this many rows run ``dp_skinny``, and others with at
# most this many terms per output ``dp_direct`` (no MFMA tile)
SKINNY_M, DIRECT_K = 8, 8

# ``dp_quad``: 32 x 32 tiles, K panels split among a block's 4 waves
QUAD_TILE = 32
# a product on 64 x 64 tiles whose K chunks have at least this many terms
# gets a ``dp_quad`` alternative; a launch group takes it when its 64 x 64
# blocks (all instances) number at most NARROW_MAX_BLOCKS, i.e. half the
# compute units or fewer: there it runs four times the waves on chains a
# quarter as long, and past that the wider tile's lower operand traffic
# per flop wins (measured on the C5 step: 256 instead of 128 blocks, no
# change; K = 64 products included or not, 63.9 steps/s either way)
QUAD_MIN_CHUNK, NARROW_MAX_BLOCKS = 64, 128


def quad_config(M, N, K, config):
    """The ``dp_quad`` configuration of a 64 x 64-tile fp32 product long
    enough in K (same K split; 128-deep panels, 64 for chunks shorter than
    128 terms, so each wave still takes 16 panel columns), else None."""
    BM, BN, split, _ = config
    chunk = ceil(K / split)
    if BM == 64 and BN == 64 and M > SKINNY_M and K > DIRECT_K and chunk >= QUAD_MIN_CHUNK:
        return QUAD_TILE, QUAD_TILE, split, 128 if chunk >= 128 else 64
    return None


def use_narrow(plan: "KernelPlan", instances: int) -> bool:
    """A launch group of ``instances`` copies of ``plan`` runs ``plan.narrow``."""
    return plan.narrow is not None and plan.grid[0] * plan.grid[1] * instances <= NARROW_MAX_BLOCKS


def dotprod_plan(stmts, dp, A=None, B=None, config=None, partial_off=None) -> KernelPlan:
    """DotProd (+ elementwise epilogue) on fp32 MFMA tiles
    (kernels/dotprod.py:7-43, dp_elw_fuse.py:26-65 semantics).  ``A``/``B``
    replace the node's operands (a gathered copy in scratch); with a K split
    (``config[2] > 1``) the blocks store partial products to scratch at
    ``partial_off`` ([chunk][M][N]) and ``stmts`` must be empty; so does an
    unsplit product whose epilogue runs as a separate pass."""
    M, N = dp.shape
    K = dp.children_shapes[0][1]
    BM, BN, split, BK = config if config is not None else dp_config(M, N, K)
    A = dp.kargs[0] if A is None else A
    B = dp.kargs[1] if B is None else B
    bound = _expr_bound(stmts, M * N, max(M, K), max(N, K))
    ity = _ity(bound)
    params = Params()
    la, _ = _loader_struct("LA", A, "A", params, ity, (M, K))
    lb, _ = _loader_struct("LB", B, "B", params, ity, (K, N))
    if M <= SKINNY_M or K <= DIRECT_K:
        assert split == 1, "a skinny or short-K DotProd is not split"
        epi = _dp_epi_struct(stmts, params, ity, M, N, partial_off, allow_vec=False)
        init = _init_list(params)
        if M <= SKINNY_M:
            call, grid = f"adhip::dp_skinny<{SKINNY_M}>", (ceil(N / 16), 1, 1)
        else:
            call, grid = "adhip::dp_direct", (ceil(M * N / 256), 1, 1)
        src = ((la + lb + epi).replace("@FIELDS@", _fields(params)) +
               f"extern \"C\" __global__ void __launch_bounds__(256) {KNAME}({_params_decl(params)}) {{\n"
               f"  {call}(LA{{{init}}}, LB{{{init}}}, EPI{{{init}}}, {M}, {N}, {K});\n}}\n")
        return KernelPlan(src, grid, (256, 1, 1), _plan_args(params), family="dotprod",
                          flops=2 * M * N * K)
    epi = _dp_epi_struct(stmts, params, ity, M, N, partial_off)
    init = _init_list(params)
    if BM == QUAD_TILE:
        assert BN == QUAD_TILE and BK in (64, 128), "dp_quad takes 32 x 32 tiles and 64- or 128-deep panels"
        src = ((la + lb + epi).replace("@FIELDS@", _fields(params)) +
               f"extern \"C\" __global__ void __launch_bounds__(256) {KNAME}({_params_decl(params)}) {{\n"
               f"  adhip::dp_quad<{split}, {BK}>(LA{{{init}}}, LB{{{init}}}, EPI{{{init}}}, {M}, {N}, {K});\n}}\n")
        grid = (ceil(N / QUAD_TILE), ceil(M / QUAD_TILE) * split, 1)
        return KernelPlan(src, grid, (256, 1, 1), _plan_args(params), family="dotprod",
                          flops=2 * M * N * K)
    nbuf = dp_buffers(M, N, K, BM, BN, split, BK)
    tmpl = f"{BM}, {BN}, {split}, {BK}" + (", LA, LB, EPI, 1" if nbuf == 1 else "")
    src = ((la + lb + epi).replace("@FIELDS@", _fields(params)) +
           f"extern \"C\" __global__ void __launch_bounds__(256) {KNAME}({_params_decl(params)}) {{\n"
           f"  adhip::dp_mfma<{tmpl}>(LA{{{init}}}, LB{{{init}}}, EPI{{{init}}}, {M}, {N}, {K});\n}}\n")
    grid = (ceil(N / BN), ceil(M / BM) * split, 1)
    return KernelPlan(src, grid, (256, 1, 1), _plan_args(params), family="dotprod",
                      flops=2 * M * N * K)


# ------------------------------------------------------------------ bf16 DotProd option
BF16_K_ALIGN = 64


def bf16_dims(M, N, K, config):
    """Padded sizes of the packed bf16 operands: rows to the block tile, K to
    a multiple of 64 (the pack tile)."""
    BM, BN = config[0], config[1]
    return ceil(M / BM) * BM, ceil(N / BN) * BN, ceil(K / BF16_K_ALIGN) * BF16_K_ALIGN


# depth of the bf16 K panels (64 measured no faster at 4096^3 and slower on
# the C5 step)
BF16_PANEL = 32


def bf16_config(M, N, K):
    """Block tile and K split of a bf16 DotProd: 256 x 128 where the product
    is that large (each wave 128 x 64, so a fragment read from LDS feeds
    more MFMAs: bf16 products are 16 times faster than fp32 ones and the
    fp32 128 x 128 tile leaves them waiting on LDS and L2; measured 4096^3
    216 -> 355 TFLOP/s with packing, C5 step 69 -> 78 steps/s), else as
    ``dp_config``; K split by the same rule."""
    if M < 256 or N < 128:
        return dp_config(M, N, K)
    BM, BN = 256, 128
    tiles = ceil(M / BM) * ceil(N / BN)
    split = 1
    while tiles * split < 256 and split < 16 and \
            K // (2 * split) >= (512 if tiles * split >= 128 and K >= 1024 else 256):
        split *= 2
    return BM, BN, split, BF16_PANEL


def pack_plan(karg, role, rows, K, rows_pad, k_pad, dst_off, dims) -> KernelPlan:
    """``scratch[dst_off]`` as bf16 ``[rows_pad][k_pad]``: the DotProd operand
    ``karg`` (``role`` "A": element (r, k) is A(r, k); "B": B(k, r)) rounded
    to bf16, k-contiguous, zero padded."""
    bound = _expr_bound([("copy", _Stmt([karg], _scratch_km(0, Global())))], 0,
                        max(rows_pad, k_pad), max(rows_pad, k_pad))
    ity = _ity(bound)
    params = Params()
    ld, _ = _loader_struct("LD", karg, role, params, ity, dims)
    dst = params.ptr("scratch", 0, dst_off)
    init = _init_list(params)
    src = (ld.replace("@FIELDS@", _fields(params)) +
           f"extern \"C\" __global__ void __launch_bounds__(256) {KNAME}({_params_decl(params)}) {{\n"
           f"  adhip::pack_bf16<{0 if role == 'A' else 1}>(LD{{{init}}}, reinterpret_cast<__bf16*>({dst}), "
           f"{rows}, {K}, {k_pad});\n}}\n")
    grid = (k_pad // 64, rows_pad // 64, 1)
    return KernelPlan(src, grid, (256, 1, 1), _plan_args(params), family="pack",
                      bytes=4 * rows * K + 2 * rows_pad * k_pad)


def dotprod_bf16_plan(stmts, dp, a_off, b_off, config, partial_off=None) -> KernelPlan:
    """DotProd (+ epilogue) over operands packed by ``pack_plan`` at scratch
    ``a_off`` / ``b_off``, on bf16 MFMA with fp32 sums; otherwise as
    ``dotprod_plan``.  The kernel is bounded to two blocks per compute unit:
    unbounded, the 256 x 128 tile took 156 VGPRs + 128 AGPRs and ran one
    wave per SIMD (4096^3: 356 TFLOP/s); bounded, 200 registers and two
    waves (443 TFLOP/s)."""
    M, N = dp.shape
    K = dp.children_shapes[0][1]
    BM, BN, split = config[0], config[1], config[2]
    _, _, k_pad = bf16_dims(M, N, K, config)
    bound = _expr_bound(stmts, M * N, max(M, K), max(N, K))
    ity = _ity(bound)
    params = Params()
    pa = params.ptr("scratch", 0, a_off)
    pb = params.ptr("scratch", 0, b_off)
    epi = _dp_epi_struct(stmts, params, ity, M, N, partial_off)
    init = _init_list(params)
    src = (epi.replace("@FIELDS@", _fields(params)) +
           f"extern \"C\" __global__ void __launch_bounds__(256, 2) {KNAME}({_params_decl(params)}) {{\n"
           f"  adhip::dp_bf16<{BM}, {BN}, {split}, {BF16_PANEL}>(reinterpret_cast<const __bf16*>({pa}), "
           f"reinterpret_cast<const __bf16*>({pb}), {k_pad}, EPI{{{init}}}, {M}, {N});\n}}\n")
    grid = (ceil(N / BN), ceil(M / BM) * split, 1)
    return KernelPlan(src, grid, (256, 1, 1), _plan_args(params), family="dotprod",
                      flops=2 * M * N * K)


# ------------------------------------------------------------------ Reduce+Elw family
def tree_inclusion(R):
    """Elements of a row that reach slot 0 of the reference's work-group tree
    (reduce.py:33-43 with L = ceil(R/2)*2), as a sorted list of indices in
    [0, L); indices >= R are zero padding."""
    L = ceil(R / 2) * 2
    if L & (L - 1) == 0:
        return list(range(L))
    sets = [{y} for y in range(L)]
    off = L // 2
    while off > 0:
        for y in range(off):
            sets[y] |= sets[y + off]
        off >>= 1
    return sorted(sets[0])


def kept_elements(R, exact=False):
    """Indices of a row that a reduction combines: those reaching the
    reference's tree (``tree_inclusion``; indices >= R are zero padding), or
    with ``exact`` every one of the R elements and no padding (the fix of the
    tree for non-power-of-two lengths and of MAX's zero padding)."""
    return list(range(R)) if exact else tree_inclusion(R)


def _cols_vec(red, exact=False) -> bool:
    """A column-mode Reduce can load 4 consecutive columns as one float4:
    the kept axis is contiguous and 4-aligned, and no row is dropped by the
    reference's tree."""
    V, R = red.children_shapes[0]
    karg = red.kargs[0]
    if not isinstance(karg, KMatrix) or V % 4 != 0 or len(kept_elements(R, exact)) < R:
        return False
    core, c = split_const(karg.access)
    vx = vec_class(core, X)
    return vx.kind == AFF and vx.al and c % 4 == 0


def reduce_mode(red):
    """``("rows"|"cols", split)`` for a Reduce: rows when the reduced axis is
    contiguous, cols when the kept axis is; rows are split into chunks over
    blocks until there are 512 blocks (two per compute unit; HBM needs that
    many loads in flight)."""
    V, R = red.children_shapes[0]
    karg = red.kargs[0]
    if isinstance(karg, KMatrix):
        core, _ = split_const(karg.access)
        if vec_class(core, Y).kind != AFF and vec_class(core, X).kind == AFF:
            blocks = ceil(V / 64)
            split = 1
            while blocks * split < 512 and split < 128 and R // (2 * split) >= 64:
                split *= 2
            return "cols", split
    return "rows", 1


def reduce_plan(stmts, red, partial_off=None, exact=False) -> KernelPlan:
    """Row reduction (+ epilogue on the reduced value)
    (kernels/reduce.py:8-66, reduce_elw_fuse.py:12-80 semantics).  When the
    columns are split, the blocks store partial results to scratch at
    ``partial_off`` ([chunk][V]) and ``stmts`` must be empty."""
    V, R = red.children_shapes[0]
    inc = kept_elements(R, exact)
    dropped = [y for y in range(R) if y not in set(inc)] if len(inc) < R else []
    pad_zero = any(y >= R for y in inc)
    bound = _expr_bound(stmts, V, V, R)
    ity = _ity(bound)
    params = Params()
    karg = red.kargs[0]
    mode, split = reduce_mode(red)
    vec = False
    if isinstance(karg, KConstant):
        at = f"return (float)({const_literal(karg.constant)});"
        at4 = "return make_float4(0.f, 0.f, 0.f, 0.f);"
    else:
        low0 = Lowerer(ity, params)
        if isinstance(karg, KConcat):
            at = f"return (float)({low0.operand(karg)});"
            at4 = "return make_float4(0.f, 0.f, 0.f, 0.f);"
        else:
            core, c = split_const(karg.access)
            p = _km_ptr(params, karg, c)
            idx = lower_index(core, ity)
            at = f"return {p}[{idx}];"
            at4 = f"return adhip::ld4<{_stream_arg(karg)}>({p} + {idx});"
            vy = vec_class(core, Y)
            if vy.kind == AFF:
                vec = vy.al and c % 4 == 0 and R % 4 == 0 and not dropped
    if dropped:
        words = [0] * ((R + 31) // 32)
        for y in inc:
            if y < R:
                words[y >> 5] |= 1 << (y & 31)
        table = ", ".join(f"{w}u" for w in words)
        inc_fn = (f"  __device__ bool inc({ity} y) const {{ constexpr unsigned t[] = {{{table}}}; "
                  f"return (t[y >> 5] >> (y & 31)) & 1u; }}\n")
    else:
        inc_fn = f"  __device__ bool inc({ity}) const {{ return true; }}\n"
    vecx = mode == "cols" and _cols_vec(red, exact)
    ld = (f"struct LD {{ static constexpr bool kVec = {'true' if vec else 'false'}; "
          f"static constexpr bool kVecX = {'true' if vecx else 'false'}; @FIELDS@\n"
          f"  __device__ float at({ity} _x, {ity} _y) const {{ (void)_x; (void)_y; {at} }}\n"
          f"  __device__ float4 at4({ity} _x, {ity} _y) const {{ (void)_x; (void)_y; {at4} }}\n{inc_fn}}};\n")
    if partial_off is not None:
        assert split > 1, "only a split Reduce stores partial results"
        assert not stmts, "a split Reduce stores partial results only"
        pp = params.ptr("scratch", 0, partial_off)
        body = f"{pp}[(unsigned long long)_chunk * {V}ull + _x] = _v;"
    else:
        low = Lowerer(ity, params)
        body = "\n    ".join(low.statements(stmts, "_v"))
    epi = (f"struct EPI {{ @FIELDS@\n"
           f"  __device__ void operator()(float _v, {ity} _x, int _chunk) const {{\n"
           f"    const {ity} _y = 0; const {ity} _global_id = _x; (void)_y; (void)_global_id; (void)_chunk;\n"
           f"    {body}\n  }} }};\n")
    op = 0 if red.op == ReduceOp.SUM else 1
    init = _init_list(params)
    call = (f"adhip::reduce_rows<{op}>" if mode == "rows" else f"adhip::reduce_cols<{op}, {split}>")
    src = ((ld + epi).replace("@FIELDS@", _fields(params)) +
           f"extern \"C\" __global__ void __launch_bounds__(256) {KNAME}({_params_decl(params)}) {{\n"
           f"  {call}(LD{{{init}}}, EPI{{{init}}}, {V}u, {R}u, {'true' if pad_zero else 'false'});\n}}\n")
    # rows: 4 waves per block, at most 2048 blocks (8 per compute unit); the
    # waves stride over the remaining rows
    grid = (min(ceil(V / 4), 2048), 1, 1) if mode == "rows" else (ceil(V / 64), split, 1)
    return KernelPlan(src, grid, (256, 1, 1), _plan_args(params), family="reduce",
                      bytes=4 * V * R + 4 * V)


# ------------------------------------------------------------------ lockstep fallback
def lockstep_plans(stmts, n, index_kind, n_cols, init_node, scratch_base, opts=DEFAULT_OPTIONS):
    """Exact lockstep semantics for a command with cross-element memory
    dependences: one kernel per statement, each computing its value for every
    element into a staging array before a second kernel stores it.  Temps and
    the DotProd/Reduce value live in scratch arrays.  Returns (plans,
    scratch floats used)."""
    temps = [node.id for kind, node in stmts if kind == "tmp"]
    alloc = ScratchAlloc(scratch_base)
    temp_off = {t: alloc.take(n) for t in temps}
    stage_off = alloc.take(n)
    init_off = alloc.take(n)
    plans = []
    if init_node is not None:
        sink = _scratch_km(init_off, _identity_access(index_kind, n_cols))
        plans.extend(first_pass_plans([("init", _ValueSink(sink))], n, init_node, alloc, opts))
    for kind, node in stmts:
        if kind == "tmp":
            continue
        plans.append(_stmt_plan(kind, node, n, index_kind, n_cols, temp_off, stage_off, init_off,
                                to_stage=True))
        plans.append(_stmt_plan(kind, node, n, index_kind, n_cols, temp_off, stage_off, init_off,
                                to_stage=False))
    return plans, alloc.used


def _identity_access(index_kind, n_cols):
    if index_kind == "dp":
        return Add(Mult(X(), Val(Constant(n_cols))), Y())
    if index_kind == "red":
        return X()
    return Global()


class _ValueSink:
    """A stand-in result node: ``kres`` receives the DotProd/Reduce value."""

    def __init__(self, kres):
        self.kres = kres
        self.kargs = []


def _stmt_plan(kind, node, n, index_kind, n_cols, temp_off, stage_off, init_off, to_stage):
    params = Params()
    bound = max(n, _expr_bound([(kind, node)], max(n - 1, 0), max(n - 1, 0), max(n_cols - 1, 0)))
    ity = _ity(bound)
    low = Lowerer(ity, params)
    # temps and the init value are scratch arrays indexed by element
    init_p = params.ptr("scratch", 0, init_off)

    def operand(karg, _orig=low.operand):
        if isinstance(karg, KMatrix) and karg.is_temp:
            p = params.ptr("scratch", 0, temp_off[karg.id])
            return f"{p}[_global_id]"
        if isinstance(karg, KConcat):
            karg = balance_concat(karg)
            cond = lower_index(karg.condition, ity)
            return f"({cond} ? ({operand(karg.karg_two)}) : ({operand(karg.karg_one)}))"
        return _orig(karg)
    low.operand = operand
    stage_p = params.ptr("scratch", 0, stage_off)
    if to_stage:
        value = low.rhs(kind, node, f"{init_p}[_global_id]")
        line = f"{stage_p}[_global_id] = {value};"
    else:
        if node.kres.is_temp:
            p = params.ptr("scratch", 0, temp_off[node.kres.id])
            line = f"{p}[_global_id] = {stage_p}[_global_id];"
        else:
            p, idx, _ = low._loc(node.kres)
            line = f"{p}[{idx}] = {stage_p}[_global_id];"
    setup = ""
    if index_kind == "dp":
        setup = (f"const {ity} _x = _global_id / ({ity}){n_cols}; "
                 f"const {ity} _y = _global_id % ({ity}){n_cols}; (void)_x; (void)_y;")
    elif index_kind == "red":
        setup = f"const {ity} _x = _global_id; const {ity} _y = 0; (void)_x; (void)_y;"
    src = f"""extern "C" __global__ void __launch_bounds__({BLOCK}) {KNAME}({_params_decl(params)}, unsigned long long n_) {{
  const {ity} _global_id = ({ity})blockIdx.x * {BLOCK}u + threadIdx.x;
  if (_global_id >= ({ity})n_) return;
  {setup}
  {line}
}}
"""
    return KernelPlan(src, (max(1, ceil(n / BLOCK)), 1, 1), (BLOCK, 1, 1), _plan_args(params, (n,)),
                      family="elw")


class _Rebound:
    """A statement node with other operands: every attribute but ``kargs``
    is the node's own (the Proc is not modified)."""

    def __init__(self, node, kargs):
        self._node = node
        self.kargs = kargs

    def __getattr__(self, name):
        return getattr(self._node, name)


# an elementwise read of an arena variable of at most this many floats that a
# later statement of the same pass overwrites is read from a snapshot copy
SNAPSHOT_MAX_FLOATS = 1 << 20


def _abs_range(km: KMatrix, buffers: BufferInfo):
    """``[lo, hi)`` of the floats an access may address, in the coordinates
    of its access expression (the tetris region's for a tetris variable)."""
    var = getattr(km, "tetris_var", None)
    if var is not None:
        return var[1], var[1] + var[2]
    size = buffers.size.get(km.id)
    return (0, size) if size is not None else None


def snapshot_reads(stmts, pairs, buffers: BufferInfo, scratch_base: int):
    """Break cross-element conflicts of an elementwise statement list that
    come from a small operand read by statement ``i`` and overwritten by a
    later statement ``j`` (a LayerNorm's row means, whose memory the squared
    deviations reuse): the operand's variable is copied to scratch first and
    ``i`` reads the copy, so ``i`` and ``j`` can share one pass.  Under the
    statement-by-statement semantics ``i`` reads the values from before the
    command, because no statement up to ``i`` writes the variable (else the
    read is left alone).  Returns ``(statements, copy plans, scratch floats)``
    or None when nothing is copied."""
    first_of = {i for i, j in pairs if i < j}
    writes = []
    for si, (kind, n) in enumerate(stmts):
        if kind in ("tmp", "load", "store") or n.kres.is_none() or n.kres.is_temp:
            continue
        writes.append((si, _region(n.kres, buffers)[0]))
    alloc = ScratchAlloc(scratch_base)
    slots = {}
    out = list(stmts)
    for si, (kind, n) in enumerate(stmts):
        if kind not in ("bin", "un", "copy") or si not in first_of:
            continue
        kargs, changed = list(n.kargs), False
        for ai, k in enumerate(kargs):
            if not isinstance(k, KMatrix) or k.is_temp or getattr(k, "scratch_offset", None) is not None:
                continue
            reg = _region(k, buffers)[0]
            span = _abs_range(k, buffers)
            if span is None or span[1] - span[0] > SNAPSHOT_MAX_FLOATS:
                continue

            def hits(w):
                return w[0] == reg[0] and w[1] < reg[2] and reg[1] < w[2]
            if any(wi <= si and hits(w) for wi, w in writes) or not any(wi > si and hits(w) for wi, w in writes):
                continue
            if split_const(k.access)[1] < span[0]:
                continue
            key = (k.id, span, getattr(k, "tetris_var", None))
            if key not in slots:
                slots[key] = alloc.take(span[1] - span[0])
            km = _scratch_km(slots[key] - span[0], k.access)
            km.shape = k.shape
            kargs[ai], changed = km, True
        if changed:
            out[si] = (kind, _Rebound(n, kargs))
    if not slots:
        return None
    plans = []
    for (bid, (lo, hi), var), off in slots.items():
        src = KMatrix(bid, Add(Val(Global()), Val(Constant(lo))), [hi - lo])
        if var is not None:
            src.tetris_var = var
        plans.append(elementwise_plan([("copy", _Stmt([src], _scratch_km(off, Val(Global()))))], hi - lo))
    return out, plans, alloc.used


# ------------------------------------------------------------------ per-command entry
def command_plans(cmd, buffers: BufferInfo, scratch_base: int, opts: PlanOptions = DEFAULT_OPTIONS):
    """Plans for one Proc command and the scratch floats they need, under
    ``opts``."""
    if isinstance(cmd, (BinaryNode, UnaryNode, ContigiousNode)):
        stmts, n, kind, cols, init = statements([cmd]), prod(cmd.shape), "global", 1, None
    elif isinstance(cmd, ElwFuse):
        stmts, n, kind, cols, init = statements(cmd.nodes), prod(cmd.init_node.shape), "global", 1, None
    elif isinstance(cmd, DotProdNode):
        stmts, n, kind, cols, init = statements([cmd]), prod(cmd.shape), "dp", cmd.shape[1], cmd
    elif isinstance(cmd, DPElwFuse):
        dp = cmd.init_node
        stmts, n, kind, cols, init = statements(cmd.nodes), prod(dp.shape), "dp", dp.shape[1], dp
    elif isinstance(cmd, ReduceNode):
        stmts, n, kind, cols, init = statements([cmd]), cmd.children_shapes[0][0], "red", 1, cmd
    elif isinstance(cmd, ReduceElwFuse):
        red = cmd.init_node
        stmts, n, kind, cols, init = statements(cmd.nodes), red.children_shapes[0][0], "red", 1, red
    else:
        raise TypeError(f"Encountered unexpected cmd: {cmd}")

    # an elementwise command is split into independent groups, each its own
    # kernel with its own ranges (same-shaped groups then share one launch)
    groups = [stmts] if init is not None else components(stmts, buffers)
    plans, end, multipass = [], scratch_base, False
    for group in groups:
        pairs = conflict_pairs(group, buffers, kind, cols)
        stmts_run, copies, snap = group, [], 0
        if pairs and init is None and not any(i == j for i, j in pairs):
            snapped = snapshot_reads(group, pairs, buffers, end)
            if snapped is not None:
                cand = conflict_pairs(snapped[0], buffers, kind, cols)
                if len(split_phases(len(group), cand)) < len(split_phases(len(group), pairs)):
                    stmts_run, copies, snap = snapped
                    pairs = cand
        if any(i == j for i, j in pairs):
            ps, need = lockstep_plans(stmts_run, n, kind, cols, init, end + snap, opts)
        else:
            ps, need = phased_plans(stmts_run, pairs, n, kind, cols, init, end + snap, opts)
        ps, need = copies + ps, need + snap
        reads, writes = stmt_regions(group, buffers) if len(groups) > 1 else (None, None)
        for p in ps + [p.narrow for p in ps if p.narrow is not None]:
            p.reads, p.writes = reads, writes
            p.scratch = (end - scratch_base, end - scratch_base + need)
        plans.extend(ps)
        multipass |= len(ps) > 1
        end += need
    return plans, end - scratch_base, multipass


class ScratchAlloc:
    """Bump allocator over a command's scratch floats (64-float aligned)."""

    def __init__(self, base=0):
        self.base = base
        self.end = base

    def take(self, nfloats):
        off = self.end
        self.end += (nfloats + 63) // 64 * 64
        return off

    @property
    def used(self):
        return self.end - self.base


class _Stmt:
    """A generated statement ``kres = kargs[0]`` (an operand gather)."""

    def __init__(self, kargs, kres):
        self.kargs = kargs
        self.kres = kres


# a DotProd operand given as a concat of matrices (nested conditions per
# element) is first gathered into a dense scratch copy when the product is
# at least this many multiply-adds
GATHER_MIN_MACS = 1 << 22


def gather_plan(karg, rows, cols, dst_off, column_major=False) -> KernelPlan:
    """Dense copy of a DotProd operand in the (_x, _y) convention of its
    kernel arg: row-major ``scratch[r * cols + c] = operand(r, c)``, or
    column-major ``scratch[c * rows + r]`` with threads along the rows."""
    sink = _scratch_km(dst_off, Global())
    if column_major:
        return elementwise_plan([("copy", _Stmt([karg], sink))], rows * cols, index_kind="dpT", n_cols=rows)
    return elementwise_plan([("copy", _Stmt([karg], sink))], rows * cols, index_kind="dp", n_cols=cols)


def _dense_scratch_operand(off, cols, rows=None):
    """The gathered copy as an operand: row-major, or column-major when
    ``rows`` is given."""
    if rows is not None:
        return _scratch_km(off, Add(Mult(Y(), Val(Constant(rows))), X()))
    return _scratch_km(off, Add(Mult(X(), Val(Constant(cols))), Y()))


def _runs_along_rows(karg) -> bool:
    """Every piece of a concat operand is contiguous along its row index
    (_x) and not along its column index (_y): a row-major gather would read
    each piece across its storage, a column-major one reads it in order."""
    leaves = [km for km in _iter_kmatrix(karg)]
    if not leaves:
        return False
    for km in leaves:
        if km.is_temp:
            return False
        core, _ = split_const(km.access)
        if vec_class(core, X).kind != AFF or vec_class(core, Y).kind == AFF:
            return False
    return True


# a DotProd epilogue reading more distinct buffer locations than this runs as
# its own elementwise pass over the stored product (the MFMA accumulator
# layout makes wide epilogue loads slow and costs registers)
EPILOGUE_MAX_LOADS = 4


def epilogue_loads(part):
    """Distinct non-temp operand locations an epilogue reads."""
    seen = set()
    for kind, n in part:
        if kind in ("tmp", "load", "store", "sum", "init"):
            continue
        for k in n.kargs:
            for km in _iter_kmatrix(k):
                if not km.is_temp:
                    seen.add((km.id, getattr(km, "scratch_offset", None), repr(km.access)))
    return len(seen)


def first_pass_plans(part, n, init_node, alloc: ScratchAlloc, opts=DEFAULT_OPTIONS):
    """Plans of the pass that runs the DotProd or Reduce of a command with
    ``part`` as its epilogue: operand gathers, then the product (or the
    reduction) with the epilogue in registers, or -- split over K / rows --
    partial results followed by an elementwise pass that combines them in
    chunk order and runs the epilogue."""
    exact = opts.exact_reduce
    if isinstance(init_node, DotProdNode):
        M, N = init_node.shape
        K = init_node.children_shapes[0][1]
        cfg = dp_config(M, N, K)
        if M <= SKINNY_M or K <= DIRECT_K:
            cfg = (cfg[0], cfg[1], 1, cfg[3])
        A, B = init_node.kargs
        if opts.dot == "bf16" and M * N * K >= opts.bf16_min_macs:
            # both operands packed to k-contiguous bf16 in scratch, then the product
            cfg = bf16_config(M, N, K)
            m_pad, n_pad, k_pad = bf16_dims(M, N, K, cfg)
            a_off = alloc.take((m_pad * k_pad + 1) // 2)
            b_off = alloc.take((n_pad * k_pad + 1) // 2)
            pre = [pack_plan(A, "A", M, K, m_pad, k_pad, a_off, (M, K)),
                   pack_plan(B, "B", N, K, n_pad, k_pad, b_off, (K, N))]
            if cfg[2] == 1 and epilogue_loads(part) <= EPILOGUE_MAX_LOADS:
                return pre + [dotprod_bf16_plan(part, init_node, a_off, b_off, cfg)]
            poff = alloc.take(cfg[2] * M * N)
            main = dotprod_bf16_plan([], init_node, a_off, b_off, cfg, partial_off=poff)
            comb = elementwise_plan([("sum", (poff, cfg[2], M * N, 0, False))] + part, M * N,
                                    index_kind="dp", n_cols=N, init_value="_value")
            return pre + [main, comb]
        pre = []
        if isinstance(A, KConcat) and M * N * K >= GATHER_MIN_MACS:
            off = alloc.take(M * K)
            by_col = _runs_along_rows(A)
            pre.append(gather_plan(A, M, K, off, by_col))
            A = _dense_scratch_operand(off, K, M if by_col else None)
        if isinstance(B, KConcat) and M * N * K >= GATHER_MIN_MACS:
            off = alloc.take(K * N)
            by_col = _runs_along_rows(B)
            pre.append(gather_plan(B, K, N, off, by_col))
            B = _dense_scratch_operand(off, N, K if by_col else None)
        quad = quad_config(M, N, K, cfg)

        def with_narrow(main, stmts, poff=None):
            if quad is not None:
                main.narrow = dotprod_plan(stmts, init_node, A, B, quad, partial_off=poff)
                assert main.narrow.args == main.args, "dp_quad alternative with other arguments"
            return main
        if cfg[2] == 1 and epilogue_loads(part) <= EPILOGUE_MAX_LOADS:
            return pre + [with_narrow(dotprod_plan(part, init_node, A, B, cfg), part)]
        poff = alloc.take(cfg[2] * M * N)
        main = with_narrow(dotprod_plan([], init_node, A, B, cfg, partial_off=poff), [], poff)
        comb = elementwise_plan([("sum", (poff, cfg[2], M * N, 0, False))] + part, M * N,
                                index_kind="dp", n_cols=N, init_value="_value")
        return pre + [main, comb]
    mode, split = reduce_mode(init_node)
    if split == 1:
        return [reduce_plan(part, init_node, exact=exact)]
    V, R = init_node.children_shapes[0]
    pad_zero = any(y >= R for y in kept_elements(R, exact))
    poff = alloc.take(split * V)
    main = reduce_plan([], init_node, partial_off=poff, exact=exact)
    op = 0 if init_node.op == ReduceOp.SUM else 1
    comb = elementwise_plan([("sum", (poff, split, V, op, pad_zero))] + part, V,
                            index_kind="red", init_value="_value")
    return [main, comb]


def split_phases(n_stmts, pairs):
    """Cut the statement list into the fewest consecutive passes such that no
    conflicting pair lies inside one pass (greedy: a pass ends right before
    the first statement that conflicts with a statement already in it).
    Returns ``[(start, end), ...]``."""
    later = {}
    for i, j in pairs:
        later.setdefault(j, []).append(i)
    phases = []
    start = 0
    for j in range(n_stmts):
        if any(i >= start for i in later.get(j, ())):
            phases.append((start, j))
            start = j
    phases.append((start, n_stmts))
    return phases


def _temp_uses(stmts):
    """Per statement index: temp ids it reads and the temp id it assigns."""
    reads, assigns = {}, {}
    for si, (kind, n) in enumerate(stmts):
        if kind == "tmp":
            continue
        rs = set()
        for k in n.kargs:
            for km in _iter_kmatrix(k):
                if km.is_temp:
                    rs.add(km.id)
        reads[si] = rs
        if not n.kres.is_none() and n.kres.is_temp:
            assigns[si] = n.kres.id
    return reads, assigns


def phased_plans(stmts, pairs, n, index_kind, n_cols, init_node, scratch_base=0, opts=DEFAULT_OPTIONS):
    """A command whose statements conflict across elements, run as several
    passes over the elements (one kernel each): the first pass is the
    DotProd/Reduce (if any) with the statements up to the first conflict in
    its epilogue, each later pass an elementwise kernel over the same element
    space.  A temp assigned in one pass and read in a later one is carried
    through a scratch array indexed by element.  Returns (plans, scratch
    floats used)."""
    phases = split_phases(len(stmts), pairs)
    reads, assigns = _temp_uses(stmts)
    decl = {node.id: (kind, node) for kind, node in stmts if kind == "tmp"}
    phase_of_stmt = {}
    for pi, (a, b) in enumerate(phases):
        for si in range(a, b):
            phase_of_stmt[si] = pi
    assigned_in = {tid: phase_of_stmt[si] for si, tid in assigns.items()}
    used_in = {}
    for si, rs in reads.items():
        for tid in rs:
            used_in.setdefault(tid, set()).add(phase_of_stmt[si])
    # scratch slot per temp that crosses a pass boundary
    alloc = ScratchAlloc(scratch_base)
    slot = {}
    for tid, pa in sorted(assigned_in.items()):
        if any(pu > pa for pu in used_in.get(tid, ())):
            slot[tid] = alloc.take(n)
    plans = []
    for pi, (a, b) in enumerate(phases):
        body = [st for st in stmts[a:b] if st[0] != "tmp"]
        touched = set()
        for si in range(a, b):
            touched |= reads.get(si, set())
            if si in assigns:
                touched.add(assigns[si])
        head = []
        for tid in sorted(touched):
            if tid in slot and assigned_in[tid] < pi:
                head.append(("load", (tid, slot[tid])))
            elif tid in decl:
                head.append(decl[tid])
        tail = [("store", (tid, slot[tid])) for tid in sorted(slot) if assigned_in[tid] == pi]
        part = head + body + tail
        if pi == 0 and init_node is not None:
            plans.extend(first_pass_plans(part, n, init_node, alloc, opts))
        else:
            kind = "global" if init_node is None else ("dp" if isinstance(init_node, DotProdNode) else "red")
            plans.append(elementwise_plan(part, n, index_kind=kind, n_cols=n_cols))
    return plans, alloc.used
