"""Write ``proc_fixtures.json``: the compiled Proc of small programs exactly
as the reference's own compile passes print it, so the front end of this
repository (tracing, graph optimisations, kernalize, fusion, in-place,
allocation and tetris packing) can be compared with the reference on whole
programs rather than on the one listing its README shows.

Runs only in the build container, where the reference is mounted read-only
at /root/reference; the committed JSON is what the tests read.  Usage:
``python tests/golden/make_proc_fixtures.py`` (each program runs in a child
interpreter of its own, since the reference keeps one global trace).

The reference imports two packages the image lacks; both are replaced in
memory only, never written to disk:

* ``colored`` (terminal colours of printed listings): a no-op whose styling
  returns the text unchanged.  Only printing uses it.
* ``toposort`` (the ordering the fusion pass walks,
  autodiff/linearize.py:10,109; unpinned version, requirements.txt:2): the
  package's published algorithm, restated -- repeatedly emit, as one set,
  every item whose dependencies have all been emitted, after dropping
  self-dependencies and adding dependencies that have no entry; a cycle
  raises.  This is also what ``ad_amd/toposort.py`` restates, so the
  fixtures pin the fusion pass's use of the layers, not the layers
  themselves.

The pass sequence is autodiff/__init__.py:44-78 without constructing a
device: dep_opt, simpl_node, repeat_opt, kernalize, linearize,
set_in_place, mem_opt, alloc, program ids.  Programs draw weights from
numpy's global generator seeded per program; the listing prints no values,
only shapes, ids, accesses and offsets.
"""
import contextlib
import io
import json
import os
import subprocess
import sys
import types

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REFERENCE = "/root/reference"
OUT = os.path.join(HERE, "proc_fixtures.json")


# ---------------------------------------------------------------- programs
# Each builder traces one program with the public API of the library module
# it is given (``autodiff`` or ``ad_amd``): nn layers, Tensor, Feeder,
# Receiver, ir_for, concat.  Weights come from numpy's global generator.

def _nn(lib):
    import importlib
    nn = importlib.import_module(lib.__name__ + ".nn")
    ln = importlib.import_module(lib.__name__ + ".nn.normalization")
    graph = importlib.import_module(lib.__name__ + ".graph")
    return nn, ln.LayerNorm, graph


def linear_example(lib):
    """examples/linear.py:16-46 (README.md:177-216 prints its listing)."""
    import numpy as np
    nn, _, graph = _nn(lib)
    net = nn.Sequential(nn.Linear(255, 255), nn.Sigmoid(), nn.Linear(255, 255))
    opt = nn.SGD(net.parameters(), lr=0.01)

    def f():
        opt.zero_grad()
        val = graph.Feeder(lambda: np.full((2, 255), 0.2, dtype=np.float32), shape=[2, 255])
        net(val).backward()
        opt.step()
    lib.ir_for(range(0, 1000), f)
    graph.Receiver(lambda *a: None, opt.parameters)


def transformer_example(lib, layers=1):
    """examples/transformer.py:13-39 with ``layers`` encoder layers."""
    import numpy as np
    nn, _, graph = _nn(lib)
    net = nn.TransformerEncoder(num_layers=layers, d_model=64, num_heads=4, ff_dim=128)
    opt = nn.SGD(net.parameters(), lr=0.01)

    def f():
        opt.zero_grad()
        val = graph.Feeder(lambda: np.full((2, 64), 0.3, dtype=np.float32), shape=[2, 64])
        net(val).backward()
        opt.step()
    lib.ir_for(range(0, 500), f)
    graph.Receiver(lambda *a: None, opt.parameters)


def transformer_two_layers(lib):
    transformer_example(lib, layers=2)


def layernorm_training(lib):
    """LayerNorm fwd+bwd with SGD on gamma/beta over [64, 128] inputs (the
    C3 configuration's program at a small size)."""
    import numpy as np
    nn, LayerNorm, graph = _nn(lib)
    x = graph.Tensor(np.random.randn(64, 128).astype(np.float32))
    dy = graph.Tensor(np.random.randn(64, 128).astype(np.float32))
    ln = LayerNorm(128)
    opt = nn.SGD(ln.parameters(), lr=0.01)

    def f():
        opt.zero_grad()
        (ln(x) * dy).backward()
        opt.step()
    lib.ir_for(range(0, 100), f)
    graph.Receiver(lambda *a: None, opt.parameters)


def encoder_mse(lib):
    """One post-norm encoder layer (d_model 32, 4 heads, ff 64) over a
    [8, 32] input Tensor, MSE-to-zero loss, SGD (the C4/C5 program at a
    small size, one sample)."""
    import numpy as np
    nn, _, graph = _nn(lib)
    net = nn.TransformerEncoder(num_layers=1, d_model=32, num_heads=4, ff_dim=64)
    opt = nn.SGD(net.parameters(), lr=0.01)
    x = graph.Tensor(np.random.randn(8, 32).astype(np.float32))

    def f():
        opt.zero_grad()
        out = net(x)
        (out * out * (1.0 / 256)).backward()
        opt.step()
    lib.ir_for(range(0, 100), f)
    graph.Receiver(lambda *a: None, opt.parameters)


def batched_encoder(lib):
    """The C4/C5 program at a small size: one post-norm encoder layer
    (d_model 32, 2 heads, ff 64) over a batch of 2 sequences of 4 rows
    stacked in one [8, 32] Tensor; per-head projections on all rows,
    attention per sample on row slices, samples concatenated along rows
    then heads concatenated (as ad_amd.workloads.transformer traces it, the
    reference having no batched matmul); MSE-to-zero loss, SGD."""
    import importlib
    import numpy as np
    nn, LayerNorm, graph = _nn(lib)
    tr = importlib.import_module(lib.__name__ + ".nn.transformer")
    d, heads, ff, seq, batch = 32, 2, 64, 4, 2
    d_v = d // heads
    wq = [nn.Linear(d, d_v, bias=False) for _ in range(heads)]
    wk = [nn.Linear(d, d_v, bias=False) for _ in range(heads)]
    wv = [nn.Linear(d, d_v, bias=False) for _ in range(heads)]
    att = [tr.Attention() for _ in range(heads)]
    wo = nn.Linear(d, d, bias=False)
    ln_att, ln_ffwd = LayerNorm(d), LayerNorm(d)
    ffwd = tr.AttentionFeedforward(d, ff)
    params = []
    for m in wq + wk + wv + [wo, ln_att, ln_ffwd, ffwd]:
        params += m.parameters()
    opt = nn.SGD(params, lr=0.01)
    x = graph.Tensor(np.random.randn(batch * seq, d).astype(np.float32))

    def f():
        opt.zero_grad()
        outs = []
        for i in range(heads):
            q, k, v = wq[i](x), wk[i](x), wv[i](x)
            per = [att[i](q[b * seq:(b + 1) * seq], k[b * seq:(b + 1) * seq], v[b * seq:(b + 1) * seq], d)
                   for b in range(batch)]
            outs.append(lib.concat(per, 0))
        y = ln_att(x + wo(lib.concat(outs, -1)))
        out = ln_ffwd(y + ffwd(y))
        (out * out * (1.0 / (batch * seq * d))).backward()
        opt.step()
    lib.ir_for(range(0, 100), f)
    graph.Receiver(lambda *a: None, opt.parameters)


def data_movement(lib):
    """Concat, transpose, slices, broadcasts and reductions outside a loop
    (the reference's concat/dotprod/layernorm tests' operations)."""
    import numpy as np
    _, _, graph = _nn(lib)
    x = graph.Tensor(np.random.randn(6, 4).astype(np.float32), requires_grad=True)
    y = graph.Tensor(np.random.randn(6, 5).astype(np.float32), requires_grad=True)
    w = graph.Tensor(np.random.randn(9, 3).astype(np.float32), requires_grad=True)
    c = lib.concat([x * 2.0, y * 3.0], 1)
    d = (c @ w).sigmoid()
    s = d.T().sum(-1)
    m = d[1:4].max(0)
    (s.sum(0) + m.sum(0)).backward()
    graph.Receiver(lambda *a: None, [c.contigious(), d, x.grad(), w.grad()])


PROGRAMS = {
    "linear_example": linear_example,
    "transformer_example": transformer_example,
    "transformer_two_layers": transformer_two_layers,
    "layernorm_training": layernorm_training,
    "encoder_mse": encoder_mse,
    "batched_encoder": batched_encoder,
    "data_movement": data_movement,
}


# ---------------------------------------------------------------- reference side
def _install_stand_ins():
    colored = types.ModuleType("colored")
    colored.stylize = lambda text, *styles: text
    colored.fore = colored.back = colored.style = lambda *a, **k: ""

    class _Blank:
        def __getattr__(self, name):
            return ""
    colored.Fore = colored.Back = colored.Style = _Blank()
    sys.modules["colored"] = colored

    tp = types.ModuleType("toposort")

    def toposort(data):
        if len(data) == 0:
            return
        data = {k: set(v) - {k} for k, v in data.items()}
        extra = set().union(*data.values()) - set(data)
        data.update({item: set() for item in extra})
        while True:
            ready = {item for item, dep in data.items() if not dep}
            if not ready:
                break
            yield ready
            data = {item: dep - ready for item, dep in data.items() if item not in ready}
        if data:
            raise ValueError("Cyclic dependencies exist among these items")
    tp.toposort = toposort
    sys.modules["toposort"] = tp


def reference_listing(name):
    """The reference's compiled Proc of program ``name`` (this process)."""
    import numpy as np
    _install_stand_ins()
    sys.path.insert(0, REFERENCE)
    import autodiff
    from autodiff.alloc import alloc
    from autodiff.context import context
    from autodiff.fusion.base import FuseBase
    from autodiff.graph import Node
    from autodiff.kernalize.kernalize import kernalize
    from autodiff.linearize import linearize
    from autodiff.opt import dep_opt, mem_opt, repeat_opt, set_in_place
    from autodiff.opt.simplify import simpl_node
    np.random.seed(0)
    sink = io.StringIO()
    with contextlib.redirect_stdout(sink):
        PROGRAMS[name](autodiff)
        context.prep_exec()
        dep_opt(context)
        simpl_node(context)
        repeat_opt(context)
        kernalize(context)
        proc = linearize(context.main_proc())
        proc = set_in_place(proc)
        proc = mem_opt(proc)
        alloc(proc)

        def assign_program_id(n, _):
            if isinstance(n, (Node, FuseBase)):
                n.program_id = context.get_prog_id()
            return n
        proc.walk(assign_program_id, step_fused=False, step_proc=True)
    return str(proc), [line for line in sink.getvalue().splitlines() if line.startswith("ALLOC DEBUG: Using")]


# ---------------------------------------------------------------- this repository
def our_listing(name):
    import numpy as np
    sys.path.insert(0, ROOT)
    import ad_amd
    ad_amd.reset()
    np.random.seed(0)
    PROGRAMS[name](ad_amd)
    sink = io.StringIO()
    with contextlib.redirect_stdout(sink):
        proc = ad_amd.compile_proc()
    return str(proc)


def main():
    if len(sys.argv) == 3 and sys.argv[1] == "--one":
        text, alloc_lines = reference_listing(sys.argv[2])
        print(json.dumps({"proc": text, "alloc": alloc_lines}))
        return
    if not os.path.isdir(os.path.join(REFERENCE, "autodiff")):
        raise SystemExit(f"the reference is not mounted at {REFERENCE}")
    out = {}
    for name in PROGRAMS:
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--one", name], capture_output=True,
                           text=True, cwd="/tmp", timeout=1200)
        if r.returncode != 0:
            raise SystemExit(f"{name}: reference run failed\n{r.stderr[-3000:]}")
        out[name] = json.loads(r.stdout.strip().splitlines()[-1])
        print(f"{name}: {len(out[name]['proc'].splitlines())} lines; {out[name]['alloc']}", flush=True)
    with open(OUT, "w") as fh:
        json.dump(out, fh, indent=1, sort_keys=True)
        fh.write("\n")
    print("wrote", OUT)


if __name__ == "__main__":
    main()
