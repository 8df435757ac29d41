#!/usr/bin/env python3
"""Benchmark of the procedural-IR execution path on one MI355X.

``python bench.py --gpus 1 --steps K --warmup W`` prints ONE JSON line:

* ``value``: training steps/s of the 4-layer transformer encoder
  (d_model 1024, 16 heads, FFN 4096, seq 512, batch 8, fp32, MSE-to-zero
  loss, fwd + bwd + SGD lr 0.01).  The loop body is compiled once by the
  full compile pipeline and executed by the HIP backend as one captured HIP
  graph per step; K steps are timed after W warm-up steps, with the input
  resident in device memory.
* ``roofline``: the fused DotProd+Elw kernel ``sigmoid(A@B + bias)`` on
  [4096,4096] x [4096,4096] fp32 (2*4096^3 flop per launch), timed with HIP
  events on the backend's stream, against the fp32 MFMA peak.
* ``microbench``: the same figures for the Reduce+Elw (``sum(-1)*c`` over
  [8192,4096]) and ElwFuse (6 ops over 64M floats) commands, HBM-bound, with
  inputs rotated across copies larger than the 256 MB last-level cache.
* ``other_configs``: C1 (the MLP of examples/linear.py, a Feeder upload per
  step), C3 (LayerNorm fwd+bwd at [16384,1024], GB/s over the Proc's
  per-command bytes and over the 5-pass HBM floor) and C4 (1-layer
  transformer) at full size, graph-replayed; and the bf16 DotProd option
  (beyond the reference): the 4096^3 DotProd+Elw and the C5 step with
  DotProd operands rounded to bf16.
* ``value_with_feeder``: the same step with X fed from the host every step
  (a Feeder; its PCIe upload overlaps the previous step).
* ``cpu_baseline``: the CPU restatement of the reference OpenCL backend
  (``oracle``, one OpenMP iteration per work-item, sequential k-loops, the
  work-group tree) running real training steps of the same Proc on this
  host's cores (2 timed steps after an untimed one by default), with the CPU
  model; ``cpu_other_configs``: C1, C3, C4 and the three single-command
  benchmarks on the same oracle.
* ``other_configs.published_config``: examples/transformer.py (the
  configuration README.md:34-45 times) replayed for 500 and 3000 steps.

Only one GPU is used: ``--gpus`` above 1 exits with a message.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "transformer train steps/s; fused DotProd TFLOP/s + ElwFuse GB/s vs MI355X peak"
PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
PEAK_BF16_MFMA_TFLOPS = 2500.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def measured_traffic(kernel):
    """HBM bytes per dispatch of ``kernel`` from the committed counter
    summary (two rocprofv3 --pmc passes, calibrated on the ElwFuse kernel),
    or None when that summary was taken of another build of the kernel."""
    path = os.path.join(ROOT, "profiles", "micro_hbm_traffic_counters.txt")
    if not os.path.exists(path):
        return None
    with open(path) as fh:
        for line in fh:
            parts = line.split()
            if len(parts) == 3 and parts[0] == "traffic" and parts[1] == kernel:
                return int(parts[2])
    return None


def _commands(proc):
    from ad_amd.fusion import FuseBase
    from ad_amd.node import Node
    return [c for c in proc.procedure if isinstance(c, (Node, FuseBase)) and hasattr(c, "program_id")
            and not type(c).__name__ in ("Feeder", "Receiver", "ForNode")]


def _time_launches(dev, cmds, reps, warmup=2):
    """Average device time per launch of ``cmds`` launched round-robin."""
    for i in range(warmup):
        dev.launch(cmds[i % len(cmds)])
    dev.ctx.sync()
    dev.ctx.event(10)
    for i in range(reps):
        dev.launch(cmds[i % len(cmds)])
    dev.ctx.event(11)
    dev.ctx.sync()
    return dev.ctx.elapsed_ms(10, 11) / reps


def vendor_gemm(reps):
    """The 4096^3 fp32 product on the vendor BLAS (torch.matmul, reduced
    precision paths off), timed with torch's events: a reference point for
    the DotProd+Elw kernel, not part of the backend.  Runs in a child
    interpreter: a process that has loaded libadhip.so has the system HIP
    runtime mapped, and torch's own runtime then finds no device."""
    import subprocess
    code = r"""
import json, torch
torch.backends.cuda.matmul.allow_tf32 = False
torch.backends.cuda.matmul.allow_fp16_reduced_precision_reduction = False
n, reps = 4096, %d
g = torch.Generator(device="cuda").manual_seed(0)
a = torch.randn(n, n, device="cuda", generator=g)
b = torch.randn(n, n, device="cuda", generator=g)
for _ in range(3):
    c = a @ b
torch.cuda.synchronize()
s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
s.record()
for _ in range(reps):
    c = a @ b
e.record(); e.synchronize()
ms = s.elapsed_time(e) / reps
print(json.dumps({"vendor_gemm_4096": {"library": "torch.matmul fp32 (hipBLASLt/rocBLAS), TF32 off", "ms": round(ms, 4),
                                        "tflops": round(2 * n ** 3 / ms / 1e9, 2)}}))
""" % reps
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=600)
    if out.returncode != 0:
        raise RuntimeError(out.stderr[-2000:])
    return json.loads(out.stdout.strip().splitlines()[-1])


def micro_dotprod(reps, dot="fp32"):
    """The 4096^3 DotProd+Elw command; with ``dot="bf16"`` its time includes
    the two operand-packing kernels."""
    import ad_amd as ad
    from ad_amd import workloads
    from ad_amd.device.hip import HIPDevice
    ad.reset()
    workloads.dotprod_elw(4096, 4096, 4096)
    proc = ad.compile_proc()
    dev = HIPDevice(dot_precision=dot)
    dev.prepare(proc)
    cmds = _commands(proc)
    assert len(cmds) == 1, [type(c).__name__ for c in cmds]
    plan = [p for p in dev.kernels[cmds[0].program_id] if p.family == "dotprod"]
    assert len(plan) == 1
    ms = _time_launches(dev, cmds, reps)
    flops = 2 * 4096 ** 3
    dev.close()
    return {"kernel": plan[0].name, "ms": ms, "flops": flops, "tflops": flops / ms / 1e9}


def micro_reduce(reps, copies=3):
    import numpy as np
    import ad_amd as ad
    from ad_amd.device.hip import HIPDevice
    from ad_amd.graph import Receiver, Tensor
    ad.reset()
    V, R = 8192, 4096
    rng = np.random.default_rng(1)
    for _ in range(copies):
        r = Tensor(rng.standard_normal((V, R), dtype=np.float32)).sum(-1) * 0.5
        Receiver(lambda v: None, [r])
    proc = ad.compile_proc()
    dev = HIPDevice()
    dev.prepare(proc)
    cmds = _commands(proc)
    assert len(cmds) == copies
    name = dev.kernels[cmds[0].program_id][0].name
    ms = _time_launches(dev, cmds, reps)
    nbytes = 4 * V * R + 4 * V
    dev.close()
    return {"kernel": name, "ms": ms, "bytes": nbytes, "gbs": nbytes / ms / 1e6}


def micro_elw(reps, copies=2, expr=None, stream=True):
    """ElwFuse over 64 M floats (two copies of slightly different lengths);
    ``expr`` replaces the default 6-op chain; ``stream=False`` keeps the
    loads and stores cached (the plain copy that calibrates the counters)."""
    import numpy as np
    import ad_amd as ad
    from ad_amd.device.hip import HIPDevice
    from ad_amd.graph import Receiver, Tensor
    ad.reset()
    n = 64 << 20
    rng = np.random.default_rng(1)
    # copies differ in length by 64 floats: ElwFuse would merge equal-length
    # independent chains into one command
    for i in range(copies):
        x = Tensor(rng.standard_normal((n + 64 * i,), dtype=np.float32))
        r = expr(x) if expr is not None else ((x * 0.5 + 1.0).exp2() + 1.0).recip() * 3.0
        Receiver(lambda v: None, [r])
    proc = ad.compile_proc()
    dev = HIPDevice() if stream else HIPDevice(stream_min_bytes=None)
    dev.prepare(proc)
    cmds = _commands(proc)
    assert len(cmds) == copies, [type(c).__name__ for c in cmds]
    name = dev.kernels[cmds[0].program_id][0].name
    ms = _time_launches(dev, cmds, reps)
    nbytes = 2 * 4 * (n + 32 * (copies - 1))      # mean over the copies
    dev.close()
    return {"kernel": name, "ms": ms, "bytes": nbytes, "gbs": nbytes / ms / 1e6}


def transformer_steps(config, steps, warmup, eager=False, lanes=1, dot="fp32", arena="packed", feeder=False):
    import ad_amd as ad
    from ad_amd import workloads
    from ad_amd.device.hip import HIPDevice
    layers, d, h, f, s, b = workloads.TRANSFORMER_CONFIGS[config]
    ad.reset()
    t0 = time.perf_counter()
    workloads.transformer(layers=layers, d_model=d, heads=h, ff=f, seq=s, batch=b, steps=1,
                          receive=False, feeder=feeder)
    proc = ad.compile_proc()
    t1 = time.perf_counter()
    step_flops = workloads.dotprod_flops(proc)
    log(f"{config}: traced + compiled in {t1 - t0:.1f} s; {step_flops / 1e12:.3f} TFLOP of DotProd per step")
    dev = HIPDevice(use_graphs=not eager, lanes=lanes, dot_precision=dot, arena=arena)
    dev.prepare(proc)
    t2 = time.perf_counter()
    log(f"{config}: device init + JIT in {t2 - t1:.1f} s; {dev.stats}")
    loop = dev.loops(proc)
    assert len(loop) == 1
    loop = loop[0]
    dev.replay(loop, max(1, warmup))           # first call captures the graph
    dev.ctx.sync()
    log(f"{config}: warm-up done")
    t3 = time.perf_counter()
    dev.ctx.event(0)
    dev.replay(loop, steps)
    dev.ctx.event(1)
    dev.ctx.sync()
    t4 = time.perf_counter()
    ev_ms = dev.ctx.elapsed_ms(0, 1)
    launches = dev.stats["launches_per_iter"]
    dev.close()
    return {"wall_s": t4 - t3, "event_ms": ev_ms, "step_flops": step_flops,
            "compile_s": t1 - t0, "init_s": t2 - t1, "launches_per_step": launches, "proc": proc}


def loop_rate(build, steps, warmup):
    """Per-iteration device time of the one ``ir_for`` a builder traces,
    replayed as a HIP graph (a Feeder's host function and upload included)."""
    import ad_amd as ad
    from ad_amd.device.hip import HIPDevice
    ad.reset()
    build()
    proc = ad.compile_proc()
    dev = HIPDevice()
    dev.prepare(proc)
    loop = dev.loops(proc)
    assert len(loop) == 1
    loop = loop[0]
    dev.replay(loop, max(1, warmup))
    dev.ctx.sync()
    t0 = time.perf_counter()
    dev.ctx.event(0)
    dev.replay(loop, steps)
    dev.ctx.event(1)
    dev.ctx.sync()
    wall = time.perf_counter() - t0
    ev_ms = dev.ctx.elapsed_ms(0, 1)
    launches = dev.stats["launches_per_iter"]
    dev.close()
    return {"ms": max(wall * 1e3, ev_ms) / steps, "launches": launches}


# bytes of the 5-pass floor of one LayerNorm fwd+bwd iteration at [16384, 1024]:
# five passes over a 64 MiB matrix
C3_FLOOR_BYTES = 5 * 4 * 16384 * 1024
# algorithmic bytes of the iteration's Proc, per command (each distinct operand
# at its true size): row mean (x in, mean out); beta grad (dy in, beta in+out);
# x - mean and its square (x, mean in; two matrices out); 1/sqrt(var + eps)
# (squares in, rstd out); dy * xhat (xc, rstd, dy in; one matrix out); gamma
# grad (that matrix in, gamma in+out): ten 64 MiB matrix passes, four 64 KiB
# row vectors, four 4 KiB parameter vectors
C3_PROC_BYTES = 10 * 4 * 16384 * 1024 + 4 * 4 * 16384 + 4 * 4 * 1024


def other_configs():
    """C1 (MLP, Feeder per step), C3 (LayerNorm fwd+bwd) and C4 (1-layer
    transformer) at their full sizes."""
    from ad_amd import workloads
    out = {}
    c1 = loop_rate(lambda: workloads.mlp(steps=1, receive=False), 1000, 50)
    out["c1_mlp"] = {"workload": "Linear(255,255)-Sigmoid-Linear(255,255), [2,255] Feeder per step, SGD",
                     "us_per_step": round(c1["ms"] * 1e3, 2), "steps_per_s": round(1e3 / c1["ms"], 1),
                     "launches_per_step": c1["launches"]}
    log(f"c1: {c1['ms'] * 1e3:.1f} us/step, {c1['launches']} launches/step")
    c3 = loop_rate(lambda: workloads.layernorm_train(rows=16384, cols=1024, steps=1, receive=False), 50, 3)
    gbs = C3_FLOOR_BYTES / c3["ms"] / 1e6
    pgbs = C3_PROC_BYTES / c3["ms"] / 1e6
    out["c3_layernorm"] = {"workload": "LayerNorm fwd+bwd [16384,1024] + SGD on gamma/beta",
                           "ms_per_iter": round(c3["ms"], 4),
                           "proc_bytes": C3_PROC_BYTES, "proc_gbs": round(pgbs, 1),
                           "frac": round(pgbs / PEAK_HBM_GBS, 4),
                           "floor_bytes": C3_FLOOR_BYTES, "floor_gbs": round(gbs, 1),
                           "launches_per_iter": c3["launches"]}
    log(f"c3: {c3['ms'] * 1e3:.1f} us/iter, {pgbs:.0f} GB/s over the Proc's bytes, "
        f"{gbs:.0f} GB/s over the 5-pass floor")
    c4 = transformer_steps("c4", 20, 3)
    ms = c4["event_ms"] / 20
    out["c4_transformer"] = {"workload": "1-layer encoder d_model 512, 8 heads, FFN 2048, seq 256, batch 16",
                             "steps_per_s": round(1e3 / ms, 2), "ms_per_step": round(ms, 3),
                             "step_dotprod_tflops": round(c4["step_flops"] / (ms * 1e9), 2),
                             "launches_per_step": c4["launches_per_step"]}
    log(f"c4: {ms:.2f} ms/step, {1e3 / ms:.1f} steps/s")
    dp = micro_dotprod(10, dot="bf16")
    c5 = transformer_steps("c5", 20, 3, dot="bf16")
    ms = c5["event_ms"] / 20
    out["bf16_dotprod"] = {
        "note": "option beyond the reference (fp32): DotProd operands rounded to bf16, fp32 sums",
        "dotprod_elw_4096_tflops": round(dp["tflops"], 1),
        "dotprod_elw_4096_frac_of_bf16_peak": round(dp["tflops"] / PEAK_BF16_MFMA_TFLOPS, 4),
        "c5_steps_per_s": round(1e3 / ms, 2), "c5_ms_per_step": round(ms, 3)}
    log(f"bf16 DotProds: 4096^3 {dp['tflops']:.1f} TFLOP/s (packing included); c5 {1e3 / ms:.1f} steps/s")
    unpacked = {"note": "option beyond the reference: every tetris variable in storage of its own, "
                        "launches ordered by data flow only; fp32"}
    for config in ("c4", "c5"):
        r = transformer_steps(config, 20, 3, arena="unpacked")
        ms = r["event_ms"] / 20
        unpacked[f"{config}_steps_per_s"] = round(1e3 / ms, 2)
        unpacked[f"{config}_launches_per_step"] = r["launches_per_step"]
        log(f"unpacked arena: {config} {1e3 / ms:.1f} steps/s, {r['launches_per_step']} launches/step")
    r = transformer_steps("c5", 20, 3, dot="bf16", arena="unpacked")
    ms = r["event_ms"] / 20
    unpacked["c5_bf16_steps_per_s"] = round(1e3 / ms, 2)
    log(f"unpacked arena and bf16 DotProds: c5 {1e3 / ms:.1f} steps/s")
    out["unpacked_arena"] = unpacked
    out["published_config"] = published_config()
    return out


def host_cpu():
    """CPU model and the OpenMP threads the oracle runs with (every core of
    this process's affinity, or OMP_NUM_THREADS if lower)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    cores = len(os.sched_getaffinity(0))
    threads = min(int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or cores, cores)
    return model, threads


def _oracle(proc):
    """The CPU restatement of the OpenCL backend with its work-item kernels
    (one OpenMP iteration per work-item, sequential k-loops, the work-group
    tree), initialised on ``proc``; returns it and the seconds its kernels
    took to compile."""
    from oracle import OracleDevice
    dev = OracleDevice(lockstep=False)
    t0 = time.perf_counter()
    dev._run_proc(proc, dev.init, init=True)
    dev._finish_init()
    return dev, time.perf_counter() - t0


def oracle_loop(proc, iterations, warmup=1):
    """Seconds per iteration of the one ``ir_for`` body of ``proc`` on the
    oracle (``warmup`` untimed iterations first)."""
    from ad_amd.graph import ForNode
    dev, jit_s = _oracle(proc)
    loops = [c for c in proc.procedure if isinstance(c, ForNode)]
    assert len(loops) == 1
    inner = loops[0].get_proc()
    for _ in range(warmup):
        dev._run_proc(inner, dev.run)
    t0 = time.perf_counter()
    for _ in range(iterations):
        dev._run_proc(inner, dev.run)
    return (time.perf_counter() - t0) / iterations, jit_s


def oracle_command(build, reps):
    """Seconds per run of the single compute command a builder traces, on
    the oracle (one untimed run first)."""
    import ad_amd as ad
    ad.reset()
    build()
    proc = ad.compile_proc()
    dev, _ = _oracle(proc)
    cmds = _commands(proc)
    assert len(cmds) == 1, [type(c).__name__ for c in cmds]
    fn = dev.funcs[cmds[0].program_id]
    fn()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    return (time.perf_counter() - t0) / reps


def cpu_baseline(proc, config, step_flops, steps=2):
    """``steps`` real training steps of ``config`` (the Proc the GPU ran) on
    the oracle's work-item kernels, after one untimed step: the reference's
    OpenCL execution path restated for the host's cores."""
    model, threads = host_cpu()
    sec, jit_s = oracle_loop(proc, steps, warmup=1)
    log(f"cpu baseline: {config} {sec:.2f} s/step on the oracle ({threads} threads, {model}); "
        f"kernels compiled in {jit_s:.1f} s")
    return {"value": round(1.0 / sec, 6), "unit": "steps/s", "cores": threads, "kind": "port",
            "cpu_model": model,
            "sample": (f"{steps} {config} training steps (after 1 untimed step) of the oracle's work-item "
                       f"kernels, the CPU restatement of the reference OpenCL backend, on {threads} "
                       f"OpenMP threads of {model}: {sec:.2f} s/step, "
                       f"{step_flops / sec / 1e9:.1f} GFLOP/s of DotProd"),
            "s_per_step": round(sec, 3)}


def cpu_other_configs():
    """The other configurations and the single-command benchmarks on the
    oracle: C1 (1000 steps), C3 (5 iterations), C4 (2 steps), the 4096^3
    DotProd+Elw (1 run), the [8192,4096] Reduce+Elw (10 runs) and the 64 M
    ElwFuse (5 runs), each after an untimed run."""
    import ad_amd as ad
    from ad_amd import workloads
    model, threads = host_cpu()
    out = {"cpu_model": model, "cores": threads}
    ad.reset()
    workloads.mlp(steps=1, receive=False)
    sec, _ = oracle_loop(ad.compile_proc(), 1000, warmup=10)
    out["c1_mlp"] = {"us_per_step": round(sec * 1e6, 1), "steps_per_s": round(1 / sec, 1)}
    ad.reset()
    workloads.layernorm_train(rows=16384, cols=1024, steps=1, receive=False)
    sec, _ = oracle_loop(ad.compile_proc(), 5)
    out["c3_layernorm"] = {"ms_per_iter": round(sec * 1e3, 2), "proc_gbs": round(C3_PROC_BYTES / sec / 1e9, 1)}
    layers, d, h, f, s, b = workloads.TRANSFORMER_CONFIGS["c4"]
    ad.reset()
    workloads.transformer(layers=layers, d_model=d, heads=h, ff=f, seq=s, batch=b, steps=1, receive=False)
    sec, _ = oracle_loop(ad.compile_proc(), 2)
    out["c4_transformer"] = {"steps_per_s": round(1 / sec, 3), "s_per_step": round(sec, 3)}
    sec = oracle_command(lambda: workloads.dotprod_elw(4096, 4096, 4096), 1)
    out["dotprod_elw_4096"] = {"s": round(sec, 3), "tflops": round(2 * 4096 ** 3 / sec / 1e12, 4)}
    sec = oracle_command(lambda: workloads.reduce_elw(8192, 4096, 0.5), 10)
    out["reduce_elw_8192x4096"] = {"ms": round(sec * 1e3, 2), "gbs": round((4 * 8192 * 4096 + 4 * 8192) / sec / 1e9, 1)}
    sec = oracle_command(lambda: workloads.elw_chain(64 << 20), 5)
    out["elw_fuse_64m"] = {"ms": round(sec * 1e3, 2), "gbs": round(2 * 4 * (64 << 20) / sec / 1e9, 1)}
    log(f"cpu: c1 {out['c1_mlp']['us_per_step']} us/step, c3 {out['c3_layernorm']['ms_per_iter']} ms/iter, "
        f"c4 {out['c4_transformer']['s_per_step']} s/step, dotprod {out['dotprod_elw_4096']['tflops']} TFLOP/s, "
        f"reduce {out['reduce_elw_8192x4096']['gbs']} GB/s, elw {out['elw_fuse_64m']['gbs']} GB/s")
    return out


def published_config():
    """examples/transformer.py (1 layer, d_model 64, 4 heads, ff 128, [2,64]
    Feeder per step) replayed for 500 and 3000 steps: README.md:34-36 times
    this configuration at 1.32 s (1 layer, CUDA backend on an A100; the step
    count is not stated; the script runs 500, the screenshot's torch run
    3000)."""
    import ad_amd as ad
    from ad_amd import workloads
    from ad_amd.device.hip import HIPDevice
    ad.reset()
    workloads.published_transformer(layers=1, steps=1)
    proc = ad.compile_proc()
    dev = HIPDevice()
    dev.prepare(proc)
    loop = dev.loops(proc)[0]
    dev.replay(loop, 32)
    dev.ctx.sync()
    out = {"workload": "examples/transformer.py: TransformerEncoder(1 layer, d_model 64, 4 heads, ff 128), "
                       "[2,64] Feeder of 0.3 per step, SGD lr 0.01",
           "readme_seconds": 1.32, "launches_per_step": dev.stats["launches_per_iter"]}
    for steps in (500, 3000):
        t0 = time.perf_counter()
        dev.replay(loop, steps)
        dev.ctx.sync()
        out[f"seconds_{steps}_steps"] = round(time.perf_counter() - t0, 4)
    dev.close()
    log(f"published config: 500 steps {out['seconds_500_steps']} s, 3000 steps {out['seconds_3000_steps']} s "
        f"(README: 1.32 s)")
    return out


def _merged_floats(ranges):
    """Floats covered by a list of (buffer, lo, hi) ranges, overlaps once."""
    by = {}
    for buf, lo, hi in ranges:
        by.setdefault(repr(buf), []).append((lo, hi))
    total = 0
    for segs in by.values():
        segs.sort()
        lo0, hi0 = segs[0]
        for lo, hi in segs[1:]:
            if lo > hi0:
                total += hi0 - lo0
                lo0, hi0 = lo, hi
            else:
                hi0 = max(hi0, hi)
        total += hi0 - lo0
    return total


def probe(config, iters, out_path):
    """Replay ``iters`` iterations of a configuration's loop body launch by
    launch (no graph: kernel tracers and counter passes see every dispatch)
    and write its launch table: per launch of one iteration, in dispatch
    order, the kernel, its instances and the floats of the ranges it may
    read and write (a command's ranges for each of its launches; scratch
    separate)."""
    import ad_amd as ad
    from ad_amd import workloads
    from ad_amd.device.hip import HIPDevice
    ad.reset()
    if config == "c1":
        workloads.mlp(steps=1, receive=False)
    elif config == "c3":
        workloads.layernorm_train(rows=16384, cols=1024, steps=1, receive=False)
    else:
        layers, d, h, f, s, b = workloads.TRANSFORMER_CONFIGS[config]
        workloads.transformer(layers=layers, d_model=d, heads=h, ff=f, seq=s, batch=b, steps=1, receive=False)
    proc = ad.compile_proc()
    dev = HIPDevice(use_graphs=False)
    dev.prepare(proc)
    loop = dev.loops(proc)[0]
    table = []
    for stretch in dev.stretch_graphs[loop.get_proc().id]:
        for name, count, _, reads, writes, flops in stretch:
            table.append({"kernel": name, "instances": count, "flops": flops,
                          "read_floats": _merged_floats([r for r in reads if r[0] != "scratch"]),
                          "write_floats": _merged_floats([w for w in writes if w[0] != "scratch"]),
                          "scratch_floats": _merged_floats([r for r in reads + writes if r[0] == "scratch"])})
    if out_path:
        with open(out_path, "w") as fh:
            json.dump(table, fh)
    log(f"probe {config}: {len(table)} launches per iteration, replaying {iters}")
    for _ in range(iters):
        dev.replay(loop, 1)
        dev.ctx.sync()
    dev.close()


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c5", choices=["c4", "c5"])
    ap.add_argument("--micro-reps", type=int, default=20)
    ap.add_argument("--cpu-steps", type=int, default=2, help="timed training steps of the CPU baseline")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-micro", action="store_true", help="skip the single-command benchmarks")
    ap.add_argument("--no-configs", action="store_true", help="skip the C1/C3/C4 measurements")
    ap.add_argument("--lanes", type=int, default=1,
                    help="streams for independent launch groups in eager runs (graphs use one)")
    ap.add_argument("--micro-only", action="store_true",
                    help="run only the single-command benchmarks (for counter passes)")
    ap.add_argument("--arena", choices=["packed", "unpacked"], default="packed",
                    help="packed: tetris variables at the reference's packed offsets (default); "
                         "unpacked: each in storage of its own")
    ap.add_argument("--eager", action="store_true",
                    help="launch the step's kernels one by one instead of replaying a HIP graph "
                         "(for kernel-trace profilers)")
    ap.add_argument("--probe", choices=["c1", "c3", "c4", "c5"],
                    help="only replay this configuration's loop body launch by launch (for kernel traces and "
                         "counter passes) and write its launch table to --probe-out")
    ap.add_argument("--probe-iters", type=int, default=3)
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="only time the 4096^3 fp32 product on the vendor BLAS through torch (a reference point)")
    ap.add_argument("--probe-out", default=None)
    args = ap.parse_args()
    if args.vendor_gemm:
        print(json.dumps(vendor_gemm(args.micro_reps)), flush=True)
        return
    if args.probe:
        probe(args.probe, args.probe_iters, args.probe_out)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}): "
              "the backend executes one Proc on one device; multi-GPU sharding is not built",
              file=sys.stderr)
        sys.exit(2)

    micro = {}
    if not args.no_micro:
        dp = micro_dotprod(args.micro_reps)
        log(f"dotprod_elw 4096^3: {dp['ms']:.3f} ms, {dp['tflops']:.1f} TFLOP/s ({dp['kernel']})")
        red = micro_reduce(args.micro_reps * 3)
        log(f"reduce_elw [8192,4096]: {red['ms'] * 1e3:.1f} us, {red['gbs']:.0f} GB/s ({red['kernel']})")
        elw = micro_elw(args.micro_reps * 2)
        log(f"elw_fuse 64M: {elw['ms'] * 1e3:.1f} us, {elw['gbs']:.0f} GB/s ({elw['kernel']})")
        cp = micro_elw(args.micro_reps * 2, expr=lambda x: x + 0.5, stream=False)
        log(f"plain copy 64M (cached loads and stores): {cp['ms'] * 1e3:.1f} us, {cp['gbs']:.0f} GB/s ({cp['kernel']})")
        micro = {
            "dotprod_elw": {"kernel": dp["kernel"], "us": round(dp["ms"] * 1e3, 2),
                            "tflops": round(dp["tflops"], 2),
                            "frac": round(dp["tflops"] / PEAK_FP32_MFMA_TFLOPS, 4)},
            "reduce_elw": {"kernel": red["kernel"], "us": round(red["ms"] * 1e3, 2),
                           "gbs": round(red["gbs"], 1), "frac": round(red["gbs"] / PEAK_HBM_GBS, 4)},
            "elw_fuse": {"kernel": elw["kernel"], "us": round(elw["ms"] * 1e3, 2),
                         "gbs": round(elw["gbs"], 1), "frac": round(elw["gbs"] / PEAK_HBM_GBS, 4)},
            "plain_copy": {"kernel": cp["kernel"], "us": round(cp["ms"] * 1e3, 2),
                           "gbs": round(cp["gbs"], 1), "frac": round(cp["gbs"] / PEAK_HBM_GBS, 4),
                           "note": "x + 0.5 over 64 M floats with cached loads and stores; calibrates "
                                   "the traffic counters"},
        }

    if args.micro_only:
        print(json.dumps({"microbench": micro or None}), flush=True)
        return
    tr = transformer_steps(args.config, args.steps, args.warmup, eager=args.eager, lanes=args.lanes,
                           arena=args.arena)
    value = args.steps / tr["wall_s"]
    ms_per_step = tr["wall_s"] * 1e3 / args.steps
    log(f"{args.config}: {ms_per_step:.2f} ms/step wall, {tr['event_ms'] / args.steps:.2f} ms/step "
        f"events, {value:.3f} steps/s, {tr['launches_per_step']} launches/step")
    # the same step with X fed from the host every step (a Feeder: the
    # [B*S, d_model] input crosses PCIe on a transfer stream while the
    # previous step computes), timed the same way
    fd = transformer_steps(args.config, args.steps, args.warmup, eager=args.eager, lanes=args.lanes,
                           arena=args.arena, feeder=True)
    fd.pop("proc")
    feeder_value = args.steps / fd["wall_s"]
    log(f"{args.config} with a Feeder per step: {fd['wall_s'] * 1e3 / args.steps:.2f} ms/step wall, "
        f"{feeder_value:.3f} steps/s")

    others = None if args.no_configs else other_configs()

    cpu = cpu_others = None
    if not args.no_cpu:
        cpu = cpu_baseline(tr["proc"], args.config, tr["step_flops"], args.cpu_steps)
        cpu_others = None if args.no_configs else cpu_other_configs()
    tr.pop("proc")

    layers, d, h, f, s, b = __import__("ad_amd.workloads", fromlist=["x"]).TRANSFORMER_CONFIGS[args.config]
    roofline = None
    if micro:
        dp = micro["dotprod_elw"]
        roofline = {"bound": "mfma", "achieved": dp["tflops"], "peak": PEAK_FP32_MFMA_TFLOPS,
                    "unit": "TFLOP/s", "frac": dp["frac"], "traffic": measured_traffic(dp["kernel"]),
                    "kernel": dp["kernel"],
                    "workload": "DotProd+Elw sigmoid(A@B+bias), [4096,4096]x[4096,4096] fp32, "
                                "2*4096^3 flop per launch"}
    out = {
        "metric": METRIC, "value": round(value, 4), "unit": "steps/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"{args.config}: {layers}-layer transformer encoder fwd+bwd+SGD, "
                               f"d_model {d}, {h} heads, FFN {f} ReLU, seq {s}, batch {b}, fp32, "
                               + ("eager launches" if args.eager else "one HIP-graph replay per step")
                               + (", unpacked arena" if args.arena == "unpacked" else ""),
                   "layers": layers, "d_model": d, "heads": h, "ffn": f, "seq_len": s, "batch": b,
                   "parallelism": "none (1 GPU)"},
        "value_with_feeder": {"value": round(feeder_value, 4), "unit": "steps/s",
                              "ms_per_step": round(fd["wall_s"] * 1e3 / args.steps, 3),
                              "note": "the same step with X fed from the host each step by a Feeder "
                                      "(PCIe upload overlapped with the previous step)"},
        "step_dotprod_tflops": round(tr["step_flops"] / (ms_per_step * 1e9), 2),
        "launches_per_step": tr["launches_per_step"],
        "roofline": roofline,
        "cpu_baseline": cpu,
        "cpu_other_configs": cpu_others,
        "microbench": micro or None,
        "other_configs": others,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
