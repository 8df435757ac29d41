"""Which float4 accesses bypass the caches (``HIPDevice._mark_streams``),
on the CPU: a read of a range no other command reads (and no later loop
iteration reads again), and a write of a range no command reads; ranges
below the size limit never."""
import numpy as np

import ad_amd as ad
from ad_amd.alloc import AllocEntry
from ad_amd.device.hip import codegen
from ad_amd.device.hip.device import HIPDevice
from ad_amd.graph import Receiver, Tensor


def _marks(min_bytes=1024):
    proc = ad.compile_proc()
    info = codegen.BufferInfo()

    def note(c, _):
        if isinstance(c, AllocEntry):
            info.size[c.id] = c.size
        return c
    proc.walk(note, step_fused=False, step_proc=True)
    dev = HIPDevice.__new__(HIPDevice)
    dev.stream_min_bytes = min_bytes
    dev._mark_streams(proc, info)
    reads, writes = set(), set()

    def visit(c, _):
        for n in getattr(c, "nodes", [c]):
            for k in getattr(n, "kargs", []):
                for km in codegen.iter_kmatrix(k):
                    if getattr(km, "stream", False):
                        reads.add(km.id)
            kres = getattr(n, "kres", None)
            if kres is not None and getattr(kres, "stream", False):
                writes.add(kres.id)
        return c
    proc.walk(visit, step_fused=False, step_proc=True)
    return reads, writes


def test_single_reader_is_streamed_and_shared_reads_are_not():
    a = Tensor(np.zeros((64, 64), np.float32))
    b = Tensor(np.zeros((64, 64), np.float32))
    Receiver(lambda *v: None, [a.sum(-1) * 0.5, b.sum(-1) * 0.5, b.max(-1) * 1.0])
    reads, _ = _marks()
    assert a.id in reads and b.id not in reads


def test_small_ranges_are_never_streamed():
    a = Tensor(np.zeros((64, 64), np.float32))
    Receiver(lambda v: None, [a.sum(-1) * 0.5])
    reads, writes = _marks(min_bytes=1 << 20)
    assert not reads and not writes


def test_loop_invariant_reads_are_not_streamed():
    """A Tensor the loop body only reads is read again by every iteration;
    a value the body writes (here a Feeder's) and one command reads is not."""
    w = Tensor(np.zeros((64, 64), np.float32))
    acc = [Tensor(np.zeros((64,), np.float32))]

    def body():
        x = ad.Feeder(lambda: np.zeros((64, 64), np.float32), shape=[64, 64])
        acc[0] += (w * 2.0).sum(-1) + (x * 3.0).sum(-1)
    ad.ir_for(range(3), body)
    Receiver(lambda v: None, [acc[0]])
    reads, _ = _marks()
    assert w.id not in reads
    assert reads            # the Feeder's value, in the arena


def test_results_no_command_reads_are_streamed_on_write():
    x = Tensor(np.zeros((1 << 12,), np.float32))
    y = ((x * 0.5 + 1.0).exp2() + 1.0).recip() * 3.0
    Receiver(lambda v: None, [y])
    reads, writes = _marks()
    assert x.id in reads and writes


def test_marks_follow_the_device_that_plans():
    """A second device on the same Proc with streaming off clears the marks
    the first one left on its accesses."""
    a = Tensor(np.zeros((64, 64), np.float32))
    Receiver(lambda v: None, [a.sum(-1) * 0.5])
    proc = ad.compile_proc()
    info = codegen.BufferInfo()
    for c in proc.procedure:
        if isinstance(c, AllocEntry):
            info.size[c.id] = c.size
    marked = []
    for min_bytes in (1024, None):
        dev = HIPDevice.__new__(HIPDevice)
        dev.stream_min_bytes = min_bytes
        dev._mark_streams(proc, info)
        marked.append(any(getattr(km, "stream", False) for c in proc.procedure
                          for n in getattr(c, "nodes", [c]) for k in getattr(n, "kargs", [])
                          for km in codegen.iter_kmatrix(k)))
    assert marked == [True, False]
