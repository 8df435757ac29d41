"""Layout of the unpacked arena (``HIPDevice(arena="unpacked")``) on the
CPU: every tetris variable gets a region of its own, disjoint from every
other variable and buffer, starting at the address its packed offset would
have modulo the 256-byte alignment (so every alignment a kernel was planned
for holds), and fewer launch groups than the packed arena."""
import ad_amd as ad
from ad_amd import workloads
from ad_amd.device.hip import codegen
from ad_amd.device.hip.device import ALIGN, HIPDevice
from ad_amd.device.hip.schedule import schedule_dag
from ad_amd.graph import ForNode


def _layout(proc, arena):
    dev = HIPDevice.__new__(HIPDevice)
    dev.arena = arena
    dev.buffers, dev.buffers_size, dev._contents = {}, {}, {}
    dev._allocs, dev._pending, dev._vars, dev._var_off = [], [], {}, {}
    dev._feeder_slots = {}

    def visit(c, _):
        dev.init(c)
        return c
    proc.walk(visit, step_fused=False, step_proc=True)
    end, info = dev._layout()
    return dev, end, info


def test_unpacked_regions_are_disjoint_and_congruent():
    workloads.transformer(layers=2, d_model=32, heads=4, ff=64, seq=8, batch=2, steps=2)
    proc = ad.compile_proc()
    dev, end, info = _layout(proc, "unpacked")
    assert info.unpacked and dev._vars
    spans = [(dev.buffers[b], dev.buffers[b] + 4 * dev.buffers_size[b]) for b in dev.buffers]
    for vid, (voff, size) in dev._vars.items():
        start = dev._var_off[vid]
        assert start % ALIGN == (4 * voff) % ALIGN
        # an access at packed float offset voff + r lands at start + 4 r
        assert dev._addr(None, voff + 3, (vid, voff, size)) == start + 12
        spans.append((start, start + 4 * size))
    spans.sort()
    for (a0, a1), (b0, b1) in zip(spans, spans[1:]):
        assert a1 <= b0
    assert spans[-1][1] <= end


def test_packed_layout_keeps_tetris_offsets():
    workloads.mlp(steps=2, din=16, dh=24, dout=8)
    proc = ad.compile_proc()
    dev, _, info = _layout(proc, "packed")
    assert not info.unpacked and not dev._var_off
    for vid, (voff, size) in dev._vars.items():
        bid = next(b for b in dev.buffers if dev.buffers_size[b] >= voff + size)
        assert dev._addr(bid, voff + 1, (vid, voff, size)) == dev.buffers[bid] + 4 * (voff + 1)


def test_unpacked_schedule_has_fewer_groups():
    workloads.transformer(layers=2, d_model=32, heads=4, ff=64, seq=8, batch=2, steps=1, receive=False)
    proc = ad.compile_proc()
    body = [c for c in proc.procedure if isinstance(c, ForNode)][0].get_proc()
    counts = {}
    for unpacked in (False, True):
        _, _, info = _layout(proc, "unpacked" if unpacked else "packed")
        launches = []
        for c in body.procedure:
            if hasattr(c, "program_id") and type(c).__name__ not in ("Feeder", "Receiver"):
                reads, writes = codegen.command_regions(c, info)
                launches.append((codegen.command_plans(c, info, 0)[0][0].name, reads, writes))
        counts[unpacked] = len(schedule_dag(launches, group_key=lambda k: k)[0])
    assert counts[True] < counts[False]
