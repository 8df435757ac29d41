"""Values both allocated and freed inside one fused group live in registers
(autodiff/alloc/temp.py:12-34)."""
from ..node import Node
from . import AllocEntry, DeallocEntry


def temp_alloc(proc, fused_ids_to_f):
    for group in fused_ids_to_f.values():
        seen = {}
        for n in group.nodes:
            if isinstance(n, AllocEntry):
                seen[n.id] = False
            elif isinstance(n, DeallocEntry):
                if n.id in seen:
                    seen[n.id] = True
        temps = set([i for i, closed in seen.items() if closed is True])
        for n in group.nodes:
            if isinstance(n, AllocEntry) and n.id in temps:
                n.is_temp = True
            if isinstance(n, DeallocEntry) and n.id in temps:
                n.is_temp = True
            if isinstance(n, Node):
                for t in temps:
                    n.change_to_temp(t)
