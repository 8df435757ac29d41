"""Values both allocated and freed inside one fused group live in registers
(the behaviour of autodiff/alloc/temp.py:12-34)."""
from ..node import Node
from . import AllocEntry, DeallocEntry


def _closed_inside(group):
    """Ids whose last allocation event in the group is a free that follows
    an allocation in the group (an id allocated again after its free is
    open again)."""
    state = {}
    for n in group.nodes:
        if isinstance(n, AllocEntry):
            state[n.id] = "open"
        elif isinstance(n, DeallocEntry) and n.id in state:
            state[n.id] = "closed"
    return {i for i, s in state.items() if s == "closed"}


def temp_alloc(proc, fused_ids_to_f):
    """Mark those ids temp: their Alloc/Dealloc entries, and every read or
    write of them by the group's nodes."""
    for group in fused_ids_to_f.values():
        temps = _closed_inside(group)
        if not temps:
            continue
        for n in group.nodes:
            if isinstance(n, (AllocEntry, DeallocEntry)):
                if n.id in temps:
                    n.is_temp = True
            elif isinstance(n, Node):
                for t in temps:
                    n.change_to_temp(t)
