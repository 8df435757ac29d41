"""Insert Alloc before a result's first definition and Dealloc after its last
read (autodiff/alloc/insert.py:10-125).

Quirks kept for offset parity:
* a re-defined result only records its larger size on the *Location*
  (insert.py:31), so the Alloc keeps its first size;
* loop bodies are keyed by the enclosing Proc's id (insert.py:68-70);
* results defined but never read are freed at the end of the main Proc.
Tensor declarations become Allocs that carry the host array."""
from math import prod
from typing import Dict, Tuple

from ..fusion import FuseBase
from ..fusion.helper import get_deps, get_res
from ..graph import Receiver, Tensor
from ..node import Node
from . import AllocEntry, DeallocEntry, Location


def insert_alloc(main_proc) -> Dict[int, FuseBase]:
    insert_locs: Dict[int, Tuple[Location, AllocEntry]] = {}
    dealloc_locs: Dict[int, Tuple[Location, DeallocEntry]] = {}
    tracker: Dict[int, bool] = {}
    fused_ids_to_f: Dict[int, FuseBase] = {}
    proc_ids_to_p: Dict[int, object] = {}
    id_to_size: Dict[int, int] = {}

    def step_node(loc: Location, n):
        assert isinstance(n, Node)
        if not isinstance(n, Receiver):
            r = list(get_res(n))[0]
            if r in insert_locs:
                insert_locs[r][0].size = max(insert_locs[r][1].size, prod(n.shape))
            elif r in id_to_size:
                assert id_to_size[r] == prod(n.shape), \
                    "In place operation dimension are not equal when inserting alloc"
            else:
                insert_locs[r] = (loc, AllocEntry(r, prod(n.shape)))
            tracker[n.id] = False
            id_to_size[n.id] = prod(n.shape)
        for dep in list(get_deps(n)):
            dealloc_locs[dep] = (loc + 1, DeallocEntry(dep, id_to_size[dep]))
            tracker[dep] = True

    def step_proc(proc, proc_id=None):
        for idx, p in enumerate(proc.procedure):
            if isinstance(p, FuseBase):
                for fuse_idx, n in enumerate(p.nodes):
                    fused_ids_to_f[p.fuse_id] = p
                    if isinstance(n, Tensor):
                        p.nodes[fuse_idx] = AllocEntry(n.id, prod(n.shape), n.arr)
                        id_to_size[n.id] = prod(n.shape)
                        continue
                    step_node(Location(fuse_idx, fused_id=p.fuse_id, proc_id=None), n)
            elif isinstance(p, Node):
                if isinstance(p, Tensor):
                    proc.procedure[idx] = AllocEntry(p.id, prod(p.shape), p.arr)
                    id_to_size[p.id] = prod(p.shape)
                    continue
                if p.get_proc() is not None:
                    proc_ids_to_p[proc.id] = p.proc
                    step_proc(p.proc, proc.id)
                    continue
                step_node(Location(idx, fused_id=None, proc_id=proc_id), p)
            else:
                raise TypeError(f"Invalid type: {type(p)}")

    step_proc(main_proc)

    leftovers = [k for k, consumed in tracker.items() if not consumed]
    for var in leftovers:
        dealloc_locs[var] = (Location(len(main_proc.procedure), None, None),
                             DeallocEntry(var, id_to_size[var]))

    total = list(dealloc_locs.values())
    total.extend(insert_locs.values())
    total = sorted(total, key=lambda x: (
        x[0].proc_id if x[0].proc_id is not None else -1,
        x[0].fused_id if x[0].fused_id is not None else -1,
        x[0].loc))

    insert_counter = {}
    for (loc, entry) in total:
        base = loc.base()
        offset = insert_counter.get(base, 0)
        insert_counter[base] = offset
        if loc.fused_id is not None:
            fused_ids_to_f[loc.fused_id].nodes.insert(loc.loc + offset, entry)
        elif loc.proc_id is not None:
            proc_ids_to_p[loc.proc_id].insert(loc.loc + offset, entry)
        else:
            main_proc.insert(loc.loc + offset, entry)
        insert_counter[base] += 1
    return fused_ids_to_f
