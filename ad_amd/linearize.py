"""Dependency collection, greedy fusion and Proc emission
(autodiff/linearize.py:13-271).

The output command order is the order of the second toposort's layers, and
every container whose iteration order feeds it (dicts keyed in traversal
order, sets of ids) is built with the same sequence of operations as the
reference.  Two things differ from a literal reading, neither of which can
change the result:

* a command's dependency set is computed once per ``fuse`` call and reused
  (kernel args are not renamed while fusing);
* the scan of every fusion attempt starts at the first layer that still holds
  an untaken node able to start a group: earlier layers only hold taken or
  non-starting nodes, which the reference visits without any effect while no
  group has started yet;
* the white list of nodes downstream of a blocked node is decided per node
  as the scan reaches it (``_LazyWhiteList``) instead of walking every later
  layer at each block (``_EagerWhiteList``, the reference's way, kept as the
  check); both give the same set at every point of the scan.
"""
from copy import deepcopy
from typing import Dict, List

from .context import Block, Proc
from .fusion.base import FuseBase, FuseResult
from .fusion.helper import get_deps, get_res
from .fusion.ops import DPElwFuse, ElwFuse, ReduceElwFuse
from .helper import walk_graph
from .node import Node
from .toposort import toposort

global_deps: Dict[int, Dict[int, set]] = {}
id_to_node: Dict[int, object] = {}
block_to_node: Dict[int, int] = {}
alr_defined_global: Dict[int, list] = {}


def reset_state():
    global global_deps, id_to_node, block_to_node, alr_defined_global
    global_deps = {}
    id_to_node = {}
    block_to_node = {}
    alr_defined_global = {}


def insert_to_global_dep(block_id: int, key: int, value):
    if block_id not in global_deps:
        global_deps[block_id] = dict()
    if key not in global_deps[block_id]:
        global_deps[block_id][key] = set({value}) if value is not None else set({})
    elif value is not None:
        global_deps[block_id][key].add(value)


def get_deps_global(block: Block, alr_defined: Dict[int, int] = None):
    """Record, per block, ``node -> ids it waits on``.  Reads of ids defined
    in an enclosing block become a dependency of the enclosing loop node
    (linearize.py:31-101)."""
    if alr_defined is None:
        alr_defined = dict()
    if block.id not in alr_defined_global:
        alr_defined_global[block.id] = list(alr_defined.keys())

    defined = dict()
    vars_need_dep = dict()
    for n in block.nodes:
        inner_bl = n.get_block()
        if inner_bl:
            def_block, need_dep_block = get_deps_global(inner_bl, alr_defined | defined)
            for (dep, block_id) in deepcopy(list(need_dep_block.items())):
                if block_id == block.id:
                    insert_to_global_dep(block.id, n.id, dep)
                    del need_dep_block[dep]
            defined.update(def_block)
            vars_need_dep.update(need_dep_block)
            block_to_node[inner_bl.id] = n.id
        else:
            _collect(n, set(), block, alr_defined, defined, vars_need_dep)
    return defined, vars_need_dep


def _collect(n, visited, block, alr_defined, defined, vars_need_dep):
    if n.id in visited or n.id in alr_defined:
        return
    if isinstance(n, Node):
        for dep in n.kargs_child_ids():
            should_visit = True
            value = dep
            if dep in alr_defined:
                value = None
                should_visit = False
                vars_need_dep[dep] = alr_defined[dep]
            if dep in defined:
                block_id_defined = defined[dep]
                if block_id_defined != block.id:
                    should_visit = False
                    value = block_to_node[block_id_defined]
            insert_to_global_dep(block.id, n.id, value)
            if should_visit:
                visited.add(n.id)
                _collect(id_to_node[dep], visited, block, alr_defined, defined, vars_need_dep)
        if n.id not in defined:
            defined[n.id] = block.id


_FUSION_FAMILIES = [DPElwFuse, ReduceElwFuse, ElwFuse]


def _walking_path(start_id, later_layers, deps_of):
    """fusion/helper.py:70-81: ``start_id`` plus every node of the later
    layers, scanned in layer order, that depends on a node already in the
    path."""
    path = set({start_id})
    for layer in later_layers:
        for nid in layer:
            if len(path.intersection(deps_of(nid))) > 0:
                path.add(nid)
    return path


class _EagerWhiteList:
    """The reference's white list: the union of the walking paths of every
    start so far, each path computed in full when it starts."""

    def __init__(self, toposort_res, deps_of):
        self.res, self.deps_of, self.nodes = toposort_res, deps_of, set()

    def reach(self, nid, layer_idx, deps_id):
        pass

    def start(self, nid, layer_idx):
        self.nodes.update(_walking_path(nid, self.res[layer_idx + 1:], self.deps_of))

    def __contains__(self, nid):
        return nid in self.nodes


class _LazyWhiteList:
    """The same set, decided per node when the scan reaches it: node ->
    lowest start layer among the paths holding it.  A node scanned in layer L
    is on the path started in layer L0 iff L > L0 and one of its
    dependencies joined that path earlier in the scan, so scanning in order
    decides membership without walking any path ahead."""

    def __init__(self, toposort_res, deps_of):
        self.low = {}

    def reach(self, nid, layer_idx, deps_id):
        if not self.low:
            return
        best = None
        for d in deps_id:
            m = self.low.get(d)
            if m is not None and m < layer_idx and (best is None or m < best):
                best = m
        if best is not None:
            self.low[nid] = best

    def start(self, nid, layer_idx):
        self.low[nid] = min(self.low.get(nid, layer_idx), layer_idx)

    def __contains__(self, nid):
        return nid in self.low


# the lazy white list is the product path; the eager one is its check
EAGER_WALKING_PATHS = False


def fuse(g_dep_id) -> Proc:
    """Toposort a block, greedily grow fused groups family by family, then
    re-toposort with groups as single commands (linearize.py:103-250)."""
    deps = global_deps[g_dep_id]
    toposort_res = list(toposort(deps))

    deps_cache: Dict[int, set] = {}

    def deps_of(nid):
        d = deps_cache.get(nid)
        if d is None:
            d = get_deps(id_to_node[nid])
            deps_cache[nid] = d
        return d

    entries: List[FuseBase] = []
    init_taken = set()

    for family in _FUSION_FAMILIES:
        probe = family.__new__(family)       # only for can_start(); allocates no id
        first_layer = 0
        while True:
            op_entry = family()
            white = (_EagerWhiteList if EAGER_WALKING_PATHS else _LazyWhiteList)(toposort_res, deps_of)
            did_start = False
            # skip leading layers in which no untaken node can start a group
            while first_layer < len(toposort_res) and not any(
                    nid not in init_taken and probe.can_start(id_to_node[nid])
                    for nid in toposort_res[first_layer]):
                first_layer += 1
            for layer_idx in range(first_layer, len(toposort_res)):
                layer = toposort_res[layer_idx]
                did_sum = False
                for nid in layer:
                    deps_id = deps_of(nid)
                    white.reach(nid, layer_idx, deps_id)
                    if nid in init_taken:
                        if len(deps_id.intersection(op_entry.result_tracker)) > 0:
                            white.start(nid, layer_idx)
                        continue
                    if nid in white:
                        continue
                    result = op_entry.attempt_fuse(id_to_node[nid], deps_id)
                    if result in (FuseResult.ADD, FuseResult.INIT):
                        init_taken.add(nid)
                        did_sum = True
                        did_start = True
                    elif len(deps_id.intersection(op_entry.result_tracker)) > 0:
                        white.start(nid, layer_idx)
                if did_start and not did_sum:
                    break
            if len(op_entry.nodes) == 0:
                break
            if len(op_entry.nodes) == 1:
                init_taken.add(op_entry.nodes[0].id)
            elif len(op_entry.nodes) > 1:
                entries.append(op_entry)

    # place each group in the layer of its last member, then drop the members
    layer_of = {}
    for idx, layer in enumerate(toposort_res):
        for nid in layer:
            layer_of.setdefault(nid, idx)
    nodes_to_remove = set()
    for entry in entries:
        idx = layer_of.get(entry.nodes[-1].id)
        if idx is None:
            raise Exception("Couldn't find node in toposort_res to insert fused entry")
        id_to_node[entry.fuse_id] = entry
        toposort_res[idx].add(entry.fuse_id)
        for node in entry.nodes:
            nodes_to_remove.add(node.id)
    for idx, layer in enumerate(toposort_res):
        toposort_res[idx] = set(filter(lambda x: x not in nodes_to_remove, layer))

    # fuse loop bodies; map ids produced inside a group/loop to the group/loop
    replace = dict()
    for layer in toposort_res:
        for nid in layer:
            node = id_to_node[nid]
            if isinstance(node, Node) and node.get_block() is not None:
                node.proc = fuse(node.get_block().id)
                replace.update({r: node.id for r in get_res(node, True)})
            if isinstance(node, FuseBase):
                replace.update({r: node.fuse_id for r in get_res(node)})

    g_dep = {}
    for layer in toposort_res:
        for nid in layer:
            node = id_to_node[nid]
            d = get_deps(node, step_proc=True)
            d = set({(replace[x] if x in replace else x) for x in d})
            key = node.id if isinstance(node, Node) else node.fuse_id
            g_dep[key] = d
    for key in g_dep:
        g_dep[key] = set(filter(lambda x: x in g_dep.keys(), g_dep[key]))

    proc = []
    for layer in list(toposort(g_dep)):
        for nid in layer:
            proc.append(id_to_node[nid])
    return Proc(proc)


def linearize(main_block: Block) -> Proc:
    global global_deps, id_to_node, block_to_node, alr_defined_global
    id_to_node = {}

    def insert_id_to_node(node, _):
        if node.id not in id_to_node:
            id_to_node[node.id] = node
        return node
    walk_graph(main_block, insert_id_to_node, walk_block=True, walk_child=True)

    global_deps = {}
    block_to_node = {}
    alr_defined_global = {}
    _, d = get_deps_global(main_block)
    assert len(d) == 0, "vars need dep not None!"
    return fuse(0)
