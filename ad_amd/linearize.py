"""Dependency collection, greedy fusion and Proc emission
(autodiff/linearize.py:13-271).

The output command order is the order of the second toposort's layers, and
every container whose iteration order feeds it (dicts keyed in traversal
order, sets of ids) is built with the same sequence of operations as the
reference.  The dependency walk runs on an explicit stack (no recursion
depth limit), visiting nodes in the order a depth-first recursion does.
Things that differ from a literal reading, none of which can change the
result:

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
from typing import Dict, List

from .context import Block, Proc
from .fusion.base import FuseBase, FuseResult
from .fusion.helper import get_deps, get_res
from .fusion.ops import DPElwFuse, ElwFuse, ReduceElwFuse
from .helper import walk_graph
from .node import Node
from .toposort import toposort

global_deps: Dict[int, Dict[int, set]] = {}      # block id -> node id -> ids it waits for
id_to_node: Dict[int, object] = {}
block_to_node: Dict[int, int] = {}               # loop body block id -> loop node id


def reset_state():
    global global_deps, id_to_node, block_to_node
    global_deps = {}
    id_to_node = {}
    block_to_node = {}


def _wait_for(block_id: int, node_id: int, dep):
    """Record that ``node_id`` (in block ``block_id``) waits for ``dep``;
    ``dep`` None records the node with nothing to wait for yet."""
    waits = global_deps.setdefault(block_id, {}).setdefault(node_id, set())
    if dep is not None:
        waits.add(dep)


def get_deps_global(block: Block, outer: Dict[int, int] = None):
    """Fill ``global_deps[block.id]``: for every node traced in ``block``,
    the ids it must wait for (linearize.py:31-101).

    ``outer`` maps ids defined in enclosing blocks to their block.  A read of
    such an id is not an edge inside this block: it is returned in
    ``needs`` (id -> defining block), and the enclosing block whose loop
    contains this one records it as a wait of that loop node.  A read of an
    id defined in a sibling loop body waits for that loop node.  Returns
    ``(defined, needs)``: ids defined in this block (and its loops), and
    outer ids it reads."""
    outer = {} if outer is None else outer
    defined: Dict[int, int] = {}
    needs: Dict[int, int] = {}
    finished = set()
    for node in block.nodes:
        body = node.get_block()
        if body is None:
            _collect(node, block, outer, defined, needs, finished)
            continue
        body_defined, body_needs = get_deps_global(body, outer | defined)
        for dep, where in list(body_needs.items()):
            if where == block.id:
                _wait_for(block.id, node.id, dep)
                del body_needs[dep]
        defined.update(body_defined)
        needs.update(body_needs)
        block_to_node[body.id] = node.id
    return defined, needs


def _collect(root, block, outer, defined, needs, finished):
    """Depth-first from ``root`` through the ids each node reads, recording
    waits.  A node's reads are visited in order, each one's subtree before
    the next read; a node is marked defined after its reads (post-order).
    Nodes of outer blocks, or already entered from this root, are not
    entered again; ids defined in another loop body stand for that loop.
    A node whose walk already finished (from an earlier root of the block)
    is not entered again either: its walk would record the same waits into
    the same sets and define nothing new."""
    entered = set()

    def enterable(node):
        return isinstance(node, Node) and node.id not in entered and node.id not in outer \
            and node.id not in finished

    if not enterable(root):
        return
    stack = [(root, root.kargs_child_ids(), [0])]
    while stack:
        node, reads, cursor = stack[-1]
        if cursor[0] == len(reads):
            stack.pop()
            finished.add(node.id)
            if node.id not in defined:
                defined[node.id] = block.id
            continue
        dep = reads[cursor[0]]
        cursor[0] += 1
        target, descend = dep, True
        if dep in outer:
            target, descend = None, False
            needs[dep] = outer[dep]
        if dep in defined and defined[dep] != block.id:
            target, descend = block_to_node[defined[dep]], False
        _wait_for(block.id, node.id, target)
        if descend:
            entered.add(node.id)
            child = id_to_node[dep]
            if enterable(child):
                stack.append((child, child.kargs_child_ids(), [0]))


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
    global global_deps, id_to_node, block_to_node
    id_to_node = {}

    def record(node, _):
        id_to_node.setdefault(node.id, node)     # the first node seen under an id
        return node
    walk_graph(main_block, record, walk_block=True, walk_child=True)

    global_deps = {}
    block_to_node = {}
    _, unresolved = get_deps_global(main_block)
    assert not unresolved, f"reads of ids defined outside the program: {sorted(unresolved)}"
    return fuse(0)
