"""Draft-tree bookkeeping (host side): ancestor masks, depths, generators.

A tree of T <= 64 nodes is a parent array with parents[0] = -1 (the root: the
last committed token) and parents[i] < i (nodes in BFS / topological order).
Node i is verified at position ctx + depth(i); its attention mask row has bit m
set iff m is an ancestor-or-self of i.
"""
import numpy as np


def depths(parents):
    parents = np.asarray(parents)
    d = np.zeros(len(parents), dtype=np.int64)
    for i in range(1, len(parents)):
        d[i] = d[parents[i]] + 1
    return d


def ancestor_masks(parents):
    """uint64 bitmask per node (returned as int64 with the same bits)."""
    parents = np.asarray(parents)
    T = len(parents)
    if T > 64:
        raise ValueError("ancestor masks need T <= 64")
    m = np.zeros(T, dtype=np.uint64)
    for i in range(T):
        p = int(parents[i])
        m[i] = (m[p] if p >= 0 else np.uint64(0)) | (np.uint64(1) << np.uint64(i))
    return m.view(np.int64)


def chain_parents(n):
    return np.arange(-1, n - 1, dtype=np.int32)


def random_tree(num_nodes, max_depth, rng):
    """EAGLE-style random tree: a spine reaching ``max_depth``, remaining nodes
    attached to uniformly chosen nodes of depth < max_depth, relabelled in BFS
    order (children in creation order).  Returns int32 parents [num_nodes]."""
    if num_nodes < max_depth + 1:
        raise ValueError("num_nodes must be >= max_depth + 1")
    par = [-1] + list(range(max_depth))          # spine 0-1-2-...-max_depth
    dep = list(range(max_depth + 1))
    while len(par) < num_nodes:
        cands = [i for i, d in enumerate(dep) if d < max_depth]
        p = cands[int(rng.integers(len(cands)))]
        par.append(p)
        dep.append(dep[p] + 1)
    children = [[] for _ in par]
    for i in range(1, len(par)):
        children[par[i]].append(i)
    order, head = [0], 0
    while head < len(order):
        order.extend(children[order[head]])
        head += 1
    new_id = {old: new for new, old in enumerate(order)}
    out = np.empty(num_nodes, dtype=np.int32)
    for old, new in new_id.items():
        out[new] = -1 if par[old] < 0 else new_id[par[old]]
    return out
