"""Draft-tree topology for tree verification: node depths, ancestor bitmasks, the greedy
acceptance walk.

* ``compile_medusa_tree`` follows axiomlm/engine/medusa.py:48-116: the prefix closure of the
  top-k rank tuples, ordered by (length, tuple), becomes nodes 1..T-1 under the root 0;
  node u's mask is its parent's mask with bit u set, its RoPE offset is its depth.
  The reference caps a tree at 32 nodes (31 paths, :73-74) because its masks are 32-bit;
  the MI355X verify kernels take 64-bit masks, so ``max_nodes`` may be raised to 64.
* ``build_candidate_tree`` is the benchmark topology of
  benchmarks/benchmark_phase2_task21_verification_latency.py:97-122 (root with 4 children,
  then 3 levels of round-robin parents), extended past 32 nodes.
* ``build_branching_tree`` is a breadth-first tree with a fixed fan-out per depth
  (Sequoia-style, e.g. (4, 4, 2, 2, 1, 1) truncated to 64 nodes).
* ``greedy_tree_walk`` is the temperature-0 acceptance walk of medusa.py:313-330.
"""

from __future__ import annotations

from typing import Any

# The reference's default Medusa tree (medusa.py:28-45): top-k ranks per head along each path.
DEFAULT_MEDUSA_TREE_CHOICES: list[tuple[int, ...]] = [
    (0,), (1,), (2,), (3,),
    (0, 0), (0, 1), (0, 2), (1, 0), (1, 1), (2, 0),
    (0, 0, 0), (0, 0, 1), (0, 1, 0), (0, 1, 1), (1, 0, 0),
    (0, 0, 0, 0),
]

MAX_TREE_NODES = 64


def _from_parents(parent: list[int]) -> tuple[list[int], list[int]]:
    """Depths and ancestor masks of a tree given in topological order (parent[u] < u)."""
    depths, masks = [0], [1]
    for u in range(1, len(parent)):
        p = parent[u]
        if not 0 <= p < u:
            raise ValueError(f"node {u}: parent {p} is not an earlier node")
        depths.append(depths[p] + 1)
        masks.append(masks[p] | (1 << u))
    return depths, masks


def compile_medusa_tree(tree_choices, num_heads: int, max_nodes: int = 32) -> dict[str, Any]:
    """Topology metadata of a Medusa tree (medusa.py:48-116): num_nodes, tree_depths,
    tree_mask, parent, children, head_idx, topk_rank, max_topk_per_head, max_depth."""
    if not 1 <= max_nodes <= MAX_TREE_NODES:
        raise ValueError(f"max_nodes must be in [1, {MAX_TREE_NODES}]")
    paths = set()
    for choice in tree_choices:
        path = tuple(int(r) for r in choice)
        if 0 < len(path) <= num_heads:
            paths.update(path[:n] for n in range(1, len(path) + 1))
    order = sorted(paths, key=lambda p: (len(p), p))[: max_nodes - 1]
    node_of = {(): 0}
    parent = [-1]
    head_idx, topk_rank = [-1], [-1]
    max_topk = [1] * num_heads
    for u, path in enumerate(order, start=1):
        node_of[path] = u
        parent.append(node_of[path[:-1]])
        head_idx.append(len(path) - 1)
        topk_rank.append(path[-1])
        max_topk[len(path) - 1] = max(max_topk[len(path) - 1], path[-1] + 1)
    depths, masks = _from_parents(parent)
    children: list[list[int]] = [[] for _ in parent]
    for u in range(1, len(parent)):
        children[parent[u]].append(u)
    return {
        "num_nodes": len(parent),
        "tree_depths": depths,
        "tree_mask": masks,
        "parent": parent,
        "children": children,
        "head_idx": head_idx,
        "topk_rank": topk_rank,
        "max_topk_per_head": max_topk,
        "max_depth": max(depths),
    }


def build_candidate_tree(n: int) -> tuple[list[int], list[int]]:
    """(tree_depths, tree_mask) of the n-node verification benchmark tree: nodes 1-4 hang off
    the root, 5-16 off nodes 1-4 in turn, 17+ off nodes 5-16 in turn."""
    if not 1 <= n <= MAX_TREE_NODES:
        raise ValueError(f"n must be in [1, {MAX_TREE_NODES}]")
    parent = [-1]
    for i in range(1, n):
        parent.append(0 if i <= 4 else (1 + (i - 5) % 4 if i <= 16 else 5 + (i - 17) % 12))
    return _from_parents(parent)


def build_branching_tree(branching, max_nodes: int = MAX_TREE_NODES) -> dict[str, Any]:
    """Breadth-first tree where every node at depth d has ``branching[d]`` children, truncated
    to ``max_nodes`` nodes; returns num_nodes, parent, children, tree_depths, tree_mask."""
    if not 1 <= max_nodes <= MAX_TREE_NODES:
        raise ValueError(f"max_nodes must be in [1, {MAX_TREE_NODES}]")
    parent = [-1]
    frontier = [0]
    for fan in branching:
        nxt = []
        for p in frontier:
            for _ in range(int(fan)):
                if len(parent) == max_nodes:
                    break
                parent.append(p)
                nxt.append(len(parent) - 1)
        frontier = nxt
    depths, masks = _from_parents(parent)
    children: list[list[int]] = [[] for _ in parent]
    for u in range(1, len(parent)):
        children[parent[u]].append(u)
    return {"num_nodes": len(parent), "parent": parent, "children": children, "tree_depths": depths,
            "tree_mask": masks}


def greedy_tree_walk(preds, node_tokens, children, max_emit: int) -> tuple[list[int], list[int]]:
    """Temperature-0 acceptance (medusa.py:313-330): from the root, emit the model's
    prediction at the current node and descend into the first child drafted with that token.
    Returns (accepted node indices starting with 0, emitted tokens)."""
    accepted, emitted = [0], []
    u = 0
    while len(emitted) < max_emit:
        tok = int(preds[u])
        emitted.append(tok)
        nxt = next((c for c in children[u] if int(node_tokens[c]) == tok), None)
        if nxt is None or len(emitted) >= max_emit:
            break
        u = nxt
        accepted.append(u)
    return accepted, emitted
