"""Draft-tree topology helpers (axiomlm_amd.tree) on the CPU.

The default Medusa tree is checked against its hand-derived node table (prefix
closure ordered by (length, tuple), medusa.py:48-116); every topology against
the defining invariants: a node's mask is exactly its ancestors plus itself,
its depth is the number of ancestors, parents precede children."""

import random

import pytest

from axiomlm_amd import tree as tr


def _ancestors(parent, u):
    out = []
    while u != -1:
        out.append(u)
        u = parent[u]
    return out


def _check_invariants(parent, depths, masks):
    for u in range(len(parent)):
        anc = _ancestors(parent, u)
        assert masks[u] == sum(1 << a for a in anc), u
        assert depths[u] == len(anc) - 1, u
        if u:
            assert parent[u] < u


def test_default_medusa_tree_table():
    t = tr.compile_medusa_tree(tr.DEFAULT_MEDUSA_TREE_CHOICES, num_heads=4)
    # Nodes: 1-4 (0)(1)(2)(3); 5-10 (0,0)(0,1)(0,2)(1,0)(1,1)(2,0); 11-15 (0,0,0)(0,0,1)(0,1,0)(0,1,1)(1,0,0);
    # 16 (0,0,0,0).
    assert t["num_nodes"] == 17
    assert t["parent"] == [-1, 0, 0, 0, 0, 1, 1, 1, 2, 2, 3, 5, 5, 6, 6, 8, 11]
    assert t["tree_depths"] == [0, 1, 1, 1, 1, 2, 2, 2, 2, 2, 2, 3, 3, 3, 3, 3, 4]
    assert t["head_idx"] == [-1, 0, 0, 0, 0, 1, 1, 1, 1, 1, 1, 2, 2, 2, 2, 2, 3]
    assert t["topk_rank"] == [-1, 0, 1, 2, 3, 0, 1, 2, 0, 1, 0, 0, 1, 0, 1, 0, 0]
    assert t["max_topk_per_head"] == [4, 3, 2, 1]
    assert t["max_depth"] == 4
    assert t["children"][0] == [1, 2, 3, 4] and t["children"][1] == [5, 6, 7] and t["children"][11] == [16]
    assert t["tree_mask"][16] == (1 << 0) | (1 << 1) | (1 << 5) | (1 << 11) | (1 << 16)
    _check_invariants(t["parent"], t["tree_depths"], t["tree_mask"])


def test_medusa_tree_prefix_closure_and_heads():
    # (2, 1) brings its missing prefix (2,); the empty path and the 3-long path (> num_heads) are dropped.
    t = tr.compile_medusa_tree([(2, 1), (), (0, 0, 0)], num_heads=2)
    assert t["num_nodes"] == 3
    assert t["parent"] == [-1, 0, 1] and t["topk_rank"] == [-1, 2, 1] and t["head_idx"] == [-1, 0, 1]
    assert t["max_topk_per_head"] == [3, 2] and t["tree_mask"] == [1, 0b11, 0b111]


def test_medusa_tree_cap_32_and_64():
    choices = [(a, b, c) for a in range(4) for b in range(4) for c in range(4)]
    t32 = tr.compile_medusa_tree(choices, num_heads=3)
    assert t32["num_nodes"] == 32  # reference cap: 31 paths + root (medusa.py:73-74)
    t64 = tr.compile_medusa_tree(choices, num_heads=3, max_nodes=64)
    assert t64["num_nodes"] == 64
    assert t64["tree_depths"][:32] == t32["tree_depths"] and t64["tree_mask"][:32] == t32["tree_mask"]
    assert t64["tree_mask"][63] >> 63 == 1
    _check_invariants(t64["parent"], t64["tree_depths"], t64["tree_mask"])
    with pytest.raises(ValueError):
        tr.compile_medusa_tree(choices, num_heads=3, max_nodes=65)


def test_candidate_tree_matches_benchmark_topology():
    d, m = tr.build_candidate_tree(32)
    # Root, 4 children, 12 grandchildren over nodes 1-4 in turn, 15 great-grandchildren over 5-16.
    assert d == [0] + [1] * 4 + [2] * 12 + [3] * 15
    assert m[5] == 0b100011 and m[17] == (1 << 17) | m[5]
    assert tr.build_candidate_tree(1) == ([0], [1])
    d64, m64 = tr.build_candidate_tree(64)
    assert d64[:32] == d and m64[:32] == m


def test_branching_tree_sequoia_64():
    t = tr.build_branching_tree((4, 4, 2, 2, 1, 1), max_nodes=64)
    assert t["num_nodes"] == 64
    depth_counts = [t["tree_depths"].count(k) for k in range(5)]
    assert depth_counts == [1, 4, 16, 32, 11]
    _check_invariants(t["parent"], t["tree_depths"], t["tree_mask"])
    small = tr.build_branching_tree((2, 1))
    assert small["parent"] == [-1, 0, 0, 1, 2]


def test_greedy_tree_walk():
    t = tr.compile_medusa_tree(tr.DEFAULT_MEDUSA_TREE_CHOICES, num_heads=4)
    rnd = random.Random(0)
    toks = [rnd.randrange(100) for _ in range(t["num_nodes"])]
    preds = [rnd.randrange(100) for _ in range(t["num_nodes"])]
    # Make the path 0 -> 2 -> 9 match: root predicts node 2's token, node 2 predicts node 9's.
    preds[0], preds[2] = toks[2], toks[9]
    toks[1] = toks[2] + 1000  # an earlier sibling with another token
    preds[9] = 12345
    acc, out = tr.greedy_tree_walk(preds, toks, t["children"], max_emit=10)
    assert acc == [0, 2, 9] and out == [toks[2], toks[9], 12345]
    acc, out = tr.greedy_tree_walk(preds, toks, t["children"], max_emit=2)
    assert acc == [0, 2] and out == [toks[2], toks[9]]
    acc, out = tr.greedy_tree_walk(preds, toks, t["children"], max_emit=1)
    assert acc == [0] and out == [toks[2]]
