"""Sequoia tree optimizer (axiomlm_amd/sequoia.py) against brute force and hand-derived
cases.

G(n) of the dynamic program must be the largest expected number of accepted tokens
over every tree of at most n nodes (depth <= num_heads, candidate ranks < max_branches),
where a tree's expectation is the sum over its nodes of the product of P[depth, rank]
along the node's path (the root counts 1); the reconstructed tree must reach it.
"""

import itertools

import numpy as np
import pytest

from axiomlm_amd.sequoia import (M3_PRO_TREE_LATENCY, MI355X_7B_Q4_TREE_LATENCY, SequoiaDPOptimizer,
                                 interpolate_hardware_latency)
from axiomlm_amd.tree import compile_medusa_tree


def tree_value(paths, P):
    v = 1.0
    for p in paths:
        prod = 1.0
        for d, r in enumerate(p):
            prod *= P[d, r]
        v += prod
    return v


def all_trees(max_nodes, D, B):
    """Every prefix-closed set of paths (ranks < B, length <= D) with at most max_nodes - 1 paths."""
    found = {frozenset()}
    frontier = [frozenset()]
    while frontier:
        nxt = []
        for t in frontier:
            if len(t) + 1 >= max_nodes:
                continue
            parents = [()] + [p for p in t if len(p) < D]
            for par in parents:
                for r in range(B):
                    c = par + (r,)
                    if c not in t:
                        u = t | {c}
                        if u not in found:
                            found.add(u)
                            nxt.append(u)
        frontier = nxt
    return found


@pytest.mark.parametrize("D,B,N,seed", [(3, 3, 7, 0), (2, 4, 8, 1), (4, 2, 8, 2), (3, 2, 9, 3)])
def test_dp_equals_brute_force(D, B, N, seed):
    rng = np.random.default_rng(seed)
    opt = SequoiaDPOptimizer(num_heads=D, max_branches=B, max_budget=N)
    opt.set_acceptance_probabilities(rng.uniform(0.05, 0.9, (D, B)))
    T, split = opt.solve_dp_tables()
    trees = all_trees(N, D, B)
    for n in range(1, N + 1):
        best = max(tree_value(t, opt.P) for t in trees if len(t) + 1 <= n)
        G = float(np.max(T[n, 0, :]))
        assert G == pytest.approx(best, rel=1e-12, abs=1e-12), n
        paths = opt.extract_tree_for_budget(n, T, split)
        assert len(paths) == len(set(paths)) and len(paths) + 1 <= n
        assert all(p[:k] in paths for p in paths for k in range(1, len(p)))  # prefix closed
        assert all(len(p) <= D and max(p) < B for p in paths)
        assert tree_value(paths, opt.P) == pytest.approx(G, rel=1e-12), n


def test_planted_mistake_fails_brute_force():
    """A recurrence that drops the subtree term (P times the child's best) undercounts:
    the brute force above would catch it."""
    rng = np.random.default_rng(5)
    opt = SequoiaDPOptimizer(num_heads=3, max_branches=3, max_budget=7)
    opt.set_acceptance_probabilities(rng.uniform(0.3, 0.9, (3, 3)))
    best = max(tree_value(t, opt.P) for t in all_trees(7, 3, 3))
    wrong = 1.0 + sum(sorted(opt.P[0], reverse=True)[:3])  # children of the root only
    assert best - wrong > 0.05


def test_default_probabilities_small_budgets_by_hand():
    """Default P (0.65, 0.45, 0.30, 0.20 per head, x 0.35 per rank): n = 2 -> one child;
    n = 3 -> a chain (1 + .65 + .2925 = 1.9425 beats two children, 1.8775); n = 4 ->
    {(0), (1), (0,0)} = 2.17 (a chain of three gives 2.03025)."""
    opt = SequoiaDPOptimizer(max_budget=8)
    T, split = opt.solve_dp_tables()
    assert opt.extract_tree_for_budget(1, T, split) == []
    assert opt.extract_tree_for_budget(2, T, split) == [(0,)]
    assert sorted(opt.extract_tree_for_budget(3, T, split)) == [(0,), (0, 0)]
    assert sorted(opt.extract_tree_for_budget(4, T, split)) == [(0,), (0, 0), (1,)]
    assert np.max(T[3, 0]) == pytest.approx(1.9425, abs=1e-12)
    assert np.max(T[4, 0]) == pytest.approx(2.17, abs=1e-12)
    c = compile_medusa_tree(opt.extract_tree_for_budget(4, T, split), 4)
    assert c["parent"] == [-1, 0, 0, 1]


def test_latency_interpolation_closed_form():
    t = interpolate_hardware_latency({2: 1.2, 4: 1.6, 8: 2.0}, max_N=10)
    assert t[1] == 1.0 and t[2] == 1.2 and t[3] == pytest.approx(1.4) and t[4] == 1.6
    assert t[6] == pytest.approx(1.8) and t[9] == 2.0 and t[10] == 2.0
    src = {4: 2.0}
    t = interpolate_hardware_latency(src, max_N=5)
    assert src == {4: 2.0}  # caller's dict untouched
    assert t[2] == pytest.approx(1 + 1 / 3) and t[5] == 2.0
    ti = interpolate_hardware_latency(M3_PRO_TREE_LATENCY, max_N=64)
    vals = [ti[n] for n in range(1, 65)]
    assert vals[0] == 1.0 and all(a <= b for a, b in zip(vals, vals[1:]))
    ti = interpolate_hardware_latency(MI355X_7B_Q4_TREE_LATENCY, max_N=64)
    assert all(ti[n] == v for n, v in MI355X_7B_Q4_TREE_LATENCY.items()) and ti[64] > ti[32] > ti[2] > 1.0


def test_default_profile_choice_is_pinned():
    """The default MI355X profile with the default acceptance probabilities picks the 15-node,
    depth-3 tree (expected 2.77 tokens, speedup 1.715), for either budget cap; a profile whose
    t(3), t(4) sit above t(8) (the decode GEMV serving up to four rows) would not."""
    for cap in (32, 64):
        r = SequoiaDPOptimizer(max_budget=cap).solve_optimal_tree()
        assert (r.optimal_N, r.max_depth) == (15, 3)
        assert r.expected_accepted_tokens == pytest.approx(2.77, abs=5e-3)
        assert r.speedup == pytest.approx(1.715, abs=5e-3)
        assert r.tree_choices == [(0,), (0, 0), (0, 0, 0), (0, 0, 1), (0, 1), (0, 1, 0), (0, 2), (1,), (1, 0),
                                  (1, 0, 0), (1, 1), (2,), (2, 0), (3,)]
    assert all(a <= b for a, b in zip(list(MI355X_7B_Q4_TREE_LATENCY.values()),
                                      list(MI355X_7B_Q4_TREE_LATENCY.values())[1:]))


def test_solve_optimal_tree_picks_max_speedup():
    opt = SequoiaDPOptimizer(max_budget=32, latency_profile=M3_PRO_TREE_LATENCY)
    r = opt.solve_optimal_tree()
    sp = {n: s["speedup"] for n, s in r.all_budget_stats.items()}
    assert r.speedup == max(sp.values()) and sp[r.optimal_N] == r.speedup
    assert min(n for n, v in sp.items() if v == r.speedup) == r.optimal_N
    s = r.all_budget_stats[r.optimal_N]
    assert s["effective_latency"] == pytest.approx(s["verification_t"] + s["draft_cost"], abs=1e-4)
    assert r.compiled_tree["num_nodes"] == len(r.tree_choices) + 1
    # with free verification and drafting every extra node pays: the largest budget wins
    flat = SequoiaDPOptimizer(max_budget=20, draft_cost_c=0.0, latency_profile={1: 1.0, 20: 1.0})
    r = flat.solve_optimal_tree()
    assert r.optimal_N == 20 and r.compiled_tree["num_nodes"] == 20


def test_budget_up_to_64_nodes():
    opt = SequoiaDPOptimizer(num_heads=6, max_branches=4, max_budget=64)
    r = opt.solve_fixed_budget(64)
    assert r.optimal_N == 64 and r.compiled_tree["num_nodes"] == 64
    assert len(r.tree_choices) == 63 and max(len(p) for p in r.tree_choices) <= 6
    assert r.compiled_tree["tree_mask"][63] >> 63 == 1
    T, _ = opt.solve_dp_tables()
    G = [float(np.max(T[n, 0])) for n in range(1, 65)]
    assert all(b >= a for a, b in zip(G, G[1:]))


def test_one_row_probabilities_scale_by_depth():
    opt = SequoiaDPOptimizer(num_heads=3)
    opt.set_acceptance_probabilities([0.5, 0.2])
    assert opt.max_branches == 2
    assert np.allclose(opt.P, [[0.5, 0.2], [0.425, 0.17], [0.36125, 0.1445]])
    with pytest.raises(ValueError):
        opt.set_acceptance_probabilities(np.zeros((2, 2, 2)))


def test_all_trees_enumerator_counts():
    # ranks < 2, depth <= 2, at most 3 nodes: {}, {0}, {1}, {0,1}, {0,00}, {0,01}, {1,10}, {1,11}
    assert len(all_trees(3, 2, 2)) == 8
    assert len(list(itertools.islice(all_trees(2, 3, 3), 10))) == 4


def _scalar_tables(P, N, D, B):
    """The recurrence as scalar loops over m (sequoia_dp.py:183-195 order): the first m
    that strictly improves the running best wins."""
    T = np.zeros((N + 1, D + 1, B + 1))
    split = np.zeros((N + 1, D + 1, B + 1), dtype=np.int32)
    T[1, :, :] = 1.0
    T[1:, :, 0] = 1.0
    T[1:, D, :] = 1.0
    for n in range(2, N + 1):
        for d in range(D - 1, -1, -1):
            for b in range(1, B + 1):
                best, best_m = T[n, d, b - 1], 0
                for m in range(1, n):
                    v = T[n - m, d, b - 1] + float(P[d, b - 1]) * float(np.max(T[m, d + 1, :]))
                    if v > best:
                        best, best_m = v, m
                T[n, d, b], split[n, d, b] = best, best_m
    return T, split


@pytest.mark.parametrize("seed", [0, 1])
def test_vectorized_tables_equal_scalar_loops(seed):
    rng = np.random.default_rng(seed)
    opt = SequoiaDPOptimizer(num_heads=5, max_branches=4, max_budget=40)
    if seed:  # ties: equal probabilities across ranks
        opt.set_acceptance_probabilities(np.full((5, 4), 0.5))
    else:
        opt.set_acceptance_probabilities(rng.uniform(0.05, 0.9, (5, 4)))
    T, split = opt.solve_dp_tables()
    T2, split2 = _scalar_tables(opt.P, 40, 5, 4)
    assert np.array_equal(T, T2) and np.array_equal(split, split2)
