"""Hardware-aware draft-tree sizing (Sequoia dynamic program) for tree verification.

The interface of axiomlm/speculative/sequoia_dp.py (``OptimalTreeResult``,
``interpolate_hardware_latency``, ``SequoiaDPOptimizer`` with
``solve_dp_tables`` / ``extract_tree_for_budget`` / ``solve_optimal_tree`` /
``solve_fixed_budget``).  The optimizer picks the tree that maximizes

    speedup(T) = G(|T|) / (t(|T|) + depth(T) * c)

where G is the expected number of accepted tokens under positional acceptance
probabilities P[d, b] (b-th candidate of draft head d accepted given its parent
was), t(N) the latency of verifying N tree nodes relative to a one-token
decode step, and c the relative cost of one draft head.

Differences from the reference, both from the hardware:
  * trees of up to 64 nodes (``MAX_TREE_NODES``): the runner's tree masks are
    64-bit, where the reference caps the budget at 32 for its 32-bit masks
    (sequoia_dp.py:96);
  * the default latency profile is this runner's on MI355X
    (``MI355X_7B_Q4_TREE_LATENCY``, the 7B Q4 model with an FP8 cache,
    measured with :func:`measure_tree_latency`) instead of the reference's Apple
    M3 Pro profile (sequoia_dp.py:99-102, kept as ``M3_PRO_TREE_LATENCY``).
With the same latency profile and probabilities and a budget of at most 32 the
optimizer returns the reference's tables, trees and statistics.
"""

from __future__ import annotations

import time
from dataclasses import dataclass
from typing import Any

import numpy as np

from .tree import MAX_TREE_NODES, compile_medusa_tree

# t(N) = verify_tree_step(N nodes) / step: Apple M3 Pro, MARLIN Q4 (sequoia_dp.py:99-102).
M3_PRO_TREE_LATENCY = {1: 1.000, 2: 1.280, 4: 1.385, 8: 1.488, 16: 2.315, 32: 3.926}
# The same ratio for this runner on one MI355X (measure_tree_latency): 7B shape (32 layers,
# d 4096, vocab 32000), MARLIN Q4 group 64, FP8 KV cache with a 2048-token prefix, branching
# trees of N nodes; host wall time of whole calls.  Two and three nodes run the decode GEMV
# with two / three token rows; from four nodes on the verify step runs the multi-token GEMM
# (the runner's switch point), so t(N) grows monotonically with N.  With the reference's
# default acceptance probabilities this profile makes the optimizer pick a 15-node tree of
# depth 3 (expected 2.77 accepted tokens per step, speedup 1.72).
MI355X_7B_Q4_TREE_LATENCY = {1: 1.0, 2: 1.27, 3: 1.42, 4: 1.50, 6: 1.51, 8: 1.52, 16: 1.56, 24: 1.73, 32: 1.79,
                             48: 2.17, 64: 2.27}


@dataclass
class OptimalTreeResult:
    """The chosen tree and its statistics (sequoia_dp.py:26-37)."""

    optimal_N: int
    max_depth: int
    expected_accepted_tokens: float
    verification_cost_t: float
    draft_cost: float
    speedup: float
    tree_choices: list[tuple[int, ...]]
    compiled_tree: dict[str, Any]
    all_budget_stats: dict[int, dict[str, float]]


def interpolate_hardware_latency(t_measured: dict[int, float], max_N: int = 32) -> dict[int, float]:
    """t(N) for every N in [1, max_N] by linear interpolation between the measured budgets
    (sequoia_dp.py:40-70): t(1) = 1 unless measured, and budgets past the last measured
    one take its value.  The caller's dict is not modified."""
    known = {int(k): float(v) for k, v in t_measured.items()}
    known.setdefault(1, 1.0)
    keys = np.array(sorted(known), dtype=np.int64)
    vals = np.array([known[k] for k in keys], dtype=np.float64)
    out: dict[int, float] = {}
    for n in range(1, max_N + 1):
        if n in known:
            out[n] = known[n]
            continue
        lo_i = int(np.searchsorted(keys, n, side="right")) - 1  # largest key <= n
        hi_i = int(np.searchsorted(keys, n, side="left"))        # smallest key >= n
        lo_i = max(lo_i, 0)
        if hi_i >= len(keys):
            hi_i = len(keys) - 1
        lo, hi = int(keys[lo_i]), int(keys[hi_i])
        if lo == hi:
            out[n] = float(vals[lo_i])
        else:
            alpha = (n - lo) / (hi - lo)
            out[n] = float(vals[lo_i] + alpha * (vals[hi_i] - vals[lo_i]))
    return out


def _default_acceptance(num_heads: int, max_branches: int) -> np.ndarray:
    """P[d, b] = p_d * 0.35^b with p_d = 0.65, 0.45, 0.30, 0.20, then 0.2 * 0.7^(d-3)
    (sequoia_dp.py:104-114)."""
    P = np.zeros((num_heads, max_branches), dtype=np.float64)
    decay = (0.65, 0.45, 0.30, 0.20)
    for d in range(num_heads):
        p = decay[d] if d < len(decay) else 0.20 * (0.7 ** (d - 3))
        for b in range(max_branches):
            P[d, b] = p * (0.35 ** b)
    return P


class SequoiaDPOptimizer:
    """Sequoia tree optimizer (sequoia_dp.py:73-337) for trees of up to 64 nodes."""

    def __init__(self, num_heads: int = 4, max_branches: int = 4, draft_cost_c: float = 0.02,
                 max_budget: int = 32, latency_profile: dict[int, float] | None = None):
        self.num_heads = int(num_heads)
        self.max_branches = int(max_branches)
        self.draft_cost_c = float(draft_cost_c)
        self.max_budget = min(int(max_budget), MAX_TREE_NODES)
        profile = MI355X_7B_Q4_TREE_LATENCY if latency_profile is None else latency_profile
        self.t_hardware = interpolate_hardware_latency(profile, max_N=self.max_budget)
        self.P = _default_acceptance(self.num_heads, self.max_branches)

    def set_hardware_latency(self, t_profile) -> None:
        """t(N) from a dict {N: t} or a list [t(1), t(2), ...] (sequoia_dp.py:116-126)."""
        if isinstance(t_profile, (list, tuple)):
            t_dict = {i + 1: float(v) for i, v in enumerate(t_profile)}
        else:
            t_dict = {int(k): float(v) for k, v in t_profile.items()}
        self.t_hardware = interpolate_hardware_latency(t_dict, max_N=self.max_budget)

    def set_acceptance_probabilities(self, P) -> None:
        """P as [num_heads, max_branches], or one row [max_branches] scaled by 0.85^d per
        head (sequoia_dp.py:128-145)."""
        arr = np.array(P, dtype=np.float64)
        if arr.ndim == 1:
            self.max_branches = len(arr)
            self.P = np.stack([arr * (0.85 ** d) for d in range(self.num_heads)]).astype(np.float64)
        elif arr.ndim == 2:
            self.num_heads, self.max_branches = int(arr.shape[0]), int(arr.shape[1])
            self.P = arr
        else:
            raise ValueError(f"Expected 1D or 2D array for P, got shape {arr.shape}")

    def solve_dp_tables(self) -> tuple[np.ndarray, np.ndarray]:
        """T[n, d, b]: the largest expected number of accepted tokens of a subtree of at most
        n nodes whose root sits at depth d and whose children are among candidates
        0..b-1; split[n, d, b]: nodes given to candidate b-1's subtree (0: none)
        (sequoia_dp.py:147-197).

            T[n, d, b] = max(T[n, d, b-1],
                             max_{1 <= m < n} T[n-m, d, b-1] + P[d, b-1] * max_j T[m, d+1, j])

        with T = 1 for a lone root (n = 1, b = 0 or d = num_heads).  The inner maximum runs
        over all m at once; the smallest maximizing m wins, and candidate b-1 is used only
        when it strictly improves on leaving it out."""
        N, D, B = self.max_budget, self.num_heads, self.max_branches
        T = np.zeros((N + 1, D + 1, B + 1), dtype=np.float64)
        split = np.zeros((N + 1, D + 1, B + 1), dtype=np.int32)
        T[1:, :, 0] = 1.0
        T[1, :, :] = 1.0
        T[1:, D, :] = 1.0
        best_sub = np.zeros((N + 1, D + 1), dtype=np.float64)  # max_j T[m, d, j], final once m < n
        best_sub[1, :] = T[1, :, :].max(axis=1)
        for n in range(2, N + 1):
            m = np.arange(1, n)
            for d in range(D - 1, -1, -1):
                sub = best_sub[m, d + 1]
                for b in range(1, B + 1):
                    vals = T[n - m, d, b - 1] + float(self.P[d, b - 1]) * sub
                    k = int(np.argmax(vals))
                    if vals[k] > T[n, d, b - 1]:
                        T[n, d, b] = vals[k]
                        split[n, d, b] = k + 1
                    else:
                        T[n, d, b] = T[n, d, b - 1]
            best_sub[n, :] = T[n, :, :].max(axis=1)
        return T, split

    def _reconstruct(self, T, split, n, d, b, path, out) -> None:
        """Candidates b-1, b-2, ... of the node at `path` from the split table (the lower
        candidates first, then candidate b-1 and its own subtree; sequoia_dp.py:199-231)."""
        while n > 1 and b > 0 and d < self.num_heads:
            m = int(split[n, d, b])
            self._reconstruct(T, split, n - m, d, b - 1, path, out)
            if m == 0:
                return
            child = path + (b - 1,)
            out.append(child)
            n, d, b, path = m, d + 1, int(np.argmax(T[m, d + 1, :])), child

    def extract_tree_for_budget(self, n: int, T: np.ndarray, split: np.ndarray) -> list[tuple[int, ...]]:
        """Draft paths (candidate ranks from the root) of the best tree of at most n nodes
        (sequoia_dp.py:233-246)."""
        if n <= 1:
            return []
        out: list[tuple[int, ...]] = []
        self._reconstruct(T, split, n, 0, int(np.argmax(T[n, 0, :])), (), out)
        return out

    def solve_optimal_tree(self, max_tree_size: int | None = None) -> OptimalTreeResult:
        """The budget N <= max_tree_size with the largest speedup G(N) / (t(N) + depth * c)
        (the first one on ties) and its tree (sequoia_dp.py:248-310)."""
        limit = min(max_tree_size or self.max_budget, self.max_budget)
        T, split = self.solve_dp_tables()
        best_speedup, best_N, best_choices = 0.0, 1, []
        stats: dict[int, dict[str, float]] = {}
        for n in range(1, limit + 1):
            G = float(np.max(T[n, 0, :]))
            t = self.t_hardware.get(n, 1.0)
            choices = self.extract_tree_for_budget(n, T, split)
            depth = max((len(p) for p in choices), default=0)
            draft = depth * self.draft_cost_c
            lat = t + draft
            sp = G / lat
            stats[n] = {"N": float(n), "expected_tokens": round(G, 4), "verification_t": round(t, 4),
                        "draft_cost": round(draft, 4), "effective_latency": round(lat, 4), "speedup": round(sp, 4)}
            if sp > best_speedup:
                best_speedup, best_N, best_choices = sp, n, choices
        compiled = compile_medusa_tree(best_choices, self.num_heads, max_nodes=self.max_budget)
        s = stats[best_N]
        return OptimalTreeResult(best_N, compiled["max_depth"], s["expected_tokens"], s["verification_t"],
                                 s["draft_cost"], s["speedup"], best_choices, compiled, stats)

    def solve_fixed_budget(self, N: int) -> OptimalTreeResult:
        """The best tree of at most N nodes (sequoia_dp.py:312-337)."""
        N = min(max(1, int(N)), self.max_budget)
        T, split = self.solve_dp_tables()
        choices = self.extract_tree_for_budget(N, T, split)
        compiled = compile_medusa_tree(choices, self.num_heads, max_nodes=self.max_budget)
        G = float(np.max(T[N, 0, :]))
        t = self.t_hardware.get(N, 1.0)
        draft = compiled["max_depth"] * self.draft_cost_c
        return OptimalTreeResult(N, compiled["max_depth"], round(G, 4), round(t, 4), round(draft, 4),
                                 round(G / (t + draft), 4), choices, compiled, {})


def measure_tree_latency(runner, cache, budgets=(2, 4, 8, 16, 32, 48, 64), reps: int = 20,
                         warmup: int = 3) -> dict[int, float]:
    """t(N) of this runner on this GPU: the average time of ``verify_tree_step`` over a
    branching tree of N nodes divided by that of a one-token ``step``, both at the cache's
    current prefix (``total_seen_tokens``), which is left unchanged (the verified slots
    lie past it); each is the median of three timed runs of ``reps`` calls.  Feed the result to :meth:`SequoiaDPOptimizer.set_hardware_latency`."""
    import torch

    from .tree import build_branching_tree

    dev = runner.device
    if cache.ring_buffer:
        raise ValueError("measure_tree_latency: needs a monotonic (non-ring) cache")
    seen = int(cache.total_seen_tokens[0])
    if seen + max(budgets) > cache.max_seq_len:
        raise ValueError("measure_tree_latency: the cache has no room for the largest tree")

    def timed(fn) -> float:
        for _ in range(warmup):
            fn()
        trials = []
        for _ in range(3):
            torch.cuda.synchronize(dev)
            t0 = time.perf_counter()
            for _ in range(reps):
                fn()
            torch.cuda.synchronize(dev)
            trials.append((time.perf_counter() - t0) / reps)
        return sorted(trials)[1]  # median of three

    tok = torch.zeros((1, 1), dtype=torch.int64, device=dev)
    base = timed(lambda: runner.step(tok, seen, seen, seen + 1))
    out = {1: 1.0}
    for n in budgets:
        tree = build_branching_tree((4, 4, 2, 2, 1, 1, 1, 1), max_nodes=int(n))
        ids = torch.zeros((1, int(n)), dtype=torch.int64, device=dev)
        t = timed(lambda: runner.verify_tree_step(ids, seen, seen, seen, tree["tree_depths"], tree["tree_mask"]))
        out[int(n)] = round(t / base, 4)
    return out
