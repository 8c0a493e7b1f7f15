"""Tree speculative decoding at temperature 0 over the MI355X runner.

The loop of axiomlm/engine/medusa.py:278-363 (the ``use_tree`` branch with
greedy acceptance): every iteration verifies one draft tree whose root is the
last emitted token (not yet in the cache) in a single ``verify_tree_step``,
takes the model's greedy token at every node, walks the tree from the root
while a child carries the predicted token (medusa.py:313-330), emits the
predictions along that path, and compacts the accepted nodes' KV slots to
the contiguous tail of the cache with ``StaticKVCache.compact_tree_path``
(paged_cache.py:376-462).  The drafter that proposes node tokens (Medusa heads
in the reference) is a caller-supplied function.
"""

from __future__ import annotations

import time
from typing import Callable, Sequence

import torch

from .kernels.ops import argmax_last_token
from .tree import greedy_tree_walk


def tree_decode_greedy(runner, cache, last_token: int, tree: dict, draft: Callable[[int, int, int], Sequence[int]],
                       n_steps: int, max_new_tokens: int | None = None,
                       on_verify: Callable[..., None] | None = None) -> dict:
    """Run up to ``n_steps`` tree verifications.

    runner: ``QuantizedDecodeRunner``; cache: its ``StaticKVCache`` (``total_seen_tokens``
    holds the committed prefix length); tree: topology with ``num_nodes``, ``tree_depths``,
    ``tree_mask`` and ``children`` (``compile_medusa_tree``, ``build_branching_tree``,
    ``sequoia.SequoiaDPOptimizer``); draft(step, root_token, seen) -> tokens of nodes
    1..T-1.  ``on_verify(step, seen, nodes, logits, preds, accepted, emitted)`` is called
    after the walk and before the compaction (logits is the runner's (1, T, V) view).

    Returns {"tokens": emitted tokens, "accepted": accepted draft nodes per step,
    "model_calls", "drafted", "seconds"} (the counters of medusa.py:291-295, 343-345)."""
    T = int(tree["num_nodes"])
    depths = [int(d) for d in tree["tree_depths"]]
    masks = [int(m) for m in tree["tree_mask"]]
    children = tree["children"]
    max_depth = max(depths)
    rope_len = runner.rope_len
    emitted_all: list[int] = []
    accepted_per_step: list[int] = []
    drafted = 0
    calls = 0
    limit = max_new_tokens if max_new_tokens is not None else n_steps * (max_depth + 1)
    dev = runner.device
    last = int(last_token)
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for step in range(n_steps):
        if len(emitted_all) >= limit:
            break
        seen = int(cache.total_seen_tokens[0])
        if seen + T > cache.max_seq_len:
            raise RuntimeError(f"tree verification needs {T} free slots after {seen} (cache of {cache.max_seq_len})")
        nodes = [last] + [int(t) for t in draft(step, last, seen)]
        if len(nodes) != T:
            raise ValueError(f"draft returned {len(nodes) - 1} tokens for a {T}-node tree")
        idx = torch.tensor([nodes], dtype=torch.int64).to(dev, non_blocking=True)
        logits = runner.verify_tree_step(idx, seen % rope_len, seen, seen, depths, masks)
        calls += 1
        drafted += min(max_depth, limit - len(emitted_all))
        preds = argmax_last_token(logits[0]).tolist()
        accepted, emitted = greedy_tree_walk(preds, nodes, children, limit - len(emitted_all))
        if on_verify is not None:
            on_verify(step, seen, nodes, logits, preds, accepted, emitted)
        cache.compact_tree_path(seen, accepted, seen + len(accepted))
        emitted_all.extend(emitted)
        accepted_per_step.append(len(accepted) - 1)
        last = emitted[-1]
    torch.cuda.synchronize(dev)
    return {"tokens": emitted_all, "accepted": accepted_per_step, "model_calls": calls, "drafted": drafted,
            "seconds": time.perf_counter() - t0}
