"""Allocation and leak invariants of the runner (the reference checks them for its
single-command-buffer runner: zero dynamic allocation over 20 steps and over tree
verification, tests/test_phase1_task14_single_command_buffer.py:84-134, and bounded
process RSS over 300 decode steps, tests/test_memory_leak_and_stress.py:41-154).

Every buffer of a step, a verify chain and a tree verification is allocated when the
runner is built; the captured graphs are made on the first call of each split bucket.
After one warm-up pass over the same positions, a second pass must leave the device's
free memory (hipMemGetInfo) and torch's allocator statistics unchanged, and a 300-step
greedy loop must not grow the process's resident set by 2 MB or more.
"""

import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _rss_mb() -> float:
    with open(f"/proc/{os.getpid()}/status") as f:
        for line in f:
            if line.startswith("VmRSS:"):
                return int(line.split()[1]) / 1024.0
    raise RuntimeError("VmRSS not found")


def _c1_runner(dev, mode="graph"):
    from test_gpu_runner import build_runner, c1_model

    cfg, ow, cos, sin = c1_model()
    runner, cache = build_runner(cfg, ow, cos, sin, dev, 512, "fp16", mode=mode)
    return cfg, runner, cache


def test_step_verify_and_tree_verify_allocate_nothing(dev):
    """20 decode steps, a 4-token verify chain and an 8-node tree verification: no device
    memory taken (hipMemGetInfo) and torch's allocator unchanged, after a warm-up pass."""
    print("[zero_alloc] C1 model", flush=True)
    cfg, runner, cache = _c1_runner(dev)
    idx = torch.tensor([[12]], device=dev, dtype=torch.int64)
    chain = torch.tensor([[3, 1, 4, 1]], device=dev, dtype=torch.int64)
    T = 8
    tree = torch.tensor([np.random.default_rng(0).integers(0, cfg.vocab, T).tolist()], device=dev,
                        dtype=torch.int64)
    depths = list(range(T))
    masks = [(1 << (i + 1)) - 1 for i in range(T)]

    def one_pass():
        for step in range(20):
            runner.step(idx, step, step, step + 1)
        runner.verify_step(chain, 20, 20, 24)
        runner.verify_tree_step(tree, 24, 24, 24, depths, masks)
        torch.cuda.synchronize()

    one_pass()
    free0, _ = torch.cuda.mem_get_info(dev)
    alloc0, res0 = torch.cuda.memory_allocated(dev), torch.cuda.memory_reserved(dev)
    one_pass()
    free1, _ = torch.cuda.mem_get_info(dev)
    alloc1, res1 = torch.cuda.memory_allocated(dev), torch.cuda.memory_reserved(dev)
    print(f"[zero_alloc] free {free0} -> {free1}, allocated {alloc0} -> {alloc1}, reserved {res0} -> {res1}",
          flush=True)
    assert (alloc1, res1) == (alloc0, res0)
    assert free1 == free0


def test_300_greedy_steps_keep_rss_flat(dev):
    """300 device-fed greedy steps: resident set growth < 2 MB.  A warm-up pass over the
    same positions first makes the graphs of every split bucket those positions use."""
    import gc

    print("[rss] C1 model", flush=True)
    cfg, runner, cache = _c1_runner(dev)

    def greedy_pass():
        runner.step(torch.tensor([[10]], device=dev, dtype=torch.int64), 0, 0, 1)
        for p in range(1, 301):
            runner.step_greedy(p, p, p + 1)
        torch.cuda.synchronize()

    greedy_pass()
    gc.collect()
    base = _rss_mb()
    greedy_pass()
    gc.collect()
    grown = _rss_mb() - base
    print(f"[rss] growth over 300 steps: {grown:.3f} MB", flush=True)
    assert grown < 2.0
