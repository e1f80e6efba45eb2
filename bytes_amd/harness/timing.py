"""Graph-replay timing shared by the harnesses (benchmarks/timing.py:6-24).

`graph_ms(fn, inputs)` warms `fn` up, captures `runs` calls in one HIP graph
(call i on inputs[i % len(inputs)]) and returns the mean milliseconds per
call over one event-timed replay.  Pass several input copies whose total size
exceeds the Infinity Cache (`copies_for`) so that no call is served from it.
"""
from __future__ import annotations

import math
from typing import Callable, Sequence

import torch

MALL_BYTES = 256 << 20          # MI355X Infinity Cache
HBM_PEAK_GBS = 8000.0           # MI355X HBM3E peak


def copies_for(nbytes: int) -> int:
    """Input copies so that consecutive calls never find their bytes in the cache."""
    return max(1, math.ceil(2 * MALL_BYTES / max(nbytes, 1)) + 1) if nbytes < 2 * MALL_BYTES else 1


def graph_ms(fn: Callable, inputs: Sequence, warmup: int = 10, runs: int = 100) -> float:
    for i in range(warmup):
        fn(inputs[i % len(inputs)])
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(runs):
            fn(inputs[i % len(inputs)])
    torch.cuda.synchronize()
    g.replay()                                  # uploads the graph
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    del g
    return e0.elapsed_time(e1) / runs


def clones(x: dict, n: int) -> list:
    out = [x]
    for _ in range(n - 1):
        out.append({k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in x.items()})
    return out
