"""HIP graph capture of a launch sequence (the correction pass), replayed with one launch.

The reference's serving path can wrap the correction step in torch.compile (config correct_compile,
dinov3_precision.py:172-629); here the equivalent is recording the pass into a HIP graph: every
kernel of the pass is a library launch on torch's current stream, none allocates, copies from the
host or synchronises, so the whole sequence records and replays as is. A replay redoes exactly the
recorded work on the recorded tensors (the usual graph contract: refresh inputs in place).
"""

from __future__ import annotations

from typing import Callable

import torch


def capture(fn: Callable[[], object], device: torch.device | int | None = None, warmup: int = 2) -> Callable[[], None]:
    """Run `fn` `warmup` times on a side stream (first-use work: tables, kernel attributes, allocator
    pools), then record one call into a graph; returns the graph's replay function."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    side = torch.cuda.Stream(device=dev)  # default priority
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for _ in range(max(1, warmup)):
            fn()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    torch.cuda.synchronize(dev)
    def replay() -> None:
        graph.replay()

    replay.graph = graph  # the graph (and its memory pool) lives as long as the function
    return replay
