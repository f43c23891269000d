"""HIP graph capture of a launch sequence (the correction pass), replayed with one launch.

The reference's serving path can wrap the correction step in torch.compile (config correct_compile,
dinov3_precision.py:172-629); here the equivalent is recording the pass into a HIP graph: every
kernel of the pass is a library launch on torch's current stream, none allocates, copies from the
host or synchronises, so the whole sequence records and replays as is. A replay redoes exactly the
recorded work on the recorded tensors (the usual graph contract: refresh inputs in place).

Scratch memory: the library's split-K partials and attention key parts live in a buffer per
(device, stream) (kernels._stream_workspace). Each graph is recorded on a stream of its own, warmed
up on that same stream (so its scratch is allocated before recording), and then takes that stream's
buffers out of the shared table: the graph owns the scratch its kernels point at, and two graphs
may replay at the same time on different streams. One graph must not be replayed concurrently with
itself (its replays share its tensors and its scratch).
"""

from __future__ import annotations

from typing import Callable

import torch

from . import kernels as K


def capture(fn: Callable[[], object], device: torch.device | int | None = None, warmup: int = 2) -> Callable[[], None]:
    """Run `fn` `warmup` times on a new stream (first-use work: tables, kernel attributes, allocator
    pools, scratch), then record one call on that stream into a graph; returns the graph's replay
    function, which keeps the graph, its stream and its scratch buffers alive."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    stream = torch.cuda.Stream(device=dev)  # default priority
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        for _ in range(max(1, warmup)):
            fn()
    torch.cuda.current_stream(dev).wait_stream(stream)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        fn()
    torch.cuda.synchronize(dev)
    scratch = K.take_stream_workspaces(dev, stream.cuda_stream)

    def replay() -> None:
        graph.replay()

    replay.graph = graph  # the graph (and its memory pool) lives as long as the function
    replay.stream = stream
    replay.scratch = scratch
    return replay
