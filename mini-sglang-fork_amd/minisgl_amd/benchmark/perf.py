"""Kernel timing in the manner of the reference's perf_cuda
(python/minisgl/benchmark/perf.py:10-51): capture N calls in a HIP graph,
replay it R times between two events on the same stream, return the mean
time of one call in ms."""

from __future__ import annotations

from typing import Any, Callable

import torch


def perf_hip(
    f: Callable[[], Any],
    *,
    repetitions: int = 10,
    graph_calls: int = 10,
    warmup: int = 2,
) -> float:
    assert repetitions > 0 and graph_calls > 0
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        f()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for _ in range(graph_calls):
                f()
        for _ in range(warmup):
            g.replay()
        tic = torch.cuda.Event(enable_timing=True)
        toc = torch.cuda.Event(enable_timing=True)
        tic.record(stream)
        for _ in range(repetitions):
            g.replay()
        toc.record(stream)
        toc.synchronize()
    return tic.elapsed_time(toc) / (graph_calls * repetitions)
