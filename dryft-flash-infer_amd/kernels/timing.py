"""Warmup-time measurement in the execution mode decode uses (engine/kernels/timing.py:9-52).

``time_calls`` is the reference's contract: median milliseconds per call over ``trials``,
each a sweep of ``reps`` passes over every operand (distinct layer weights, so that a
projection whose weight would fit the 256 MB Infinity Cache is not timed hot), captured
in one HIP graph when ``use_graph`` -- so host launch overhead cannot decide a race between
kernels that will run inside the decode graph.
"""

import statistics

import torch


@torch.no_grad()
def time_calls(fn, operands, *, reps=3, trials=5, use_graph=True):
    """Median milliseconds per ``fn(operand)`` call, cycling through ``operands``."""
    if not operands or reps < 1 or trials < 1:
        raise ValueError("timing needs operands and positive repeat counts")

    def sweep():
        for _ in range(reps):
            for operand in operands:
                fn(operand)

    if use_graph:
        # Warm up outside the capture: first calls allocate (outputs' pool, split-K tickets).
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            for operand in operands[:4]:
                fn(operand)
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            sweep()
        for _ in range(2):
            graph.replay()
        run = graph.replay
    else:
        for operand in operands[:4]:
            fn(operand)
        run = sweep

    torch.cuda.synchronize()
    start, end = (torch.cuda.Event(enable_timing=True) for _ in range(2))
    times = []
    for _ in range(trials):
        start.record()
        run()
        end.record()
        end.synchronize()
        times.append(start.elapsed_time(end) / (reps * len(operands)))
    return statistics.median(times)
