"""Warmup-time clock for decode kernels on MI355X.

``time_calls(fn, operands, *, reps=3, trials=5, use_graph=True)`` keeps the contract of
engine/kernels/timing.py:9-52 -- the median milliseconds of one ``fn(operand)`` call
while cycling through ``operands`` -- and is built around two facts of this GPU:

* **The 256 MB Infinity Cache.** A decode step streams 2-4 GB of distinct weights, so no
  projection finds its weight in a cache. A rotation whose operands occupy less than
  ``ROTATION_BYTES`` (1 GiB, four times the cache) is therefore extended with device copies
  of the operands until it does; cycling 36 layers is not enough here (36 W4 qkv weights
  are 292 MB).
* **Launch cost.** One sweep (``reps`` passes over the rotation) is captured into a HIP
  graph and replayed, so host-side launch overhead does not decide a race between kernels
  that run inside the decode graph. All ``trials`` replays are queued back to back behind
  one leading event, each followed by its own event; the host synchronises once.
"""

import copy
import math
import statistics

import torch

#: Bytes a timing rotation must cover so that the Infinity Cache cannot serve it hot.
ROTATION_BYTES = 1 << 30
#: Most calls one sweep of the rotation may take (tiny operands stop growing there).
MAX_ROTATION_CALLS = 2048


def footprint(operand) -> int:
    """Bytes of distinct device storage reachable from ``operand`` (tensors inside tuples,
    lists, dicts and objects' attributes; each storage counted once)."""
    seen, total, stack = set(), 0, [operand]
    while stack:
        obj = stack.pop()
        if isinstance(obj, torch.Tensor):
            key = (obj.device, obj.untyped_storage().data_ptr())
            if obj.device.type == "cuda" and key not in seen:
                seen.add(key)
                total += obj.untyped_storage().nbytes()
        elif isinstance(obj, (tuple, list)):
            stack.extend(obj)
        elif isinstance(obj, dict):
            stack.extend(obj.values())
        elif hasattr(obj, "__dict__") or hasattr(type(obj), "__slots__"):
            stack.extend(vars(obj).values() if hasattr(obj, "__dict__") else ())
            for name in getattr(type(obj), "__slots__", ()):
                if hasattr(obj, name):
                    stack.append(getattr(obj, name))
    return total


def rotation(operands, min_bytes=ROTATION_BYTES, max_calls=MAX_ROTATION_CALLS):
    """``operands`` followed by as many deep copies of the whole list as it takes to cover
    ``min_bytes`` of device memory (at most ``max_calls`` operands in all)."""
    ops = list(operands)
    size = sum(footprint(op) for op in ops)
    if size <= 0 or size >= min_bytes:
        return ops
    copies = min(math.ceil(min_bytes / size) - 1, max_calls // len(ops) - 1)
    for _ in range(max(copies, 0)):
        ops.extend(copy.deepcopy(op) for op in operands)
    return ops


@torch.no_grad()
def time_calls(fn, operands, *, reps=3, trials=5, use_graph=True):
    """Median milliseconds per ``fn(operand)`` call over a cache-defeating rotation."""
    if not operands or reps < 1 or trials < 1:
        raise ValueError("timing needs operands and positive repeat counts")
    ops = rotation(operands)

    def sweep():
        for _ in range(reps):
            for op in ops:
                fn(op)

    # One eager pass first: lazily created state (output allocations, split-K ticket
    # buffers, first-call kernel attributes) must exist before a capture.
    for op in ops:
        fn(op)
    torch.cuda.synchronize()
    run = sweep
    if use_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            sweep()
        graph.replay()  # the first replay uploads the graph
        torch.cuda.synchronize()
        run = graph.replay

    marks = [torch.cuda.Event(enable_timing=True) for _ in range(trials + 1)]
    marks[0].record()
    for i in range(trials):
        run()
        marks[i + 1].record()
    marks[-1].synchronize()
    calls = reps * len(ops)
    return statistics.median(marks[i].elapsed_time(marks[i + 1]) / calls for i in range(trials))
