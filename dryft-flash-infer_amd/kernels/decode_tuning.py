"""Warmup-time selection inside the captured decode step: drop-in for the reference's
``kernels.decode_tuning`` (engine/kernels/decode_tuning.py:17-79).

The reference races its output projection's split-K schedules with the whole decode step
captured, because a race of the projection alone misses how the schedules interact with the
launches around them and with the plane consumer. The contract kept here: the candidates are
the incumbent and a few split-K schedules; each is captured as a whole decode step; the
incumbent stays unless another is faster by a clear margin, consistently; the engine's
``partial_config["o"]`` and ``matmul["o"]`` then carry the winner and its position and token are
as before; ``tune_output_projection(engine)`` returns whether it changed anything.

Both races here run on one primitive, ``race_steps``: one HIP graph per candidate step, replayed
in rounds whose order is a fresh random permutation each round, every candidate's time in a
round compared with the incumbent's time in the same round. ``race_steps`` also chooses between
whole-step paths, such as the decode executor and a graph of single calls.
"""

import functools
import random
import statistics
import sys

import torch

from . import cuda_fp8

#: Split-K counts tried for the output projection (K = 4096: 32 groups of 128), each with the
#: incumbent's other config fields.
O_SPLITS = (1, 2, 4, 8, 16)


@torch.no_grad()
def race_steps(steps, incumbent, rounds=9, replays=10, margin=0.01, agreement=0.75, seed=0):
    """Race whole steps: ``steps`` maps a name to a callable that runs one step on the current
    stream and can be captured (it may also set the state it is captured with). Each step runs
    once eagerly on a side stream, is captured once, and its graph is replayed ``replays``
    times per round between two events. Returns ``(winner, median ms per step by name)``: the
    fastest by median, if it is faster than ``incumbent`` by ``margin`` and beat it in at least
    ``agreement`` of the rounds; else ``incumbent``."""
    if incumbent not in steps:
        raise ValueError("the incumbent must be one of the steps")
    names = list(steps)
    graphs = {}
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for name in names:
            steps[name]()
    side.synchronize()
    for name in names:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            steps[name]()
        graphs[name] = graph
    torch.cuda.synchronize()
    for name in names:  # uploads each graph once before anything is timed
        graphs[name].replay()
    torch.cuda.synchronize()
    rng = random.Random(seed)
    per_round = {name: [] for name in names}
    for _ in range(rounds):
        order = names[:]
        rng.shuffle(order)
        marks = {name: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                 for name in order}
        for name in order:
            start, end = marks[name]
            start.record()
            for _ in range(replays):
                graphs[name].replay()
            end.record()
        torch.cuda.synchronize()
        for name in order:
            start, end = marks[name]
            per_round[name].append(start.elapsed_time(end) / replays)
    medians = {name: statistics.median(v) for name, v in per_round.items()}
    best = min(names, key=medians.get)
    if best != incumbent:
        beat = sum(b < i for b, i in zip(per_round[best], per_round[incumbent]))
        if medians[best] > (1.0 - margin) * medians[incumbent] or beat < agreement * rounds:
            best = incumbent
    return best, medians


@torch.no_grad()
def tune_output_projection(engine, candidates=None):
    """Race the output projection's split-K schedules inside the whole captured decode step
    (the reference's conditions: a captured graph, no drafting, at most 16 rows, no integer MLP,
    the FP8 family and a split-K config for o). Returns True when the schedule changed."""
    if (engine.graph is None or engine.draft or engine.batch > 16 or engine.integer_mlp
            or engine.families.get("o") != "fp8" or "o" not in engine.partial_config):
        return False
    incumbent = tuple(engine.partial_config["o"])
    if candidates is None:
        candidates = [incumbent] + [(incumbent[0], s) + incumbent[2:] for s in O_SPLITS]
    candidates = list(dict.fromkeys(tuple(c) for c in candidates))
    if incumbent not in candidates:
        candidates.insert(0, incumbent)
    position, token = engine.pos.clone(), engine.token.clone()

    def step_with(config):
        def step():
            engine.partial_config["o"] = config  # read while the step is traced and captured
            engine._decode_step()
            engine.pos.copy_(position)
            engine.token.copy_(token)
        return step

    try:
        best, medians = race_steps({c: step_with(c) for c in candidates}, incumbent)
    except Exception:
        engine.partial_config["o"] = incumbent
        raise
    finally:
        engine.pos.copy_(position)
        engine.token.copy_(token)
        torch.cuda.synchronize()
    engine.partial_config["o"] = best
    if best != incumbent:
        engine.matmul["o"] = functools.partial(cuda_fp8.matmul, config=best)
        engine._ordinary_matmul = dict(engine.matmul)
    print(f"engine: o split-K schedule at batch {engine.batch}: {best} "
          f"({medians[best]:.4f} ms per step; incumbent {incumbent}: {medians[incumbent]:.4f} ms)", file=sys.stderr)
    return best != incumbent
