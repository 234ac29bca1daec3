"""GPU parity of the stream executor (kernels.decode_stack.StreamStack; csrc/stream_exec.hip).

The same chains as the first executor's tests (tests/test_gpu_decode_stack.py): chained
projections read what earlier ones of the same launch published, inputs change between runs
(a stale read of an earlier run would show), every output is checked against the single-call
linear on the executor's own input to within one bf16 rounding step (its fp32 sums are four
K-interleaved partials added in wave order), against the CPU oracle to the north star's
relative L2 bound, and for determinism.
"""

import pytest
import torch

from kernels import qlinear
from kernels.decode_stack import StreamStack
from test_gpu_decode_stack import CHAIN, DEV, QWEN_LAYER, bits16, check_against_single_calls, oracle_check, rand, \
    source

pytestmark = pytest.mark.gpu


def build_stream(fmt, m, seed, chain_def=None):
    quant = qlinear.FORMATS[fmt][0]
    bufs = {"x": rand((m, 1024), seed).to(DEV), "g": rand((m, 9728), seed + 1).to(DEV),
            "x2560": rand((m, 2560), seed + 2).to(DEV)}
    weights, raw = {}, {}
    chain = StreamStack(fmt, m)
    for idx, (name, n, k, src, sw) in enumerate(chain_def or CHAIN):
        w = rand((n, k), seed + 10 + idx, std=0.02).to(DEV)
        packed = quant(w)
        raw[name] = packed
        weights[name] = qlinear.prepare(packed)
        bufs[name] = torch.empty((m, n // 2 if sw else n), dtype=torch.bfloat16, device=DEV)
        chain.add(weights[name], source(bufs, src), bufs[name], swiglu=sw)
    chain.build()
    return chain, bufs, weights, raw


@pytest.mark.parametrize("fmt,m", [("w4a16", 1), ("w8a16", 1), ("fp8", 1), ("fp8", 2)])
def test_stream_chain_matches_single_calls_and_oracle(fmt, m):
    print(f"stream exec {fmt} m={m}", flush=True)
    chain, bufs, weights, raw = build_stream(fmt, m, 100 * m + 3)
    assert chain.grid >= 256 and chain.launch.ring_lines >= 8
    for run in range(3):
        if run:
            bufs["x"].copy_(rand((m, 1024), 7 * run + m).to(DEV))
            bufs["g"].copy_(rand((m, 9728), 9 * run + m).to(DEV))
        chain.run()
        torch.cuda.synchronize()
        assert not chain.failed(), chain.failed_waits()
        first = {name: bufs[name].clone() for name, *_ in CHAIN}
        chain.run()
        torch.cuda.synchronize()
        assert not chain.failed(), chain.failed_waits()
        for name, *_ in CHAIN:
            assert torch.equal(bufs[name], first[name]), (fmt, m, run, name, "deterministic")
        check_against_single_calls(fmt, bufs, weights, ("stream", fmt, m, run))
    for name in ("c2", "d", "e", "i"):
        src = [c for c in CHAIN if c[0] == name][0][3]
        assert oracle_check(fmt, bits16(source(bufs, src)), raw[name], bufs[name]) < 1e-2, name


@pytest.mark.parametrize("fmt", ["w4a16", "w8a16", "fp8"])
def test_stream_layer_chain(fmt):
    """A Qwen3-4B layer at M = 1 through the stream executor."""
    print(f"stream exec layer {fmt}", flush=True)
    chain, bufs, weights, raw = build_stream(fmt, 1, 31, chain_def=QWEN_LAYER)
    for run in range(2):
        if run:
            bufs["x2560"].copy_(rand((1, 2560), 99).to(DEV))
        chain.run()
        torch.cuda.synchronize()
        assert not chain.failed(), chain.failed_waits()
        check_against_single_calls(fmt, bufs, weights, ("stream layer", fmt, run), chain_def=QWEN_LAYER)
    for name in ("o", "dn"):
        src = [c for c in QWEN_LAYER if c[0] == name][0][3]
        assert oracle_check(fmt, bits16(source(bufs, src)), raw[name], bufs[name]) < 1e-2, name


def test_stream_bounded_wait_gives_up_and_recovers():
    """A zero wait budget makes the waits give up (forced from the host): the kernel still ends
    and flags the run; after reset() a normal run is right again."""
    print("stream exec bounded wait", flush=True)
    chain, bufs, weights, _ = build_stream("fp8", 1, 55)
    chain.run(budget_us=0)
    torch.cuda.synchronize()
    assert chain.failed()
    chain.reset()
    chain.run()
    torch.cuda.synchronize()
    assert not chain.failed()
    check_against_single_calls("fp8", bufs, weights, "stream after reset")
