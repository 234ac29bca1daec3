"""GPU parity of the decode-step executor (one cooperative launch for a chain of projections).

Every output of the chain must equal, bit for bit, the single-call linear run with the plan
the executor chose (``DecodeStack.configs``), fed with the same inputs -- including
projections that read what an earlier projection of the same launch wrote. The single-call
linears are themselves checked against the CPU oracle (test_gpu_qlinear.py); one projection
per format is checked against the oracle here as well. Inputs change between runs, so a
stale read of an earlier run's intermediate would show.
"""

import numpy as np
import pytest
import torch

import oracle as O
from kernels import qlinear
from kernels.decode_stack import DecodeStack

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def bits16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def rand(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)


# (name, n, k, input, swiglu): a layer-like chain where later projections consume earlier
# outputs, plus a tiny projection (fewer work items than workgroups) and a long-K one.
CHAIN = [
    ("a", 2048, 1024, "x", False),
    ("b", 3072, 2048, "a", True),      # SwiGLU: out 1536
    ("c", 1024, 1536, "b", False),
    ("d", 4096, 1024, "c", False),
    ("e", 16, 4096, "d", False),
    ("f", 1024, 9728, "g", False),     # reads an input the host writes
    ("h", 9728 * 2, 1024, "f", True),  # SwiGLU: out 9728
    ("i", 1024, 9728, "h", False),
]


def build_chain(fmt, m, seed):
    quant = qlinear.FORMATS[fmt][0]
    bufs = {"x": rand((m, 1024), seed).to(DEV), "g": rand((m, 9728), seed + 1).to(DEV)}
    weights, raw = {}, {}
    chain = DecodeStack(fmt, m)
    for idx, (name, n, k, src, sw) in enumerate(CHAIN):
        w = rand((n, k), seed + 10 + idx, std=0.02).to(DEV)
        packed = quant(w)
        raw[name] = packed
        weights[name] = qlinear.prepare(packed)
        bufs[name] = torch.empty((m, n // 2 if sw else n), dtype=torch.bfloat16, device=DEV)
        chain.add(weights[name], bufs[src], bufs[name], swiglu=sw)
    chain.build()
    return chain, bufs, weights, raw


def single_calls(fmt, chain, bufs, weights):
    linear = qlinear.FORMATS[fmt][1]
    out = {"x": bufs["x"], "g": bufs["g"]}
    for (name, n, k, src, sw), cfg in zip(CHAIN, chain.configs):
        out[name] = linear(out[src], weights[name], config=cfg, swiglu=sw)
    return out


@pytest.mark.parametrize("fmt", ["w4a16", "w8a16", "fp8"])
@pytest.mark.parametrize("m", [1, 5, 16])
def test_chain_matches_single_calls_bitwise(fmt, m):
    print(f"decode stack {fmt} m={m}", flush=True)
    chain, bufs, weights, raw = build_chain(fmt, m, 100 * m)
    assert chain.grid >= 256 and chain.lds > 0
    for run in range(3):
        if run:
            bufs["x"].copy_(rand((m, 1024), 7 * run + m).to(DEV))
            bufs["g"].copy_(rand((m, 9728), 9 * run + m).to(DEV))
        chain.run()
        want = single_calls(fmt, chain, bufs, weights)
        torch.cuda.synchronize()
        assert not chain.failed()
        assert chain.sync[:2].tolist() == [0, 0], "the last workgroup resets the counters"
        for name, *_ in CHAIN:
            assert torch.equal(bufs[name], want[name]), (fmt, m, run, name, chain.configs)
    # One projection against the oracle (the dequantize-then-matmul statement).
    x = bits16(bufs["c"])
    if fmt == "fp8":
        q, s = raw["d"]
        ref = O.linear_fp8_w8a8(x, q.view(torch.uint8).cpu().numpy(), bits16(s))
    elif fmt == "w8a16":
        q, s = raw["d"]
        ref = O.linear_dequant(x, O.dequantize(q.cpu().numpy(), bits16(s)[:, None], bits=8,
                                               scale_dtype="bf16", storage="signed"))
    else:
        q, s = raw["d"]
        ref = O.linear_dequant(x, O.dequantize(O.unpack_int4_k32(q.cpu().numpy()), bits16(s), bits=4,
                                               scale_dtype="bf16"))
    assert O.rel_l2(bufs["d"].float().cpu().numpy(), ref) < 1e-2


def test_bounded_wait_gives_up_and_recovers():
    """A spin limit of one sleep makes the waits give up (forced from the host): the kernel
    still ends, flags the run, and after reset() a normal run is exact again."""
    m = 2
    chain, bufs, weights, _ = build_chain("fp8", m, 55)
    chain.run(spin_limit=1)
    torch.cuda.synchronize()
    assert chain.failed()
    chain.reset()
    chain.run()
    want = single_calls("fp8", chain, bufs, weights)
    torch.cuda.synchronize()
    assert not chain.failed()
    for name, *_ in CHAIN:
        assert torch.equal(bufs[name], want[name]), name


def test_chain_contract():
    w = qlinear.prepare(qlinear.quantize_w4(rand((64, 256), 0, 0.02).to(DEV)))
    chain = DecodeStack("w4a16", 2)
    with pytest.raises(ValueError):
        chain.add(w, torch.empty((3, 256), dtype=torch.bfloat16, device=DEV),
                  torch.empty((3, 64), dtype=torch.bfloat16, device=DEV))
    with pytest.raises(ValueError):
        chain.add(qlinear.prepare(qlinear.quantize_fp8(rand((64, 256), 0, 0.02).to(DEV))),
                  torch.empty((2, 256), dtype=torch.bfloat16, device=DEV),
                  torch.empty((2, 64), dtype=torch.bfloat16, device=DEV))
    with pytest.raises(ValueError):
        DecodeStack("w4a16", 17)
    with pytest.raises(ValueError):
        DecodeStack("int8", 1)
    with pytest.raises(ValueError):
        DecodeStack("w4a16", 1).build()
