"""GPU parity of the decode-step executor (one launch for a chain of projections).

The executor cuts each projection's K range into pieces of its own (balanced over the
workgroups), so its fp32 sums are ordered differently from a single-call linear's: every
output is checked against the single-call linear on the executor's own input to within one
bf16 rounding step (most outputs are identical), against the CPU oracle to the north star's
relative L2 bound, and for determinism (identical bits on every run). Chained projections
read what an earlier projection of the same launch wrote, and inputs change between runs, so
a stale read of an earlier run's intermediate would show.
"""

import numpy as np
import pytest
import torch

import oracle as O
from oracle import bf16_to_f32, f32_to_bf16
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
# outputs, plus a tiny projection (fewer block-steps than workgroups) and long-K ones.
CHAIN = [
    ("a", 2048, 1024, "x", False),
    ("b", 3072, 2048, "a", True),      # SwiGLU: out 1536
    ("c", 1024, 1536, "b", False),
    ("c2", 1024, 512, "c[:512]", False),  # the first 512 columns of c's output
    ("d", 4096, 1024, "c", False),
    ("e", 16, 4096, "d", False),
    ("f", 1024, 9728, "g", False),     # reads an input the host writes
    ("h", 9728 * 2, 1024, "f", True),  # SwiGLU: out 9728
    ("i", 1024, 9728, "h", False),
]


# One Qwen3-4B decoder layer's projections (hidden 2560, intermediate 9728; o reads the query
# part of qkv): at M = 1 the planner cuts no row block into K pieces, so the launch runs the
# kernel instance without the piece reduction (and with deeper prefetch).
QWEN_LAYER = [
    ("qkv", 6144, 2560, "x2560", False),
    ("o", 2560, 4096, "qkv[:4096]", False),
    ("gu", 19456, 2560, "o", True),
    ("dn", 2560, 9728, "gu", False),
]


def source(bufs, src):
    """The input tensor named by `src`: a buffer, or "name[:k]" for its first k columns."""
    if "[" in src:
        name, k = src[:-1].split("[:")
        return bufs[name][:, :int(k)]
    return bufs[src]


def build_chain(fmt, m, seed, kw=0, waves=8, lanes=1, chain_def=None):
    quant = qlinear.FORMATS[fmt][0]
    bufs = {"x": rand((m, 1024), seed).to(DEV), "g": rand((m, 9728), seed + 1).to(DEV),
            "x2560": rand((m, 2560), seed + 2).to(DEV)}
    weights, raw = {}, {}
    chain = DecodeStack(fmt, m, waves=waves, groups_per_cu=lanes)
    for idx, (name, n, k, src, sw) in enumerate(chain_def or CHAIN):
        w = rand((n, k), seed + 10 + idx, std=0.02).to(DEV)
        packed = quant(w)
        raw[name] = packed
        weights[name] = qlinear.prepare(packed)
        bufs[name] = torch.empty((m, n // 2 if sw else n), dtype=torch.bfloat16, device=DEV)
        chain.add(weights[name], source(bufs, src), bufs[name], swiglu=sw, kw=kw)
    chain.build()
    return chain, bufs, weights, raw


def check_against_single_calls(fmt, bufs, weights, tag, chain_def=None):
    """Each projection vs the single-call linear on the executor's own input."""
    linear = qlinear.FORMATS[fmt][1]
    for name, n, k, src, sw in chain_def or CHAIN:
        want = linear(source(bufs, src).contiguous(), weights[name], swiglu=sw).float()
        got = bufs[name].float()
        diff = (got - want).abs()
        # fp32 sums in another order: at most a rounding step of bf16 (2^-7 relative; SwiGLU
        # rounds g, u and silu(g) to bf16 first, so allow two steps there), plus a small
        # absolute term for outputs near zero, where the sums cancel (2^-9 of the row's max)
        rowmax = want.abs().amax(dim=1, keepdim=True)
        tol = (2.0 ** -6 if sw else 2.0 ** -7) * want.abs() + 2.0 ** -9 * rowmax
        bad = (diff > tol).sum().item()
        assert bad == 0, (tag, name, bad, diff.max().item())
        same = (diff == 0).float().mean().item()
        assert same > 0.5, (tag, name, "most outputs are bitwise equal", same)


def oracle_check(fmt, x_bits, packed, y, swiglu=False):
    """rel-L2 of y against the oracle's product (with swiglu: the oracle's SwiGLU of the
    bf16-rounded gate/up product, reference.py:74-79)."""
    q, s = packed
    if fmt == "fp8":
        ref = O.linear_fp8_w8a8(x_bits, q.view(torch.uint8).cpu().numpy(), bits16(s))
    elif fmt == "w8a16":
        ref = O.linear_dequant(x_bits, O.dequantize(q.cpu().numpy(), bits16(s)[:, None], bits=8,
                                                    scale_dtype="bf16", storage="signed"))
    else:
        ref = O.linear_dequant(x_bits, O.dequantize(O.unpack_int4_k32(q.cpu().numpy()), bits16(s), bits=4,
                                                    scale_dtype="bf16"))
    if swiglu:
        ref = bf16_to_f32(O.swiglu(f32_to_bf16(np.asarray(ref, np.float32))))
    return O.rel_l2(y.float().cpu().numpy(), ref)


def run_chain_checks(fmt, m, waves=8):
    chain, bufs, weights, raw = build_chain(fmt, m, 100 * m, waves=waves)
    assert chain.grid >= 256 and chain.lds > 0 and chain.launch.waves == waves
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
        for name, *_ in CHAIN:
            assert torch.equal(bufs[name], first[name]), (fmt, m, run, name, "deterministic")
        check_against_single_calls(fmt, bufs, weights, (fmt, m, run))
    for name in ("b", "c2", "d", "h", "i"):
        _, _, _, src, sw = [c for c in CHAIN if c[0] == name][0]
        assert oracle_check(fmt, bits16(source(bufs, src)), raw[name], bufs[name], swiglu=sw) < 1e-2, name


@pytest.mark.parametrize("fmt", ["w4a16", "w8a16", "fp8"])
@pytest.mark.parametrize("m", [1, 5, 16])
def test_chain_matches_single_calls_and_oracle(fmt, m):
    print(f"decode stack {fmt} m={m}", flush=True)
    run_chain_checks(fmt, m)


@pytest.mark.parametrize("fmt", ["w4a16", "w8a16", "fp8"])
@pytest.mark.parametrize("m", [1, 5, 16])
def test_four_wave_chain_matches_single_calls_and_oracle(fmt, m):
    """Workgroups of 4 waves (half the staging threads: m = 16 at FP8 takes more than one pass
    over each row for the token maxima) give the same results as the single-call linears."""
    print(f"decode stack 4 waves {fmt} m={m}", flush=True)
    run_chain_checks(fmt, m, waves=4)


@pytest.mark.parametrize("fmt", ["w4a16", "w8a16", "fp8"])
def test_layer_chain_without_pieces(fmt):
    """A Qwen3-4B layer at M = 1 (the decode step's shapes): no row block is cut into pieces,
    so the run takes the executor instance without the piece reduction; same bounds as the
    other chains, deterministic, and within the north star's bound of the oracle."""
    print(f"decode stack layer {fmt}", flush=True)
    chain, bufs, weights, raw = build_chain(fmt, 1, 31, chain_def=QWEN_LAYER)
    assert chain.launch.pieces == 0 and all(c[3] == 1 for c in chain.configs), chain.configs
    for run in range(2):
        if run:
            bufs["x2560"].copy_(rand((1, 2560), 99).to(DEV))
        chain.run()
        torch.cuda.synchronize()
        assert not chain.failed(), chain.failed_waits()
        first = {name: bufs[name].clone() for name, *_ in QWEN_LAYER}
        chain.run()
        torch.cuda.synchronize()
        for name, *_ in QWEN_LAYER:
            assert torch.equal(bufs[name], first[name]), (fmt, run, name, "deterministic")
        check_against_single_calls(fmt, bufs, weights, (fmt, "layer", run), chain_def=QWEN_LAYER)
    for name, _, _, src, sw in QWEN_LAYER:  # every projection, gate_up through its SwiGLU
        assert oracle_check(fmt, bits16(source(bufs, src)), raw[name], bufs[name], swiglu=sw) < 1e-2, name


@pytest.mark.parametrize("kw,fmt,waves", [(kw, "w4a16", 8) for kw in (1, 2, 4, 8)] +
                         [(kw, "fp8", 4) for kw in (1, 2, 4)])
def test_every_tile_split_is_exact(kw, fmt, waves):
    """Forced waves-per-tile settings (every divisor of the workgroup's waves) change the
    pieces, not the results' bound."""
    print(f"decode stack kw={kw} {fmt} waves={waves}", flush=True)
    chain, bufs, weights, _ = build_chain(fmt, 3, 77, kw=kw, waves=waves)
    assert all(c[1] == kw for c in chain.configs)
    assert chain.launch.pieces == int(any(c[3] > 1 for c in chain.configs))
    chain.run()
    torch.cuda.synchronize()
    assert not chain.failed()
    check_against_single_calls(fmt, bufs, weights, ("kw", kw, waves))


@pytest.mark.parametrize("fmt,waves,lanes,m", [("fp8", 4, 3, 4), ("w4a16", 4, 2, 4), ("w8a16", 8, 2, 4),
                                               ("fp8", 8, 2, 8)])
def test_lanes_and_small_workgroups(fmt, waves, lanes, m):
    """Projections spread over several lanes (chained inputs cross lanes) give the same
    results as the single-call linears (FP8 at 8 tokens: token maxima published by a
    projection of another lane)."""
    print(f"decode stack lanes {fmt} waves={waves} lanes={lanes} m={m}", flush=True)
    chain, bufs, weights, _ = build_chain(fmt, m, 300 + lanes, waves=waves, lanes=lanes)
    assert chain.launch.lanes >= 1 and chain.launch.waves == waves
    for run in range(2):
        if run:
            bufs["x"].copy_(rand((m, 1024), 11).to(DEV))
            bufs["g"].copy_(rand((m, 9728), 12).to(DEV))
        chain.run()
        torch.cuda.synchronize()
        assert not chain.failed()
        check_against_single_calls(fmt, bufs, weights, (fmt, waves, lanes, run))


@pytest.mark.parametrize("waves,m", [(8, 2), (4, 2), (8, 8)])
def test_bounded_wait_gives_up_and_recovers(waves, m):
    """A zero wait budget makes the waits give up (forced from the host): the kernel still
    ends, flags the run, and after reset() a normal run is right again (FP8 at 8 tokens: the
    wait for the published token maxima too)."""
    print(f"decode stack bounded wait waves={waves} m={m}", flush=True)
    chain, bufs, weights, _ = build_chain("fp8", m, 55, waves=waves)
    chain.run(budget_us=0)
    torch.cuda.synchronize()
    assert chain.failed()
    chain.reset()
    chain.run()
    torch.cuda.synchronize()
    assert not chain.failed()
    check_against_single_calls("fp8", bufs, weights, "after reset")


def test_chain_rejects_hazards():
    """Outputs may not overlap each other or an input read from memory."""
    w = qlinear.prepare(qlinear.quantize_w8(rand((64, 256), 0, 0.02).to(DEV)))
    x = torch.zeros((1, 256), dtype=torch.bfloat16, device=DEV)
    big = torch.zeros((1, 512), dtype=torch.bfloat16, device=DEV)
    chain = DecodeStack("w8a16", 1).add(w, x, big[:, :64]).add(w, x, big[:, 32:96])
    with pytest.raises(ValueError, match="overlap"):
        chain.build()
    y = torch.zeros((1, 64), dtype=torch.bfloat16, device=DEV)
    chain = DecodeStack("w8a16", 1).add(w, big[:, :256], y).add(w, x, big[:, 128:192])
    with pytest.raises(ValueError, match="writes"):
        chain.build()


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
        chain.add(w, torch.empty((2, 256), dtype=torch.bfloat16, device=DEV),
                  torch.empty((2, 64), dtype=torch.bfloat16, device=DEV), kw=3).build()
    with pytest.raises(ValueError):
        DecodeStack("w4a16", 17)
    with pytest.raises(ValueError):
        DecodeStack("int8", 1)
    with pytest.raises(ValueError):
        DecodeStack("w4a16", 1).build()


@pytest.mark.parametrize("fmt,m", [("fp8", 1), ("w4a16", 5), ("fp8", 8)])
def test_captured_runs_replay_as_new_runs(fmt, m):
    """A run captured into a HIP graph: each replay takes the next epoch from the arena, so it
    waits for this replay's values, not the last one's. Replays alternate with eager input
    changes, eager runs and synchronisations; every replay equals an eager run on its inputs."""
    print(f"decode stack graph {fmt} m={m}", flush=True)
    chain, bufs, weights, _ = build_chain(fmt, m, 500 + m)
    chain.run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        chain.run()
    for rep in range(4):
        bufs["x"].copy_(rand((m, 1024), 40 + rep).to(DEV))
        bufs["g"].copy_(rand((m, 9728), 60 + rep).to(DEV))
        for name, *_ in CHAIN:
            bufs[name].fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert not chain.failed(), (rep, chain.failed_waits())
        replayed = {name: bufs[name].clone() for name, *_ in CHAIN}
        chain.run()
        torch.cuda.synchronize()
        for name, *_ in CHAIN:
            assert torch.equal(bufs[name], replayed[name]), (fmt, m, rep, name)
    check_against_single_calls(fmt, bufs, weights, (fmt, m, "graph"))
