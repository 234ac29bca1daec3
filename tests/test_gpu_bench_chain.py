"""The chain bench.py times, checked: ``bench.Model(fmt, 1).linear_chain()`` -- 36 Qwen3-4B
layers (rmsnorm -> qkv, o on the query columns of qkv, residual + rmsnorm -> gate_up with the
fused SwiGLU, down, residual into the next layer's rmsnorm) and the final norm -> 151936-row
lm_head, 145 projections and 73 residual + RMSNorm stages in one executor launch -- in FP8 W8A8
and W4A16 at M = 1.

* every stage's residual (written to its resid_out) bit-exact against the oracle's residual
  add, on the chain's own residual and delta;
* every one of the 145 outputs against the single-call linear on the executor's own input
  within one bf16 rounding step: a plain input read back, a normed input recomputed by the
  oracle's RMSNorm (bit-exact with the stage, tests/test_gpu_norm_stages.py) from the chain's
  own residual;
* layers 0, 17 and 35 (all four projections) and 32 spread 16-row tiles of the lm_head against
  the CPU oracle at relative L2 <= 1e-2 (the north star's bound);
* identical bits on a second run, and on a replay of the run captured in a HIP graph.
"""

import numpy as np
import pytest
import torch

import bench
import oracle as O
from oracle import bf16_to_f32, f32_to_bf16
from kernels import qlinear

pytestmark = pytest.mark.gpu

ORACLE_LAYERS = (0, 17, 35)
HEAD_TILES = 32


def bits16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def dev_bits(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to("cuda")


def inputs_of(model):
    """The input of every projection of the chain: plain inputs as wired, normed inputs from the
    oracle's residual add + RMSNorm of the chain's own residual and delta. Checks each stage's
    residual output bit for bit on the way."""
    xs = []
    for i, wire in enumerate(model.wiring):
        if "x" in wire:
            xs.append(wire["x"])
            continue
        w = bits16(wire["w"])
        if wire["delta"] is None:
            r = bits16(wire["resid"])
            normed = O.rms_norm(r, w, bench.EPS)
        else:
            r, normed = O.add_rms_norm(bits16(wire["resid"]), bits16(wire["delta"]), w, bench.EPS)
        assert np.array_equal(bits16(wire["resid_out"]), r), (i, "residual")
        xs.append(dev_bits(normed))
    return xs


def oracle_rows(fmt, tiled, x, rows=None):
    """The oracle's product of x with the row-major weight (optionally a subset of rows)."""
    w = bench.untile(tiled.weight.cpu())
    s = tiled.scale.cpu()
    if rows is not None:
        w, s = w[rows], s[rows]
    xb = bits16(x)
    if fmt == "fp8":
        return O.linear_fp8_w8a8(xb, w.contiguous().view(torch.uint8).numpy(), bits16(s))
    deq = O.dequantize(O.unpack_int4_k32(w.contiguous().numpy()), bits16(s), bits=4, scale_dtype="bf16")
    return O.linear_dequant(xb, deq)


@pytest.mark.parametrize("fmt", ["fp8", "w4a16"])
def test_bench_chain_matches_single_calls_and_oracle(fmt):
    print(f"bench chain {fmt}: building 36 layers + lm_head", flush=True)
    stack = bench.Model(fmt, 1)
    chain = stack.linear_chain()
    assert len(chain.calls) == 4 * bench.LAYERS + 1
    chain.run()
    torch.cuda.synchronize()
    assert not chain.failed(), chain.failed_waits()
    first = [y.clone() for y in stack.outs]
    chain.run()
    torch.cuda.synchronize()
    assert not chain.failed(), chain.failed_waits()
    for i, (y, f) in enumerate(zip(stack.outs, first)):
        assert torch.equal(y, f), (fmt, i, "deterministic")
        assert bool(torch.isfinite(y).all()), (fmt, i, "finite")
    # a captured run replays as a new run (the epoch advances on the device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        chain.run()
    for y in stack.outs:
        y.zero_()
    graph.replay()
    torch.cuda.synchronize()
    assert not chain.failed(), chain.failed_waits()
    for i, (y, f) in enumerate(zip(stack.outs, first)):
        assert torch.equal(y, f), (fmt, i, "graph replay")
    print(f"bench chain {fmt}: deterministic, graph replay identical", flush=True)

    linear = qlinear.FORMATS[fmt][1]
    xs = inputs_of(stack)
    print(f"bench chain {fmt}: 73 stage residuals bit-exact against the oracle", flush=True)
    worst = 0.0
    for i, ((name, tiled, k, sw), x, y) in enumerate(zip(stack.calls, xs, stack.outs)):
        want = linear(x.contiguous(), tiled, swiglu=sw).float()
        got = y.float()
        diff = (got - want).abs()
        rowmax = want.abs().amax(dim=1, keepdim=True)
        tol = (2.0 ** -6 if sw else 2.0 ** -7) * want.abs() + 2.0 ** -9 * rowmax
        bad = int((diff > tol).sum())
        assert bad == 0, (fmt, i, name, bad, diff.max().item())
        worst = max(worst, float((diff / (want.abs() + 2.0 ** -9 * rowmax)).max()))
    print(f"bench chain {fmt}: 145 projections within one rounding step of the single calls "
          f"(largest relative step {worst:.2e})", flush=True)

    for layer in ORACLE_LAYERS:
        for j in range(4):
            i = 4 * layer + j
            name, tiled, k, sw = stack.calls[i]
            ref = oracle_rows(fmt, tiled, xs[i])
            if sw:
                ref = bf16_to_f32(O.swiglu(f32_to_bf16(np.asarray(ref, np.float32))))
            err = O.rel_l2(stack.outs[i].float().cpu().numpy(), ref)
            print(f"bench chain {fmt}: layer {layer} {name} rel-L2 {err:.2e}", flush=True)
            assert err <= 1e-2, (fmt, layer, name, err)
    name, tiled, k, sw = stack.calls[-1]
    tiles = np.linspace(0, tiled.rows // 16 - 1, HEAD_TILES).astype(int)
    rows = torch.from_numpy(np.concatenate([np.arange(16 * t, 16 * t + 16) for t in tiles]))
    ref = oracle_rows(fmt, tiled, xs[-1], rows)
    err = O.rel_l2(stack.outs[-1][:, rows].float().cpu().numpy(), ref)
    print(f"bench chain {fmt}: lm_head ({len(rows)} sampled rows) rel-L2 {err:.2e}", flush=True)
    assert err <= 1e-2, (fmt, "lm_head", err)
    del chain, stack
    torch.cuda.empty_cache()
