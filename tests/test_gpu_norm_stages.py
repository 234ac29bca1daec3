"""GPU parity of the executor's residual add + RMSNorm input stages (kernels.decode_stack
DecodeStack.add_normed; csrc/decode_stack.hip stage_norm): whole decode layers whose norms run
inside the launch. Every stage's residual and normed input are checked bit for bit against the
oracle on the chain's own inputs, every projection against the single-call linear on its stage's
normed input (within one bf16 rounding step) and o / down against the oracle, and two runs for
bitwise equality.
"""

import numpy as np
import pytest
import torch

import oracle as O
from kernels import qlinear
from kernels.decode_stack import DecodeStack
from test_gpu_decode_stack import DEV, bits16, oracle_check, rand

pytestmark = pytest.mark.gpu


def build_norm_chain(fmt, m, seed, layers=2, waves=8):
    """`layers` Qwen3-4B layers with their residual adds and RMSNorms inside the chain, then a
    final norm into a small head: qkv <- rmsnorm(h); o; gate_up <- rmsnorm(h + o); down; the next
    qkv <- rmsnorm(h + o + down); ..."""
    quant = qlinear.FORMATS[fmt][0]
    chain = DecodeStack(fmt, m, waves=waves)
    bufs = {"h_in": rand((m, 2560), seed).to(DEV)}
    weights, raw, stages = {}, {}, []
    eps = 1e-6

    def proj(name, n, k, idx):
        packed = quant(rand((n, k), seed + 10 + idx, std=0.02).to(DEV))
        raw[name] = packed
        weights[name] = qlinear.prepare(packed)

    def out(name, n):
        bufs[name] = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
        return bufs[name]

    def norm_w(name, idx):
        g = torch.Generator().manual_seed(seed + 500 + idx)
        bufs[name] = (1.0 + 0.1 * torch.randn(2560, generator=g)).to(torch.bfloat16).to(DEV)
        return bufs[name]

    resid, delta = "h_in", None
    for L in range(layers):
        for i, (n, k) in enumerate(((6144, 2560), (2560, 4096), (19456, 2560), (2560, 9728))):
            proj(f"{('qkv', 'o', 'gu', 'dn')[i]}{L}", n, k, 4 * L + i)
        chain.add_normed(weights[f"qkv{L}"], bufs[resid], out(f"qkv{L}", 6144), norm_w(f"win{L}", 2 * L), eps,
                         delta=None if delta is None else bufs[delta], resid_out=out(f"h0_{L}", 2560),
                         normed_out=out(f"nq{L}", 2560))
        stages.append((resid, delta, f"win{L}", f"h0_{L}", f"nq{L}", f"qkv{L}", False))
        chain.add(weights[f"o{L}"], bufs[f"qkv{L}"][:, :4096], out(f"o{L}", 2560))
        chain.add_normed(weights[f"gu{L}"], bufs[f"h0_{L}"], out(f"gu{L}", 9728), norm_w(f"wpost{L}", 2 * L + 1), eps,
                         delta=bufs[f"o{L}"], resid_out=out(f"h1_{L}", 2560), normed_out=out(f"ng{L}", 2560),
                         swiglu=True)
        stages.append((f"h0_{L}", f"o{L}", f"wpost{L}", f"h1_{L}", f"ng{L}", f"gu{L}", True))
        chain.add(weights[f"dn{L}"], bufs[f"gu{L}"], out(f"dn{L}", 2560))
        resid, delta = f"h1_{L}", f"dn{L}"
    proj("head", 1024, 2560, 99)
    chain.add_normed(weights["head"], bufs[resid], out("head", 1024), norm_w("wfin", 99), eps, delta=bufs[delta],
                     resid_out=out("h_fin", 2560), normed_out=out("nfin", 2560))
    stages.append((resid, delta, "wfin", "h_fin", "nfin", "head", False))
    chain.build()
    return chain, bufs, weights, raw, stages


@pytest.mark.parametrize("fmt,m,waves", [("fp8", 1, 8), ("w4a16", 1, 8), ("w8a16", 1, 8), ("fp8", 2, 8),
                                         ("w4a16", 3, 8), ("fp8", 4, 8), ("w4a16", 8, 8), ("fp8", 8, 8),
                                         ("w8a16", 16, 8), ("fp8", 16, 8), ("fp8", 3, 4), ("w4a16", 5, 4)])
def test_decode_layers_with_residual_and_norm(fmt, m, waves):
    """Residual add + RMSNorm (+ FP8 per-token quantize) as input stages of the executor (one
    chunk per thread at M = 1, three from M = 2 at k = 2560; past four token rows per pass --
    M > 4 at 8 waves, M > 2 at 4 -- in several passes of whole token rows): every stage's
    residual and normed input are bit-exact against the oracle on the chain's own inputs, every
    projection agrees with the single-call linear on its stage's normed input (and o / down with
    the oracle), and two runs are bitwise equal."""
    print(f"norm chain {fmt} m={m} waves={waves}", flush=True)
    chain, bufs, weights, raw, stages = build_norm_chain(fmt, m, 700 + m, waves=waves)
    linear = qlinear.FORMATS[fmt][1]
    for run in range(2):
        if run:
            bufs["h_in"].copy_(rand((m, 2560), 7000 + m).to(DEV))
        chain.run()
        torch.cuda.synchronize()
        assert not chain.failed(), chain.failed_waits()
        snap = {k: v.clone() for k, v in bufs.items()}
        chain.run()
        torch.cuda.synchronize()
        assert not chain.failed(), chain.failed_waits()
        for k, v in bufs.items():
            assert torch.equal(v, snap[k]), (fmt, m, run, k, "deterministic")
        for resid, delta, w, r_out, n_out, y, sw in stages:
            if delta is None:
                o_r, o_n = bits16(bufs[resid]), O.rms_norm(bits16(bufs[resid]), bits16(bufs[w]), 1e-6)
            else:
                o_r, o_n = O.add_rms_norm(bits16(bufs[resid]), bits16(bufs[delta]), bits16(bufs[w]), 1e-6)
            assert np.array_equal(bits16(bufs[r_out]), o_r), (fmt, m, run, r_out, "residual")
            assert np.array_equal(bits16(bufs[n_out]), o_n), (fmt, m, run, n_out, "normed input")
            want = linear(bufs[n_out], weights[y], swiglu=sw).float()
            got = bufs[y].float()
            rowmax = want.abs().amax(dim=1, keepdim=True)
            tol = (2.0 ** -6 if sw else 2.0 ** -7) * want.abs() + 2.0 ** -9 * rowmax
            assert ((got - want).abs() > tol).sum().item() == 0, (fmt, m, run, y)
        for L in range(2):
            assert oracle_check(fmt, bits16(bufs[f"qkv{L}"][:, :4096].contiguous()), raw[f"o{L}"],
                                bufs[f"o{L}"]) < 1e-2
            assert oracle_check(fmt, bits16(bufs[f"gu{L}"]), raw[f"dn{L}"], bufs[f"dn{L}"]) < 1e-2


def test_norm_chain_bounded_wait_gives_up_and_recovers():
    """A zero wait budget makes every wait give up, the norm stages' too (forced from the host):
    the kernel still ends and flags the run; after reset() a normal run is right again."""
    print("norm chain bounded wait", flush=True)
    chain, bufs, weights, raw, stages = build_norm_chain("fp8", 1, 55, layers=1)
    chain.run(budget_us=0)
    torch.cuda.synchronize()
    assert chain.failed()
    chain.reset()
    chain.run()
    torch.cuda.synchronize()
    assert not chain.failed(), chain.failed_waits()
    for resid, delta, w, r_out, n_out, y, sw in stages:
        if delta is None:
            o_r, o_n = bits16(bufs[resid]), O.rms_norm(bits16(bufs[resid]), bits16(bufs[w]), 1e-6)
        else:
            o_r, o_n = O.add_rms_norm(bits16(bufs[resid]), bits16(bufs[delta]), bits16(bufs[w]), 1e-6)
        assert np.array_equal(bits16(bufs[r_out]), o_r), (r_out, "residual after reset")
        assert np.array_equal(bits16(bufs[n_out]), o_n), (n_out, "normed input after reset")
