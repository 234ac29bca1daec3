"""GPU parity of the executor's attention stage (DecodeStack.add_attention; csrc/decode_stack.hip
exec_attention / exec_merge): the head norm + RoPE, the cache writes and the split attention with
its merge inside the same launch as the projections around them.

The separate calls are the checker, on the chain's own qkv output: the caches the chain leaves
must equal, bit for bit, those qkv_norm_rope_to_cache leaves (the same rope arithmetic); the
attention output must agree with DecodeAttention on the rope kernel's query (the same products,
summed over other splits: within 2^-7 of each value plus 2^-9 of the row's largest, and under the
reference's 0.04 bound); o must be within one bf16 rounding step of the single-call linear on the
chain's own attention output. Graph replays follow the position.
"""

import pytest
import torch

from kernels import DecodeAttention, qlinear, qkv_norm_rope_to_cache
from kernels.decode_stack import DecodeStack
from test_gpu_decode_stack import DEV, rand

pytestmark = pytest.mark.gpu

EPS = 1e-6
N_Q, N_KV = 32, 8


def make_case(fmt, capacity, seed):
    quant = qlinear.FORMATS[fmt][0]
    g = torch.Generator().manual_seed(seed)
    w = {
        "qkv": qlinear.prepare(quant(rand((6144, 2560), seed + 1, std=0.02).to(DEV))),
        "o": qlinear.prepare(quant(rand((2560, 4096), seed + 2, std=0.02).to(DEV))),
    }
    t = {
        "h": rand((1, 2560), seed + 3).to(DEV),
        "w_in": (1.0 + 0.1 * torch.randn(2560, generator=g)).to(torch.bfloat16).to(DEV),
        "qn": (1.0 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16).to(DEV),
        "kn": (1.0 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16).to(DEV),
    }
    angles = torch.randn(capacity, 128, generator=g)
    t["cos"], t["sin"] = angles.cos().bfloat16().to(DEV), angles.sin().bfloat16().to(DEV)
    t["kc"] = torch.randn(1, N_KV, capacity, 128, generator=g).to(torch.bfloat16).to(DEV)
    t["vc"] = torch.randn(1, N_KV, capacity, 128, generator=g).to(torch.bfloat16).to(DEV)
    return w, t


def build(fmt, w, t, positions, splits):
    chain = DecodeStack(fmt, 1)
    t["qkv"] = torch.empty(1, 6144, dtype=torch.bfloat16, device=DEV)
    t["r0"] = torch.empty(1, 2560, dtype=torch.bfloat16, device=DEV)
    t["att"] = torch.empty(1, 4096, dtype=torch.bfloat16, device=DEV)
    t["o"] = torch.empty(1, 2560, dtype=torch.bfloat16, device=DEV)
    chain.add_normed(w["qkv"], t["h"], t["qkv"], t["w_in"], EPS, resid_out=t["r0"])
    chain.add_attention(t["qkv"], N_Q, N_KV, t["qn"], t["kn"], t["cos"], t["sin"], positions, t["kc"], t["vc"],
                        t["att"], EPS, splits=splits)
    chain.add(w["o"], t["att"], t["o"])
    return chain.build()


def separate(t, kc, vc, positions, capacity):
    """The same step's rope and attention as separate calls, on the chain's qkv output."""
    q = qkv_norm_rope_to_cache(t["qkv"], N_Q, N_KV, t["qn"], t["kn"], t["cos"], t["sin"], positions, 1, kc, vc, EPS)
    att = DecodeAttention(1, N_KV, 4, 128, capacity, DEV, config=4)(q, kc, vc, positions)
    return att.clone()


def close(got, want, what):
    got, want = got.float(), want.float()
    rowmax = want.abs().amax()
    diff = (got - want).abs()
    tol = 2.0 ** -7 * want.abs() + 2.0 ** -9 * rowmax
    assert (diff > tol).sum().item() == 0, (what, diff.max().item())
    assert diff.max().item() <= 0.04, what


@pytest.mark.parametrize("fmt", ["fp8", "w4a16"])
@pytest.mark.parametrize("pos,splits", [(512, 4), (37, 2), (639, 8), (0, 4)])
def test_attention_stage_matches_separate_calls(fmt, pos, splits):
    print(f"executor attention {fmt} pos={pos} splits={splits}", flush=True)
    capacity = 640
    w, t = make_case(fmt, capacity, 70 + pos)
    positions = torch.tensor([pos], dtype=torch.int32, device=DEV)
    kc0, vc0 = t["kc"].clone(), t["vc"].clone()
    chain = build(fmt, w, t, positions, splits)
    chain.run()
    torch.cuda.synchronize()
    assert not chain.failed(), chain.failed_waits()
    kc, vc = kc0.clone(), vc0.clone()
    att = separate(t, kc, vc, positions, capacity)
    assert torch.equal(t["kc"], kc) and torch.equal(t["vc"], vc), (fmt, pos, "caches differ from the rope kernel's")
    close(t["att"], att, (fmt, pos, "attention"))
    linear = qlinear.FORMATS[fmt][1]
    want = linear(t["att"].contiguous(), w["o"]).float()
    diff = (t["o"].float() - want).abs()
    tol = 2.0 ** -7 * want.abs() + 2.0 ** -9 * want.abs().amax()
    assert (diff > tol).sum().item() == 0, (fmt, pos, "o", diff.max().item())
    # a second run (same position) gives the same bits
    first = {k: t[k].clone() for k in ("att", "o", "kc", "vc")}
    chain.run()
    torch.cuda.synchronize()
    for k, v in first.items():
        assert torch.equal(t[k], v), (fmt, pos, k, "second run differs")


def test_attention_stage_graph_replays_follow_the_position():
    """Captured once, replayed at advancing positions with eager runs between: every replay
    writes the key and value at its position and attends over keys 0 .. position."""
    fmt, capacity = "fp8", 640
    w, t = make_case(fmt, capacity, 91)
    positions = torch.tensor([300], dtype=torch.int32, device=DEV)
    chain = build(fmt, w, t, positions, 4)
    chain.run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        chain.run()
    for step, pos in enumerate((301, 302, 331, 332)):
        print(f"executor attention graph replay pos={pos}", flush=True)
        positions.fill_(pos)
        t["h"].copy_(rand((1, 2560), 200 + step).to(DEV))
        kc, vc = t["kc"].clone(), t["vc"].clone()
        graph.replay()
        torch.cuda.synchronize()
        assert not chain.failed(), chain.failed_waits()
        att = separate(t, kc, vc, positions, capacity)
        assert torch.equal(t["kc"], kc) and torch.equal(t["vc"], vc), pos
        close(t["att"], att, ("replay", pos))


def test_attention_stage_contract_errors():
    fmt = "fp8"
    w, t = make_case(fmt, 64, 5)
    positions = torch.tensor([3], dtype=torch.int32, device=DEV)
    chain = DecodeStack(fmt, 2)
    with pytest.raises(ValueError):
        chain.add_attention(torch.empty(2, 6144, dtype=torch.bfloat16, device=DEV), N_Q, N_KV, t["qn"], t["kn"],
                            t["cos"], t["sin"], positions, t["kc"], t["vc"],
                            torch.empty(1, 4096, dtype=torch.bfloat16, device=DEV), EPS)
    chain = DecodeStack(fmt, 1)
    with pytest.raises(ValueError):  # qkv is not an output of the chain
        chain.add_attention(torch.empty(1, 6144, dtype=torch.bfloat16, device=DEV), N_Q, N_KV, t["qn"], t["kn"],
                            t["cos"], t["sin"], positions, t["kc"], t["vc"],
                            torch.empty(1, 4096, dtype=torch.bfloat16, device=DEV), EPS)


@pytest.mark.parametrize("fmt", ["fp8", "w4a16"])
def test_one_launch_decode_step_matches_split_launches(fmt):
    """bench.Model's one-launch decode step (executor_one_launch: attention stages inside the
    chain) against the same step on executor launches split at attention with the rope and
    attention kernels between them (executor_step), four layers: the logits within relative L2
    1e-2 and the caches' new rows within 2^-6 of each value plus 2^-8 of the row's largest (the
    attention outputs differ in their last bits, so later layers' inputs do too); every cache row
    but the position's untouched."""
    import bench
    print(f"one-launch decode step {fmt}", flush=True)
    model = bench.Model(fmt, 1, layers=4, attention=True)
    pos = int(model.positions.item())
    k0 = [k.clone() for k in model.k_cache]
    v0 = [v.clone() for v in model.v_cache]
    step = model.executor_step()
    step()
    torch.cuda.synchronize()
    assert not any(seg.failed() for seg in model.segments)
    want = model.logits.float().clone()
    kw = [k.clone() for k in model.k_cache]
    vw = [v.clone() for v in model.v_cache]
    for i in range(model.layers):
        model.k_cache[i].copy_(k0[i])
        model.v_cache[i].copy_(v0[i])
    chain = model.executor_one_launch(4)
    chain.run()
    torch.cuda.synchronize()
    assert not chain.failed(), chain.failed_waits()
    got = model.logits1.float()
    rel = ((got - want).norm() / want.norm()).item()
    assert rel <= 1e-2, (fmt, rel)
    for i in range(model.layers):
        for new, ref, old in ((model.k_cache[i], kw[i], k0[i]), (model.v_cache[i], vw[i], v0[i])):
            mask = torch.ones(new.shape[2], dtype=torch.bool, device=DEV)
            mask[pos] = False
            assert torch.equal(new[:, :, mask], old[:, :, mask]), (fmt, i, "rows other than the position changed")
            a, b = new[:, :, pos].float(), ref[:, :, pos].float()
            tol = 2.0 ** -6 * b.abs() + 2.0 ** -8 * b.abs().amax()
            assert ((a - b).abs() > tol).sum().item() == 0, (fmt, i, (a - b).abs().max().item())
