"""GPU parity of the QKV consumer (head norm + RoPE + cache write) and decode attention.

Ports of the reference's GPU checks (bench/gpu_checks.py:4-42 check_rope_fusion, :45-86
check_attention_dispatch, :207-265 check_kv_int8), with the oracle (oracle/attention_oracle.py)
as the checker: the rope kernel bit-exact, attention within the reference's own bound
(max |delta| <= 0.04 against exact attention) and the north star's rel-L2 <= 1e-2.
"""

import numpy as np
import pytest
import torch

import oracle.attention_oracle as A
from oracle import bf16_to_f32, rel_l2

pytestmark = pytest.mark.gpu

EPS = 1e-6


def bits(t):
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def dev_bits(a, device="cuda"):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(device)


def rope_inputs(rows, capacity, seed, width=6144):
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn(rows, width, generator=g).to(torch.bfloat16).cuda()
    qn = torch.randn(128, generator=g).to(torch.bfloat16).cuda()
    kn = torch.randn(128, generator=g).to(torch.bfloat16).cuda()
    angles = torch.randn(capacity, 128, generator=g)
    return qkv, qn, kn, angles.cos().bfloat16().cuda(), angles.sin().bfloat16().cuda()


@pytest.mark.parametrize("batch", [1, 4, 16])
@pytest.mark.parametrize("length", [1, 17])
def test_qkv_norm_rope_matches_oracle_and_separate_kernels(batch, length):
    """check_rope_fusion (gpu_checks.py:4-42): the fused kernel, the separate Q and K/V kernels
    and the oracle agree bit for bit; batches around the destination stay untouched."""
    from kernels import kv_norm_rope_to_cache, q_norm_rope, qkv_norm_rope_to_cache
    capacity = length + 12
    qkv, qn, kn, cos, sin = rope_inputs(batch * length, capacity, 31 + batch + length)
    positions = torch.arange(5, 5 + length, device="cuda", dtype=torch.int32)
    shape = (batch + 2, 8, capacity, 128)
    want_k = torch.full(shape, -37.0, dtype=torch.bfloat16, device="cuda")
    want_v = torch.full_like(want_k, 41.0)
    got_k, got_v = want_k.clone(), want_v.clone()
    sep_q = q_norm_rope(qkv, 32, qn, cos, sin, positions, length, EPS)
    kv_norm_rope_to_cache(qkv, 4096, 8, kn, cos, sin, positions, length, want_k[1:1 + batch], want_v[1:1 + batch], EPS)
    got_q = qkv_norm_rope_to_cache(qkv, 32, 8, qn, kn, cos, sin, positions, length,
                                   got_k[1:1 + batch], got_v[1:1 + batch], EPS)
    torch.cuda.synchronize()
    assert torch.equal(got_q, sep_q) and torch.equal(got_k, want_k) and torch.equal(got_v, want_v)

    ok = np.full(shape, bits(torch.tensor(-37.0).bfloat16()), np.uint16)
    ov = np.full(shape, bits(torch.tensor(41.0).bfloat16()), np.uint16)
    oq = A.qkv_norm_rope_to_cache(bits(qkv), 32, 8, bits(qn), bits(kn), bits(cos), bits(sin),
                                  positions.cpu().numpy(), length, ok[1:1 + batch], ov[1:1 + batch], EPS)
    assert np.array_equal(bits(got_q), oq)
    assert np.array_equal(bits(got_k), ok) and np.array_equal(bits(got_v), ov)


@pytest.mark.parametrize("splits", [1, 2, 3])
def test_qkv_planes_norm_rope_matches_oracle(splits):
    """qkv_planes_norm_rope_to_cache: the planes summed in slice order and rounded once, then the
    same bits as the bf16 kernel (rope.py:169-218; gpu_checks.py:197-202)."""
    from kernels import qkv_norm_rope_to_cache, qkv_planes_norm_rope_to_cache
    batch, length, capacity = 3, 2, 16
    rows = batch * length
    g = torch.Generator().manual_seed(7 + splits)
    planes = torch.randn(splits, rows, 6144, generator=g).cuda()
    _, qn, kn, cos, sin = rope_inputs(1, capacity, 11)
    positions = torch.tensor([3, 9], device="cuda", dtype=torch.int64)
    kp = torch.zeros(batch, 8, capacity, 128, dtype=torch.bfloat16, device="cuda")
    vp = torch.zeros_like(kp)
    q = qkv_planes_norm_rope_to_cache(planes, 32, 8, qn, kn, cos, sin, positions, length, kp, vp, EPS)
    reduced = planes[0].clone()
    for s in range(1, splits):
        reduced += planes[s]
    reduced = reduced.bfloat16()
    kr, vr = torch.zeros_like(kp), torch.zeros_like(vp)
    qr = qkv_norm_rope_to_cache(reduced, 32, 8, qn, kn, cos, sin, positions, length, kr, vr, EPS)
    torch.cuda.synchronize()
    assert torch.equal(q, qr) and torch.equal(kp, kr) and torch.equal(vp, vr)
    ok = np.zeros((batch, 8, capacity, 128), np.uint16)
    ov = ok.copy()
    oq = A.qkv_norm_rope_to_cache(bits(reduced), 32, 8, bits(qn), bits(kn), bits(cos), bits(sin),
                                  positions.cpu().numpy(), length, ok, ov, EPS)
    assert np.array_equal(bits(q), oq) and np.array_equal(bits(kp), ok) and np.array_equal(bits(vp), ov)


@pytest.mark.parametrize("batch,length", [(1, 1), (4, 1), (2, 9)])
def test_int8_cache_writes_match_oracle(batch, length):
    """check_kv_int8's write half (gpu_checks.py:216-265): INT8 codes and scales bit-exact against
    the oracle, Q unchanged, the bf16 copies equal to the bf16 cache, dequantised values within
    half a step, the planes kernel identical."""
    from kernels import qkv_norm_rope_to_cache, qkv_planes_norm_rope_to_cache
    capacity = 40
    qkv, qn, kn, cos, sin = rope_inputs(batch * length, capacity, 61 + batch)
    positions = torch.arange(3, 3 + length, device="cuda", dtype=torch.int32)
    shape = (batch, 8, capacity, 128)
    k16 = torch.zeros(shape, dtype=torch.bfloat16, device="cuda")
    v16 = torch.zeros_like(k16)
    q16 = qkv_norm_rope_to_cache(qkv, 32, 8, qn, kn, cos, sin, positions, length, k16, v16, EPS)
    k8 = torch.zeros(shape, dtype=torch.int8, device="cuda")
    v8 = torch.zeros_like(k8)
    ks = torch.zeros(shape[:-1], dtype=torch.float32, device="cuda")
    vs = torch.zeros_like(ks)
    kc = torch.zeros(batch, 8, length, 128, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    q8 = qkv_norm_rope_to_cache(qkv, 32, 8, qn, kn, cos, sin, positions, length, k8, v8, EPS,
                                k_scale=ks, v_scale=vs, k_copy=kc, v_copy=vc)
    torch.cuda.synchronize()
    assert torch.equal(q8, q16)
    for t, p in enumerate(range(3, 3 + length)):
        assert torch.equal(kc[:, :, t], k16[:, :, p]) and torch.equal(vc[:, :, t], v16[:, :, p])
    ok8, ov8 = np.zeros(shape, np.int8), np.zeros(shape, np.int8)
    oks, ovs = np.zeros(shape[:-1], np.float32), np.zeros(shape[:-1], np.float32)
    okc, ovc = np.zeros((batch, 8, length, 128), np.uint16), np.zeros((batch, 8, length, 128), np.uint16)
    A.qkv_norm_rope_to_cache(bits(qkv), 32, 8, bits(qn), bits(kn), bits(cos), bits(sin), positions.cpu().numpy(),
                             length, ok8, ov8, EPS, oks, ovs, okc, ovc)
    assert np.array_equal(k8.cpu().numpy(), ok8) and np.array_equal(v8.cpu().numpy(), ov8)
    assert np.array_equal(ks.cpu().numpy().view(np.uint32), oks.view(np.uint32))
    assert np.array_equal(vs.cpu().numpy().view(np.uint32), ovs.view(np.uint32))
    assert np.array_equal(bits(kc), okc) and np.array_equal(bits(vc), ovc)
    written = torch.zeros(capacity, dtype=torch.bool, device="cuda")
    written[3:3 + length] = True
    for c8, sc, c16 in ((k8, ks, k16), (v8, vs, v16)):
        err = (c8.float() * sc[..., None] - c16.float())[:, :, written].abs()
        assert (err <= (sc[:, :, written] * 0.5 + 1e-6)[..., None]).all()
    planes = torch.stack([qkv.float() * 0.25, qkv.float() * 0.75])
    k8b, v8b, ksb, vsb = torch.zeros_like(k8), torch.zeros_like(v8), torch.zeros_like(ks), torch.zeros_like(vs)
    kcb, vcb = torch.zeros_like(kc), torch.zeros_like(vc)
    qp = qkv_planes_norm_rope_to_cache(planes, 32, 8, qn, kn, cos, sin, positions, length, k8b, v8b, EPS,
                                       k_scale=ksb, v_scale=vsb, k_copy=kcb, v_copy=vcb)
    ref = planes.sum(0).to(torch.bfloat16)
    k8r, v8r, ksr, vsr = torch.zeros_like(k8), torch.zeros_like(v8), torch.zeros_like(ks), torch.zeros_like(vs)
    kcr, vcr = torch.zeros_like(kc), torch.zeros_like(vc)
    qr = qkv_norm_rope_to_cache(ref, 32, 8, qn, kn, cos, sin, positions, length, k8r, v8r, EPS,
                                k_scale=ksr, v_scale=vsr, k_copy=kcr, v_copy=vcr)
    torch.cuda.synchronize()
    assert torch.equal(qp, qr) and torch.equal(k8b, k8r) and torch.equal(v8b, v8r)
    assert torch.equal(ksb, ksr) and torch.equal(vsb, vsr) and torch.equal(kcb, kcr) and torch.equal(vcb, vcr)


def test_norm_rope_position_outside_tables_is_loud_and_writes_nothing():
    from kernels import qkv_norm_rope_to_cache
    qkv, qn, kn, cos, sin = rope_inputs(2, 8, 3)
    positions = torch.tensor([8], device="cuda", dtype=torch.int32)  # table has rows 0..7
    kc = torch.full((2, 8, 8, 128), 5.0, dtype=torch.bfloat16, device="cuda")
    vc = kc.clone()
    q = qkv_norm_rope_to_cache(qkv, 32, 8, qn, kn, cos, sin, positions, 1, kc, vc, EPS)
    torch.cuda.synchronize()
    assert torch.isnan(q).all()
    assert (kc == 5.0).all() and (vc == 5.0).all()


def attention_case(batch, tokens, capacity, seed, n_kv=8, group=4, quant=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(batch * tokens, n_kv * group * 128, generator=g).to(torch.bfloat16).cuda()
    keys = torch.randn(batch, n_kv, capacity, 128, generator=g)
    values = torch.randn(batch, n_kv, capacity, 128, generator=g)
    if not quant:
        return q, keys.bfloat16().cuda(), values.bfloat16().cuda(), None, None
    ks = keys.abs().amax(-1) / 127.0
    vs = values.abs().amax(-1) / 127.0
    k8 = torch.round(keys / ks[..., None]).clamp(-127, 127).to(torch.int8)
    v8 = torch.round(values / vs[..., None]).clamp(-127, 127).to(torch.int8)
    return q, k8.cuda(), v8.cuda(), ks.cuda(), vs.cuda()


def oracle_attention(q, k, v, first, tokens, group, ks=None, vs=None):
    if ks is None:
        return A.decode_attention(bits(q), bits(k), bits(v), first, tokens, group)
    return A.decode_attention(bits(q), k.cpu().numpy(), v.cpu().numpy(), first, tokens, group,
                              ks.cpu().numpy(), vs.cpu().numpy())


@pytest.mark.parametrize("quant", [False, True])
@pytest.mark.parametrize("batch", [1, 4])
@pytest.mark.parametrize("tokens", [1, 2, 3])
def test_decode_attention_matches_oracle(batch, tokens, quant):
    """check_attention_dispatch (gpu_checks.py:45-86) and check_kv_int8's read half: causal
    boundaries, keys past the live ones poisoned with NaN, several split counts."""
    from kernels import DecodeAttention
    capacity, group = 521, 4
    q, k, v, ks, vs = attention_case(batch, tokens, capacity, 47 + batch * 3 + tokens, quant=quant)
    for first in (0, 127, capacity - tokens):
        kp, vp = k.clone(), v.clone()
        if not quant:  # NaN where no row may look
            kp[:, :, first + tokens:] = float("nan")
            vp[:, :, first + tokens:] = float("nan")
        pos = torch.tensor([first], device="cuda", dtype=torch.int32)
        want = oracle_attention(q, k, v, first, tokens, group, ks, vs)
        for config in (None, 1, 4, 16, 64):
            att = DecodeAttention(batch, 8, group, 128, capacity, "cuda", tokens=tokens, config=config, quant=quant)
            got = att(q, kp, vp, pos, ks, vs).float().cpu().numpy()
            assert np.isfinite(got).all(), (first, config)
            err = np.abs(got - want).max()
            assert err <= 0.04, (first, config, err)
            assert rel_l2(got, want) <= 1e-2, (first, config)


@pytest.mark.parametrize("quant", [False, True])
@pytest.mark.parametrize("tokens", [5, 8, 10, 16])
def test_decode_attention_many_query_rows(tokens, quant):
    """More than 16 query rows per KV head (speculative verification widths): 2, 2, 3 and 4 row
    tiles (20, 32, 40, 64 rows at group 4), bf16 and INT8 caches. Past the live keys the bf16
    cache holds NaN and the INT8 cache's scales hold NaN (the codes stay): no row may read them."""
    from kernels import DecodeAttention
    batch, capacity, group = 2, 300, 4
    q, k, v, ks, vs = attention_case(batch, tokens, capacity, 5 + tokens, quant=quant)
    first = capacity - tokens - 7
    pos = torch.tensor([first], device="cuda", dtype=torch.int32)
    want = oracle_attention(q, k, v, first, tokens, group, ks, vs)
    kp, vp, ksp, vsp = k.clone(), v.clone(), ks, vs
    if quant:
        ksp, vsp = ks.clone(), vs.clone()
        ksp[:, :, first + tokens:] = float("nan")
        vsp[:, :, first + tokens:] = float("nan")
    else:
        kp[:, :, first + tokens:] = float("nan")
        vp[:, :, first + tokens:] = float("nan")
    for config in (1, 8):
        print(f"attention rows: tokens {tokens} quant {quant} splits {config}", flush=True)
        got = DecodeAttention(batch, 8, group, 128, capacity, "cuda", tokens=tokens, config=config, quant=quant)(
            q, kp, vp, pos, ksp, vsp).float().cpu().numpy()
        assert np.isfinite(got).all(), (tokens, quant, config)
        assert np.abs(got - want).max() <= 0.04 and rel_l2(got, want) <= 1e-2, (tokens, quant, config)


def test_decode_attention_long_context_and_determinism():
    from kernels import DecodeAttention
    batch, capacity, group = 1, 32768, 4
    q, k, v, _, _ = attention_case(batch, 1, capacity, 101)
    first = capacity - 1
    pos = torch.tensor([first], device="cuda", dtype=torch.int32)
    att = DecodeAttention(batch, 8, group, 128, capacity, "cuda")
    a = att(q, k, v, pos).clone()
    b = att(q, k, v, pos).clone()
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    want = oracle_attention(q, k, v, first, 1, group)
    got = a.float().cpu().numpy()
    assert np.abs(got - want).max() <= 0.04 and rel_l2(got, want) <= 1e-2


def test_decode_attention_graph_replays_follow_pos():
    """The grid is fixed and the live length comes from pos on the device: one captured call,
    replayed at several positions, matches the eager call at each (replays interleaved with
    eager work and synchronisations)."""
    from kernels import DecodeAttention
    batch, capacity, group = 2, 640, 4
    q, k, v, _, _ = attention_case(batch, 1, capacity, 77)
    att = DecodeAttention(batch, 8, group, 128, capacity, "cuda")
    pos = torch.tensor([10], device="cuda", dtype=torch.int32)
    att(q, k, v, pos)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            out = att(q, k, v, pos)
    torch.cuda.current_stream().wait_stream(stream)
    for first in (10, 300, 639, 0, 511):
        pos.fill_(first)
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = DecodeAttention(batch, 8, group, 128, capacity, "cuda", config=att.splits)(q, k, v, pos)
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), first


def test_decode_attention_tuned_keeps_agreement():
    from kernels import DecodeAttention
    batch, capacity, group = 1, 2048, 4
    _, k, v, _, _ = attention_case(batch, 1, capacity, 13)
    att = DecodeAttention(batch, 8, group, 128, capacity, "cuda")
    best = att.tuned([k], [v], 100, capacity - 1, use_graph=True)
    q, _, _, _, _ = attention_case(batch, 1, capacity, 14)
    pos = torch.tensor([capacity - 1], device="cuda", dtype=torch.int32)
    want = oracle_attention(q, k, v, capacity - 1, 1, group)
    got = best(q, k, v, pos).float().cpu().numpy()
    assert rel_l2(got, want) <= 1e-2
