"""GPU parity of the reference-API drop-ins: cuda_fp8, fp8, cuda_int8, cuda_small, swiglu, norm.

Ports of the reference's own checks -- tests/test_engine.py:431-490 (layouts, 4-bit
packing) and bench/gpu_checks.py (check_fp8, check_fp8_mma, check_int4,
check_partial_swiglu, check_separate_decode_norm, check_cuda_small) and
bench/next_probe.py (check_reference, check_integer_norm) -- with the same seeds and
tolerances, run through the C ABI on MI355X, plus byte-exact comparison with the golden
vectors written from the reference's own functions.
"""

import importlib
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_quant.npz")


def kmod(name):
    return importlib.import_module(f"kernels.{name}")


def bits16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(u16):
    return torch.from_numpy(np.ascontiguousarray(u16).view(np.int16)).view(torch.bfloat16)


def test_golden_quantize_prepare_fp8_int8_bytes():
    """Every golden vector of the reference's quantize/prepare/fp8/int8 functions, byte for byte."""
    cuda_fp8, fp8, cuda_int8 = kmod("cuda_fp8"), kmod("fp8"), kmod("cuda_int8")
    d = np.load(GOLDEN)
    assert np.array_equal(cuda_fp8._permutation("cpu").numpy(), d["permutation"])
    for name in "abc":
        w = from_bits(d[f"{name}_w"]).to(DEV)
        k = w.shape[1]
        for bits in (8, 4):
            for group in (64, 128):
                if f"{name}_q{bits}_g{group}" not in d:
                    continue
                q, s, b = cuda_fp8.quantize(w, group=group, bits=bits)
                assert np.array_equal(q.cpu().numpy(), d[f"{name}_q{bits}_g{group}"]), (name, bits, group)
                assert np.array_equal(bits16(s), d[f"{name}_s{bits}_g{group}"]), (name, bits, group)
                deq = cuda_fp8.dequantize((q, s, b))
                assert np.array_equal(bits16(deq), d[f"{name}_deq{bits}_g{group}"]), (name, bits, group)
        packed = cuda_fp8.quantize(w)
        tiled = cuda_fp8.prepare(packed, tiled=True)
        flat = cuda_fp8.prepare(packed, tiled=False)
        assert np.array_equal(tiled.weight.cpu().numpy(), d[f"{name}_prep8_tiled"])
        assert np.array_equal(flat.weight.cpu().numpy(), d[f"{name}_prep8_rowmajor"])
        assert np.array_equal(tiled.row_major().cpu().numpy(), d[f"{name}_prep8_rowmajor"])
        assert np.array_equal(bits16(tiled.scale), d[f"{name}_prep8_scale"])
        i8 = cuda_int8.Prepared(tiled)
        assert np.array_equal(i8.weight.cpu().view(torch.uint8).numpy(), d[f"{name}_int8_prepared"])
        four = cuda_fp8.prepare(cuda_fp8.quantize(w, bits=4), tiled=True)
        assert np.array_equal(four.weight.cpu().numpy(), d[f"{name}_prep4_tiled"])
        for group in (128, k):
            e, s = fp8.quantize(w, group=group)
            assert np.array_equal(e.view(torch.uint8).cpu().numpy(), d[f"{name}_fp8_g{group}"]), (name, group)
            assert np.array_equal(bits16(s), d[f"{name}_fp8s_g{group}"]), (name, group)


def test_tiled_weight_layout_round_trips():
    """tests/test_engine.py:431-451 on the GPU."""
    cuda_fp8 = kmod("cuda_fp8")
    torch.manual_seed(0)
    weight = torch.randn(64, 256, dtype=torch.bfloat16).to(DEV)
    packed = cuda_fp8.quantize(weight)
    rowmajor = cuda_fp8.prepare(packed, tiled=False)
    tiled = cuda_fp8.prepare(packed, tiled=True)
    assert tiled.tiled and not rowmajor.tiled
    assert tiled.weight.shape == rowmajor.weight.shape
    assert not torch.equal(tiled.weight, rowmajor.weight)
    assert torch.equal(tiled.row_major(), rowmajor.weight)
    tile = tiled.weight.view(4, 2, 2, 2, 8, 4, 16)[1, 0]
    rows = rowmajor.weight.view(4, 16, 2, 2, 4, 16)[1, :, 0]
    assert torch.equal(tile[0, 0, 3, 2], rows[3, 0, 2])
    assert torch.equal(tile[1, 1, 5, 1], rows[13, 1, 1])
    assert tiled.bytes_moved() == rowmajor.bytes_moved()


def test_int4_weights_pack_two_values_per_byte():
    """tests/test_engine.py:454-490 on the GPU."""
    cuda_fp8 = kmod("cuda_fp8")
    torch.manual_seed(1)
    weight = torch.randn(32, 256, dtype=torch.bfloat16).to(DEV)
    packed = cuda_fp8.quantize(weight, bits=4)
    bytes_, scale, bits = packed
    assert bits == 4 and bytes_.min() >= 1 and bytes_.max() <= 15
    exact = cuda_fp8.dequantize(packed).float()
    rel = ((exact - weight.float()).norm() / weight.float().norm()).item()
    assert 0.02 < rel < 0.2
    step = scale.float().repeat_interleave(64, dim=1)
    assert ((exact - weight.float()).abs() <= step * 0.5 + exact.abs() * 2 ** -8 + 1e-6).all()
    eight = cuda_fp8.prepare(cuda_fp8.quantize(weight), tiled=True)
    four = cuda_fp8.prepare(packed, tiled=True)
    assert four.bits == 4 and four.weight.shape == (32, 128)
    assert four.weight.numel() * 2 == eight.weight.numel()
    assert four.bytes_moved() == four.weight.numel() + four.scale.numel() * 2
    tile4 = four.weight.view(2, 2, 2, 8, 4, 16)[0, 0]
    values8 = cuda_fp8.quantize(weight, bits=4)[0]
    codes = cuda_fp8.prepare((values8, scale, 8), tiled=True).weight.view(2, 2, 2, 2, 8, 4, 16)[0, 0]
    assert torch.equal(tile4 & 0x0F, codes[:, 0]) and torch.equal(tile4 >> 4, codes[:, 1])
    with pytest.raises(ValueError):
        cuda_fp8.prepare(packed, tiled=False)


def _ref_linear(x, exact):
    return F.linear(x.float(), exact.float())


@pytest.mark.parametrize("bits", [8, 4])
def test_cuda_fp8_matmul_planes_swiglu(bits):
    """check_fp8_mma (seed 53) and check_int4 (seed 71), bench/gpu_checks.py:122-204, 392-448."""
    cuda_fp8 = kmod("cuda_fp8")
    norm = kmod("norm")
    torch.manual_seed(53 if bits == 8 else 71)
    configs = [c for c in cuda_fp8.CONFIGS if c[1] in (1, 4, 16)][:4]
    for n, k in ((6144, 2560), (2560, 4096), (2560, 9728), (19456, 2560)):
        weight = (torch.randn(n, k, dtype=torch.bfloat16, device=DEV) * 0.02)
        packed = cuda_fp8.quantize(weight, bits=bits)
        for tiled in ((True, False) if bits == 8 else (True,)):
            prepared = cuda_fp8.prepare(packed, tiled=tiled)
            exact = cuda_fp8.dequantize(packed)
            for batch in (1, 3, 8, 17, 32):
                x = torch.randn(batch, k, dtype=torch.bfloat16, device=DEV)
                reference = _ref_linear(x, exact)
                scale = reference.abs().max().item()
                for config in configs:
                    out = cuda_fp8.matmul(x, prepared, config=config).float()
                    err = (out - reference).abs().max().item() / scale
                    assert torch.isfinite(out).all() and err <= 1e-2, (bits, n, k, batch, config, err)
                    l2 = ((out - reference).norm() / reference.norm()).item()
                    assert l2 <= 1e-2, (bits, n, k, batch, config, l2)
                    if cuda_fp8.splits(prepared, batch, config) > 1:
                        planes = cuda_fp8.matmul_partials(x, prepared, config)
                        assert planes.shape[0] == cuda_fp8.splits(prepared, batch, config)
                        acc = torch.zeros_like(planes[0])
                        for p in planes:
                            acc += p
                        assert torch.equal(acc.to(torch.bfloat16).float(), out), "planes == reduced split path"
                        if n == 2560:
                            residual = torch.randn(batch, n, dtype=torch.bfloat16, device=DEV)
                            gain = torch.randn(n, dtype=torch.bfloat16, device=DEV)
                            r0, y0 = norm.add_rms_norm(residual, out.to(torch.bfloat16), gain, 1e-6)
                            r1, y1 = norm.add_rms_norm_partials(residual, planes, gain, 1e-6)
                            assert torch.equal(r0, r1) and torch.equal(y0, y1)
                if n == 19456 and batch <= 32:
                    inter = n // 2
                    want = (F.silu(reference[:, :inter].to(torch.bfloat16)).to(torch.bfloat16).float()
                            * reference[:, inter:].to(torch.bfloat16).float())
                    for config in cuda_fp8.SWIGLU_CONFIGS[:2]:
                        got = cuda_fp8.gate_up_swiglu(x, prepared, config=config).float()
                        err = (got - want).abs().max().item() / want.abs().max().item()
                        assert torch.isfinite(got).all() and err <= 2e-2, (bits, batch, config, err)


def test_fp8_matmul_groups_partial_tiles_zero_row():
    """check_fp8 (seed 59), bench/gpu_checks.py:89-119: 73 rows, groups 64 and 128."""
    fp8 = kmod("fp8")
    torch.manual_seed(59)
    for group in (64, 128):
        weight = torch.randn(73, 384, dtype=torch.bfloat16, device=DEV)
        weight[0].zero_()
        packed, scales = fp8.quantize(weight, group=group)
        restored = (packed.float().view(73, -1, group) * scales.float()[:, :, None]).reshape_as(weight).bfloat16()
        for batch in (1, 2, 3, 4, 16):
            x = torch.randn(batch, 384, dtype=torch.bfloat16, device=DEV)
            expected = _ref_linear(x, restored)
            scale = expected.abs().max().item()
            for config in ((32, 4, 4, 1), (16, 4, 4, 4), None):
                actual = fp8.fp8_matmul(x, (packed, scales), config=config)
                relative = (actual.float() - expected).abs().max().item() / scale
                assert torch.isfinite(actual).all() and relative <= 0.02, (group, batch, config, relative)
                assert torch.count_nonzero(actual[:, 0]).item() == 0, "zero row preserved"


def test_cuda_int8_quantize_matmul_add_norm_quant():
    """next_probe.check_reference / check_integer_norm (seed 71) and the oracle's W8A8 product."""
    cuda_fp8, cuda_int8, norm = kmod("cuda_fp8"), kmod("cuda_int8"), kmod("norm")
    torch.manual_seed(71)
    for n, k in ((64, 256), (2560, 4096)):
        w = torch.randn(n, k, device=DEV, dtype=torch.bfloat16) * (0.02 if n > 64 else 1.0)
        packed = cuda_fp8.quantize(w)
        source = cuda_fp8.prepare(packed)
        prepared = cuda_int8.Prepared(source)
        for m in (1, 3, 16, 32):
            x = torch.randn(m, k, device=DEV, dtype=torch.bfloat16)
            q, s, _, _ = cuda_int8.quantize_activation(x)
            oq, os_ = O.int8_quantize_activation(bits16(x))
            assert np.array_equal(q.cpu().numpy(), oq) and np.array_equal(s.cpu().numpy(), os_)
            q1, s1, q2, s2 = cuda_int8.quantize_activation(x, components=2)
            assert torch.equal(q1, q) and torch.equal(s1, s)
            _, _, oq2, os2 = O.int8_quantize_activation(bits16(x), components=2)
            assert np.array_equal(q2.cpu().numpy(), oq2) and np.array_equal(s2.cpu().numpy(), os2), \
                (n, k, m, "second component vs oracle")
            want = O.linear_w8a8_int8(bits16(x), prepared.weight.cpu().numpy(), bits16(prepared.scale))
            for config in ((4, 1), (8, 2), (4, 4)):
                got = cuda_int8.matmul(x, prepared, config=config).float().cpu().numpy()
                err = np.abs(got - want).max() / np.abs(want).max()
                assert err <= 1e-2, (n, k, m, config, err)
                two = cuda_int8.matmul(x, prepared, config=config, components=2).float().cpu().numpy()
                exact = x.float().cpu().numpy() @ cuda_fp8.dequantize(packed).float().cpu().numpy().T
                assert O.rel_l2(two, exact) <= O.rel_l2(got, exact) + 1e-3, "residual component refines"
            if n % 32 == 0:
                sw = cuda_int8.matmul(x, prepared, config=(4, 1), mode=2).float().cpu().numpy()
                full = cuda_int8.matmul(x, prepared, config=(4, 1)).cpu()
                ref = O.bf16_to_f32(O.swiglu(bits16(full)))
                assert O.rel_l2(sw, ref) <= 2e-2
    for m in (1, 3, 16, 24, 32):
        for splits in (1, 2, 4, 8):
            x = torch.randn(m, 2560, device=DEV, dtype=torch.bfloat16)
            delta = torch.randn(splits, m, 2560, device=DEV, dtype=torch.float32)
            weight = torch.randn(2560, device=DEV, dtype=torch.bfloat16)
            want_res, want_norm = norm.add_rms_norm_partials(x, delta, weight, 1.e-6)
            expected = cuda_int8.quantize_activation(want_norm)
            got_res, actual = cuda_int8.add_norm_quant(x, delta, weight, 1.e-6)
            assert torch.equal(got_res, want_res), (m, splits)
            assert torch.equal(actual[0], expected[0]) and torch.equal(actual[1], expected[1]), (m, splits)
            o_res, o_q, o_s = O.add_norm_quant(bits16(x), delta.cpu().numpy(), bits16(weight), 1.e-6)
            assert np.array_equal(bits16(got_res), o_res), (m, splits, "residual vs oracle")
            assert np.array_equal(actual[0].cpu().numpy(), o_q), (m, splits, "int8 codes vs oracle")
            assert np.array_equal(actual[1].cpu().numpy(), o_s), (m, splits, "scales vs oracle")


def test_plane_consumers_bit_exact():
    """check_separate_decode_norm (812), check_partial_swiglu, check_cuda_small (29) vs the oracle."""
    cuda_small, swiglu_mod, norm = kmod("cuda_small"), kmod("swiglu"), kmod("norm")
    torch.manual_seed(29)
    worst = 0
    for rows in (1, 3, 4, 8, 16, 17, 32, 64):
        x = torch.randn(rows, 2560, dtype=torch.bfloat16, device=DEV)
        w = (1.0 + 0.1 * torch.randn(2560, dtype=torch.bfloat16)).to(torch.bfloat16).to(DEV)
        for splits in (1, 2, 4, 8, 16):
            planes = torch.randn(splits, rows, 2560, dtype=torch.float32, device=DEV)
            r1, y1 = cuda_small.add_rms_norm_partials_separate(x, planes, w, 1e-6)
            r0 = O.residual_partials(bits16(x), planes.cpu().numpy())
            assert np.array_equal(bits16(r1), r0), (rows, splits)
            y0 = O.rms_norm(r0, bits16(w), 1e-6)
            assert np.array_equal(bits16(y1), y0), (rows, splits, "exact-sum RMSNorm is bit-exact")
            r2, y2 = norm.add_rms_norm_partials(x, planes, w, 1e-6)
            assert torch.equal(r2, r1) and torch.equal(y2, y1)
            r3, y3 = norm.add_rms_norm_partials_separate(x, planes, w, 1e-6)
            assert torch.equal(r3, r1) and torch.equal(y3, y1)
            assert torch.equal(norm.rms_norm(r1, w, 1e-6), y1), "rms_norm of the residual"
            d = torch.randn(rows, 2560, dtype=torch.bfloat16, device=DEV)
            r4, y4 = norm.add_rms_norm_separate(x, d, w, 1e-6)
            r5, y5 = O.add_rms_norm(bits16(x), bits16(d), bits16(w), 1e-6)
            assert np.array_equal(bits16(r4), r5) and np.array_equal(bits16(y4), y5), (rows, "separate form")
            reduced = torch.empty(rows, 2560, dtype=torch.bfloat16, device=DEV)
            cuda_fp8 = kmod("cuda_fp8")
            cuda_fp8._module_for(1, 1).kernel("reduce_partials")(0, 256, planes, reduced, reduced.numel(), splits)
            assert np.array_equal(bits16(reduced), O.reduce_partials(planes.cpu().numpy()))
        for splits in (1, 4, 8):
            planes = torch.randn(splits, rows, 2 * 9728, dtype=torch.float32, device=DEV)
            a = swiglu_mod.swiglu_partials(planes)
            ref = O.swiglu_partials(planes.cpu().numpy())
            ulps = np.abs(bits16(a).astype(np.int32) - ref.astype(np.int32)).max()
            worst = max(worst, ulps)
            assert ulps <= 1, (rows, splits, ulps)
            reduced = torch.empty(rows, 2 * 9728, dtype=torch.bfloat16, device=DEV)
            kmod("cuda_fp8")._module_for().kernel("reduce_partials")(0, 256, planes, reduced, reduced.numel(), splits)
            assert torch.equal(swiglu_mod.swiglu(reduced), a), "swiglu(reduce(planes)) == swiglu_partials"
    print(f"plane consumers: worst difference {worst} bf16 ulp")


def test_norm_and_swiglu_match_transformers_qwen3():
    """tests/test_numerics.py:45-64, 103-116: the kernels against transformers' Qwen3 modules."""
    from transformers.models.qwen3.configuration_qwen3 import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3MLP, Qwen3RMSNorm
    norm, swiglu_mod = kmod("norm"), kmod("swiglu")
    torch.manual_seed(0)
    x = torch.randn(64, 2560, dtype=torch.bfloat16)
    ref = Qwen3RMSNorm(2560, eps=1e-6).to(torch.bfloat16)
    ref.weight.data = torch.randn(2560, dtype=torch.bfloat16)
    with torch.no_grad():
        want = ref(x)
    got = norm.rms_norm(x.to(DEV), ref.weight.data.to(DEV), 1e-6).cpu()
    ulps = (got.view(torch.int16).int() - want.view(torch.int16).int()).abs().max().item()
    assert ulps <= 1
    torch.manual_seed(3)
    cfg = Qwen3Config(hidden_size=2560, intermediate_size=9728, num_hidden_layers=1, num_attention_heads=32,
                      num_key_value_heads=8, head_dim=128, rms_norm_eps=1e-6, rope_theta=5e6)
    mlp = Qwen3MLP(cfg).to(torch.bfloat16)
    xs = torch.randn(32, 2560, dtype=torch.bfloat16)
    with torch.no_grad():
        gate, up = mlp.gate_proj(xs), mlp.up_proj(xs)
        reference = mlp.act_fn(gate) * up
    got = swiglu_mod.swiglu(torch.cat([gate, up], dim=1).to(DEV)).cpu()
    ulps = (got.view(torch.int16).int() - reference.view(torch.int16).int()).abs().max().item()
    assert ulps <= 1


def test_drop_in_error_conventions():
    cuda_fp8 = kmod("cuda_fp8")
    w = torch.randn(64, 256, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        cuda_fp8.quantize(w, bits=3)
    with pytest.raises(ValueError):
        cuda_fp8.quantize(w[:, :200].contiguous())
    with pytest.raises(ValueError):
        cuda_fp8.Prepared(torch.zeros(24, 256, dtype=torch.uint8, device=DEV),
                          torch.zeros(24, 4, dtype=torch.float16, device=DEV))
    prepared = cuda_fp8.prepare(cuda_fp8.quantize(w))
    with pytest.raises(ValueError):
        cuda_fp8.matmul(torch.randn(1, 128, dtype=torch.bfloat16, device=DEV), prepared)
    with pytest.raises(ValueError):
        cuda_fp8.quantize(w.cpu())  # no CPU path
    assert cuda_fp8.ready()
