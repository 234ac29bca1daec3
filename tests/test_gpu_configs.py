"""GPU parity at the measurement configurations (BASELINE configs 1 and 4) built exactly as
specified, and the per-shape kernel race (engine/kernels/gemm.py:134-261)."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from kernels import cuda_fp8, gemm, qlinear
from kernels.decode_stack import DecodeStack

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def bits16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def test_config1_w8a16_gemv_down():
    """Config 1: W int8 [2560, 9728] = randint(-127, 128), bf16 scales U(0.001, 0.02),
    x bf16 [1, 9728] = N(0, 1), drawn in that order from one seeded CPU generator."""
    g = torch.Generator().manual_seed(0)
    q = torch.randint(-127, 128, (2560, 9728), generator=g).to(torch.int8)
    s = (torch.rand(2560, generator=g) * (0.02 - 0.001) + 0.001).to(torch.bfloat16)
    x = torch.randn(1, 9728, generator=g).to(torch.bfloat16)
    ref = O.linear_dequant(bits16(x), O.dequantize(q.numpy(), bits16(s)[:, None], bits=8, scale_dtype="bf16",
                                                   storage="signed"))
    packed = (q.to(DEV), s.to(DEV))
    for weight in (packed, qlinear.prepare(packed, "w8a16")):
        y = qlinear.linear_w8a16(x.to(DEV), weight)
        assert O.rel_l2(y.float().cpu().numpy(), ref) < 1e-2


@pytest.mark.parametrize("m", [16, 32, 64])
def test_config4_fused_mlp_w4(m):
    """Config 4: gate_up (2 x 9728 rows) with the SwiGLU epilogue, then down, W4A16 g128,
    at M = 16, 32, 64; against dequantize-then-matmul in fp64 with the reference's SwiGLU
    rounding. At M = 16 also through the decode executor (gate_up -> down chained)."""
    g = torch.Generator().manual_seed(40 + m)
    w_gu = (torch.randn(2 * 9728, 2560, generator=g) * 0.02).to(torch.bfloat16)
    w_dn = (torch.randn(2560, 9728, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(m, 2560, generator=g).to(torch.bfloat16)
    gu = qlinear.quantize_w4(w_gu.to(DEV))
    dn = qlinear.quantize_w4(w_dn.to(DEV))
    act = qlinear.linear_w4a16(x.to(DEV), gu, swiglu=True)
    y = qlinear.linear_w4a16(act, dn)

    def deq(p):
        q, s = p
        return O.dequantize(O.unpack_int4_k32(q.cpu().numpy()), bits16(s), bits=4, scale_dtype="bf16")
    gate_up = O.linear_dequant(bits16(x), deq(gu))
    want_act = O.swiglu(O.f32_to_bf16(gate_up.astype(np.float32)))
    assert O.rel_l2(act.float().cpu().numpy(), O.bf16_to_f32(want_act)) < 1e-2
    want_y = O.linear_dequant(bits16(act), deq(dn))
    assert O.rel_l2(y.float().cpu().numpy(), want_y) < 1e-2
    if m <= 16:
        chain = DecodeStack("w4a16", m)
        a2 = torch.empty_like(act)
        y2 = torch.empty_like(y)
        chain.add(qlinear.prepare(gu), x.to(DEV), a2, swiglu=True).add(qlinear.prepare(dn), a2, y2).build()
        chain.run()
        torch.cuda.synchronize()
        assert not chain.failed()
        assert O.rel_l2(a2.float().cpu().numpy(), O.bf16_to_f32(want_act)) < 1e-2
        assert O.rel_l2(y2.float().cpu().numpy(), O.linear_dequant(bits16(a2), deq(dn))) < 1e-2


@pytest.mark.parametrize("bits", [8, 4])
def test_pick_matmul_races_and_returns_a_valid_kernel(bits):
    """The race returns a callable that agrees with F.linear and reports a rate; family
    restrictions hold (fp8 only, bf16 only)."""
    g = torch.Generator().manual_seed(bits)
    every = [(torch.randn(2560, 2560, generator=g) * 0.02).to(torch.bfloat16).to(DEV) for _ in range(3)]
    packed = [cuda_fp8.prepare(cuda_fp8.quantize(w, bits=bits)) for w in every]
    x = torch.randn(1, 2560, generator=g).to(torch.bfloat16).to(DEV)
    ref = F.linear(x, every[0]).float()
    scale = ref.abs().max().item()
    tol = 0.08 if bits == 8 else 0.3
    fn, transpose, note = gemm.pick_matmul(1, every, reps=1, trials=2, packed=packed)
    assert transpose in (False, "fp8") and "TB/s" in note
    out = fn(x, packed[0] if transpose == "fp8" else every[0])
    assert (out.float() - ref).abs().max().item() / scale < tol
    fn, transpose, note = gemm.pick_matmul(1, every, reps=1, trials=2, packed=packed, family="fp8", quick=True)
    assert transpose == "fp8" and fn.keywords["config"] == cuda_fp8.CONFIGS[0]
    assert (fn(x, packed[0]).float() - ref).abs().max().item() / scale < tol
    fn, transpose, _ = gemm.pick_matmul(1, every, reps=1, trials=2, packed=packed, family="bf16")
    assert fn is F.linear and transpose is False
    with pytest.raises(ValueError):
        gemm.pick_matmul(1, every, reps=1, trials=2, packed=None, family="fp8")
