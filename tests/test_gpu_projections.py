"""GPU parity of every Qwen3-4B projection shape in every north-star format at the batches
BASELINE configs 2 and 3 name, the lm_head included, and of the fused GEMM + residual add +
RMSNorm (``cuda_fp8.matmul_add_norm``), against the CPU oracle through the C ABI.

* Config 2 (FP8 W8A8): qkv, o, gate_up (2560 -> 2 x 9728, with the fused SwiGLU) and down
  at M = 1 and 8; config 3 (W4A16 g128): the same four plus the lm_head 2560 -> 151936 at
  M = 1, 4 and 8; the lm_head in all three formats. Weights are N(0, 0.02), activations
  N(0, 1). The oracle multiplies in fp64 (dequantize-then-matmul, or (x_q s_x)(w_q s_w)^T
  for FP8); the bar is the north star's relative L2 <= 1e-2. The lm_head is checked on a
  fixed sample of 2048 of its rows (the product of all 151936 in fp64 is minutes of CPU).
* The codes the linears consume are the library's own pack output, which
  tests/test_gpu_qlinear.py checks bit for bit against the oracle's pack.
* ``matmul_add_norm`` (engine/kernels/cuda_fp8.py:1333-1374): the delta it leaves in
  scratch within rel-L2 1e-2 of the oracle's product, and the new residual and the normed
  output bit-exact against ``oracle.add_rms_norm`` of that delta, at batch 1, 8 and 16.
"""

import numpy as np
import pytest
import torch

import oracle as O
from kernels import cuda_fp8, qlinear

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

QWEN = {"qkv": (6144, 2560), "o": (2560, 4096), "gate_up": (19456, 2560), "down": (2560, 9728),
        "lm_head": (151936, 2560)}
SAMPLE = 2048
SEEDS = {"qkv": 11, "o": 12, "gate_up": 13, "down": 14, "lm_head": 15}


def bits16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def weight(name, seed):
    n, k = QWEN[name]
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16)


def acts(m, k, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(m, k, generator=g).to(torch.bfloat16)


def sample_rows(n, swiglu):
    """Rows checked: all of them, or for the lm_head a fixed sample including both ends."""
    if n <= 20000:
        return np.arange(n // 2 if swiglu else n)
    rng = np.random.default_rng(n)
    return np.unique(np.concatenate([[0, 1, n - 1], rng.choice(n, SAMPLE, replace=False)]))


def oracle_rows(fmt, packed, rows, x_bits, swiglu):
    """The oracle's output at the given output columns (gate rows i and I + i for SwiGLU)."""
    q, s = packed
    n = q.shape[0]
    pick = np.concatenate([rows, rows + n // 2]) if swiglu else rows
    qn, sn = q.view(torch.uint8 if fmt == "fp8" else q.dtype).cpu().numpy()[pick], bits16(s)
    sn = sn[pick]
    if fmt == "fp8":
        y = O.linear_fp8_w8a8(x_bits, qn, sn[:, None])
    elif fmt == "w4a16":
        y = O.linear_dequant(x_bits, O.dequantize(O.unpack_int4_k32(qn), sn, bits=4, scale_dtype="bf16"))
    else:
        y = O.linear_dequant(x_bits, O.dequantize(qn, sn[:, None], scale_dtype="bf16", storage="signed"))
    if swiglu:
        return O.bf16_to_f32(O.swiglu(O.f32_to_bf16(y.astype(np.float32))))  # [gate rows | up rows]
    return y


CASES = ([("fp8", name, m) for name in ("qkv", "o", "gate_up", "down", "lm_head") for m in (1, 8)]
         + [("w4a16", name, m) for name in ("qkv", "o", "gate_up", "down", "lm_head") for m in (1, 4, 8)]
         + [("w8a16", "lm_head", m) for m in (1, 8)])


@pytest.mark.parametrize("fmt,name,m", CASES)
def test_qwen3_projection(fmt, name, m):
    print(f"projection {fmt} {name} m={m}", flush=True)
    n, k = QWEN[name]
    swiglu = name == "gate_up"
    quant, linear, _ = qlinear.FORMATS[fmt]
    packed = quant(weight(name, SEEDS[name]))
    tiles = qlinear.prepare(packed, fmt)
    x = acts(m, k, 7 * m + len(name))
    rows = sample_rows(n, swiglu)
    want = oracle_rows(fmt, packed, rows, bits16(x), swiglu)
    for operand in (tiles, packed) if m == 1 and name != "lm_head" else (tiles,):
        y = linear(x.to(DEV), operand, swiglu=swiglu).float().cpu().numpy()[:, rows]
        err = O.rel_l2(y, want)
        assert np.isfinite(y).all() and err <= 1e-2, (fmt, name, m, err)


def _ref_weights(kind, w):
    if kind == "ref8-rowmajor":
        return cuda_fp8.prepare(cuda_fp8.quantize(w), tiled=False)
    if kind == "ref8-tiled":
        return cuda_fp8.prepare(cuda_fp8.quantize(w), tiled=True)
    if kind == "ref4":
        return cuda_fp8.prepare(cuda_fp8.quantize(w, bits=4))
    return cuda_fp8.prepare(cuda_fp8.quantize(w, bits=4 if kind == "w4a16" else 8, fmt=kind))


@pytest.mark.parametrize("kind", ["ref8-rowmajor", "ref8-tiled", "ref4", "w8a16", "w4a16", "fp8"])
@pytest.mark.parametrize("name", ["o", "down"])
def test_matmul_add_norm_single_launch(kind, name):
    n, k = QWEN[name]
    w = weight(name, 31)
    prepared = _ref_weights(kind, w)
    bits = 4 if kind in ("ref4", "w4a16") else 8
    exact = cuda_fp8.dequantize(cuda_fp8.quantize(w, bits=bits, fmt="ref" if kind.startswith("ref") else kind))
    exact = exact.float().cpu().numpy()
    g = torch.Generator().manual_seed(17)
    gain = (1.0 + 0.1 * torch.randn(n, generator=g)).to(torch.bfloat16)
    for batch in (1, 8, 16):
        print(f"matmul_add_norm {kind} {name} batch={batch}", flush=True)
        x = acts(batch, k, 50 + batch)
        residual = acts(batch, n, 60 + batch)
        scratch = cuda_fp8.add_norm_scratch(batch, n, DEV)
        for call in range(2):  # the counter is left at zero for the next call
            res, normed = cuda_fp8.matmul_add_norm(x.to(DEV), prepared, residual.to(DEV), gain.to(DEV), 1e-6, scratch)
            torch.cuda.synchronize()
            assert scratch[1].item() == 0, (kind, batch, call)
            delta = bits16(scratch[0])
            if kind == "fp8":
                q, s = cuda_fp8.quantize(w, fmt="fp8")[:2]
                want = O.linear_fp8_w8a8(bits16(x), q.view(torch.uint8).cpu().numpy(), bits16(s)[:, None])
            else:
                want = x.float().numpy().astype(np.float64) @ exact.astype(np.float64).T
            err = O.rel_l2(O.bf16_to_f32(delta), want)
            assert err <= 1e-2, (kind, name, batch, err)
            r_want, y_want = O.add_rms_norm(bits16(residual), delta, bits16(gain), 1e-6)
            assert np.array_equal(bits16(res), r_want), (kind, name, batch)
            assert np.array_equal(bits16(normed), y_want), (kind, name, batch)


@pytest.mark.parametrize("fmt", ["w4a16", "w8a16", "fp8"])
@pytest.mark.parametrize("m", [1, 8, 17])
def test_reference_signatures_on_north_star_weights(fmt, m):
    """The engine's call sites (engine.py:881-906, 950-951) on north-star weights: weights from
    ``cuda_fp8.prepare(cuda_fp8.quantize(w, bits, fmt=...))``, then ``cuda_fp8.matmul`` (o and
    qkv), ``matmul_partials`` with the reference's split-K configs (planes summed in slice
    order == the reduced matmul's fp32 sum within one bf16 rounding, ``splits`` = plane count)
    and ``gate_up_swiglu`` (gate_up with the fused SwiGLU), each against the oracle's product at
    rel-L2 <= 1e-2. 17 tokens take the skinny GEMM behind the same signatures."""
    bits = 4 if fmt == "w4a16" else 8
    for name in ("qkv", "o", "gate_up"):
        print(f"reference signatures {fmt} {name} m={m}", flush=True)
        n, k = QWEN[name]
        w = weight(name, SEEDS[name] + 100)
        packed = cuda_fp8.quantize(w, bits=bits, fmt=fmt)
        prepared = cuda_fp8.prepare(packed)
        assert prepared.bits == bits and prepared.k == k and prepared.rows == n
        x = acts(m, k, 90 + m + len(name))
        swiglu = name == "gate_up"
        rows = sample_rows(n, swiglu)
        want = oracle_rows(fmt, packed[:2], rows, bits16(x), swiglu)
        if swiglu:
            y = cuda_fp8.gate_up_swiglu(x.to(DEV), prepared, config=(8, 1, 1, 1, 0))
            err = O.rel_l2(y.float().cpu().numpy()[:, rows], want)
            assert tuple(y.shape) == (m, n // 2) and err <= 1e-2, (fmt, name, m, err)
            continue
        y = cuda_fp8.matmul(x.to(DEV), prepared, config=(8, 1))
        err = O.rel_l2(y.float().cpu().numpy()[:, rows], want)
        assert tuple(y.shape) == (m, n) and err <= 1e-2, (fmt, name, m, err)
        if m > 16:
            continue  # split-K planes are a decode-kernel output (B <= 16 here)
        for config in ((8, 2, 1, 1, 0), (4, 4, 1, 1, 2), (8, 16, 1, 1, 2)):
            planes = cuda_fp8.matmul_partials(x.to(DEV), prepared, config)
            assert planes.dtype == torch.float32 and tuple(planes.shape[1:]) == (m, n)
            assert planes.shape[0] == cuda_fp8.splits(prepared, m, config), (fmt, name, config)
            total = planes[0].clone()
            for p in planes[1:]:
                total += p
            err = O.rel_l2(total.cpu().numpy()[:, rows], want)
            assert err <= 1e-2, (fmt, name, m, config, err)
            diff = (total.bfloat16().float() - y.float()).abs()
            tol = 2.0 ** -7 * y.float().abs() + 2.0 ** -9 * y.float().abs().amax(dim=1, keepdim=True)
            assert bool((diff <= tol).all()), (fmt, name, m, config, "planes vs matmul")
