"""The persistent single-call GEMMs: a projection with at least two row blocks per workgroup --
the 151936-row lm_head -- runs as persistent workgroups looping over row blocks, W4A16 with its
code-bias totals computed on the first row block only. W4A16 at one tile per wave takes the
direct-to-LDS weight ring (gemm_ring_w4_kernel: two workgroups per CU with 3-step rings at 1-4
tokens, one with 4-step rings at 8 and 16); FP8 the register pipeline (gemm_persist_kernel).
Their outputs must be bit-identical to the one-workgroup-per-row-block kernel on the same
plan: a slice of whole tiles of the same tile-layout weight (too few row blocks for a
persistent launch) gives the same rows bit for bit. SwiGLU outputs of a persistent launch are
within one bf16 step of the SwiGLU of its own bf16 outputs, and everything is within the
north star's rel-L2 of the oracle."""

import numpy as np
import pytest
import torch

import oracle as O
from kernels import qlinear

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def tile_slice(t, t0, t1):
    """Rows [16 t0, 16 t1) of a tile-layout weight: tiles are stored one after another."""
    per_tile = t.weight.numel() // (t.rows // 16)
    w = t.weight.reshape(-1)[t0 * per_tile:t1 * per_tile].reshape(16 * (t1 - t0), -1)
    return qlinear.Tiled(w, t.scale[16 * t0:16 * t1], 16 * (t1 - t0), t.k, t.fmt)


@pytest.mark.parametrize("fmt", ["w4a16", "fp8"])
@pytest.mark.parametrize("m", [1, 4, 8, 16])
def test_persistent_lm_head_equals_per_block_kernel(fmt, m):
    print(f"persistent lm_head {fmt} m={m}", flush=True)
    n, k = 151936, 2560
    g = torch.Generator(device=DEV).manual_seed(40 + m)
    w = (torch.randn(n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    quant, linear, _ = qlinear.FORMATS[fmt]
    packed = quant(w)
    t = qlinear.prepare(packed, fmt)
    x = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16)
    cfg = (8, 1, 1, 1)  # 8 waves, one per tile, whole K: 1187 row blocks
    full = linear(x, t, config=cfg)
    ntiles = n // 16
    for t0 in (0, 4000, ntiles - 128):
        part = linear(x, tile_slice(t, t0, t0 + 128), config=cfg)  # 16 row blocks: one per workgroup
        assert torch.equal(full[:, 16 * t0:16 * (t0 + 128)], part), (fmt, m, t0)
    rows = np.arange(0, n, 97)
    q, s = packed
    qn = q.view(torch.uint8 if fmt == "fp8" else q.dtype).cpu().numpy()[rows]
    sn = s.cpu().view(torch.int16).numpy().view(np.uint16)[rows]
    xb = x.cpu().view(torch.int16).numpy().view(np.uint16)
    if fmt == "fp8":
        want = O.linear_fp8_w8a8(xb, qn, sn[:, None])
    else:
        want = O.linear_dequant(xb, O.dequantize(O.unpack_int4_k32(qn), sn, bits=4, scale_dtype="bf16"))
    assert O.rel_l2(full.float().cpu().numpy()[:, rows], want) <= 1e-2


def test_persistent_swiglu_w4():
    """A gate_up-shaped W4A16 weight with enough rows for the persistent launch (2 x 40960 rows,
    640 row blocks): SwiGLU output within one bf16 step of the SwiGLU of the bf16 output."""
    inter, k, m = 40960, 512, 4
    g = torch.Generator(device=DEV).manual_seed(9)
    w = (torch.randn(2 * inter, k, generator=g, device=DEV) * 0.05).to(torch.bfloat16)
    t = qlinear.prepare(qlinear.quantize_w4(w), "w4a16")
    x = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16)
    cfg = (8, 1, 1, 1)
    act = qlinear.linear_w4a16(x, t, config=cfg, swiglu=True)
    both = qlinear.linear_w4a16(x, t, config=cfg)
    want = torch.from_numpy(O.bf16_to_f32(O.swiglu(both.cpu().view(torch.int16).numpy().view(np.uint16))))
    got = act.float().cpu()
    tol = 2.0 ** -7 * want.abs() + 1e-6
    assert bool(((got - want).abs() <= tol).all())


@pytest.mark.parametrize("m", [1, 4])
def test_ring_row_major_equals_tiled(m):
    """The ring kernel reads tile-layout weights through a buffer resource (a scalar offset per
    2 KB step) and row-major packed weights through per-lane addresses: the same codes reach
    the same lanes, so the lm_head output is bit-identical either way."""
    print(f"ring row-major vs tiled m={m}", flush=True)
    n, k = 151936, 2560
    g = torch.Generator(device=DEV).manual_seed(60 + m)
    w = (torch.randn(n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    packed = qlinear.quantize_w4(w)
    t = qlinear.prepare(packed, "w4a16")
    x = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16)
    cfg = (8, 1, 1, 1)
    assert torch.equal(qlinear.linear_w4a16(x, t, config=cfg), qlinear.linear_w4a16(x, packed, config=cfg))
