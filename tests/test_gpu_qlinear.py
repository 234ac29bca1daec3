"""GPU parity of the north-star formats (W8A16, W4A16 g128, FP8 W8A8) against the CPU oracle.

Quantize and pack must be bit-exact; linear outputs must be within relative L2 1e-2 of
the reference's dequantize-then-matmul and close to the exact
per-group statement of what the kernel computes. Every call goes through the C ABI.
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from kernels import _lib, qlinear

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def bits16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def weights(n, k, seed, std=0.02, edge=True):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(n, k, generator=g) * std).to(torch.bfloat16)
    if edge and n >= 8:
        w[0].zero_()
        w[1] = (torch.randn(k, generator=g) * 1e-9).to(torch.bfloat16)
        w[2] = (torch.randn(k, generator=g) * 300.0).to(torch.bfloat16)
        w[3, : k // 2] = 0
    return w


def acts(m, k, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(m, k, generator=g).to(torch.bfloat16)


def test_single_hip_runtime_in_process():
    """The library shares torch's HIP runtime (one libamdhip64 mapped)."""
    _lib.lib()
    torch.zeros(1, device=DEV)
    maps = open("/proc/self/maps").read()
    paths = {line.split()[-1] for line in maps.splitlines() if "libamdhip64" in line}
    assert len(paths) == 1, paths
    assert any("libqlinear.so" in line for line in maps.splitlines())


@pytest.mark.parametrize("n,k,seed", [(64, 256, 0), (256, 2560, 1), (96, 9728, 2)])
def test_quantize_w4_bit_exact(n, k, seed):
    w = weights(n, k, seed)
    q, s = qlinear.quantize_w4(w.to(DEV))
    oq, os_ = O.quantize_int4_g128(bits16(w))
    assert np.array_equal(q.cpu().numpy(), oq)
    assert np.array_equal(bits16(s), os_)
    deq = qlinear.dequantize_w4((q, s))
    assert np.array_equal(bits16(deq), O.dequantize(O.unpack_int4_k32(oq), os_, bits=4, scale_dtype="bf16"))


@pytest.mark.parametrize("n,k,seed", [(64, 256, 0), (128, 9728, 3)])
def test_quantize_w8_bit_exact(n, k, seed):
    w = weights(n, k, seed)
    q, s = qlinear.quantize_w8(w.to(DEV))
    oq, os_ = O.quantize_w8_per_channel(bits16(w))
    assert np.array_equal(q.cpu().numpy(), oq)
    assert np.array_equal(bits16(s), os_)


@pytest.mark.parametrize("n,k,seed", [(64, 256, 0), (128, 2560, 4)])
def test_quantize_fp8_bit_exact(n, k, seed):
    w = weights(n, k, seed)
    q, s = qlinear.quantize_fp8(w.to(DEV))
    oq, os_ = O.fp8_quantize(bits16(w), group=k)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), oq)
    assert np.array_equal(bits16(s), os_[:, 0])


def test_fp8_quantizer_fast_path_is_exact_on_every_input():
    """The FP8 quantizers' quotient (a reciprocal and one fma correction) and hardware cast
    give the codes of IEEE division + clamp + RNE cast on every input they can see: every bf16
    maximum with every bf16 value of no larger magnitude, and every NaN. About 2^30 cases."""
    counts = torch.zeros(66, dtype=torch.int64, device=DEV)
    rc = _lib.lib().qlx_fp8_selfcheck(ctypes.c_void_p(counts.data_ptr()),
                                      ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, _lib.last_error()
    c = counts.cpu().tolist()
    assert c[0] == 0, [hex(v & (2 ** 64 - 1)) for v in c[2:2 + min(c[1], 8)]]


@pytest.mark.parametrize("m", [1, 3, 16])
def test_add_norm_quant_fp8_matches_oracle(m):
    """Fused residual + RMSNorm + FP8 per-token quantize: residual, normed row, codes and scales
    bit-exact against the oracle (add_rms_norm then quantize_fp8_activation), for a bf16 delta,
    fp32 planes and no delta; the codes feed the FP8 GEMM exactly as its own prologue would."""
    g = torch.Generator().manual_seed(101 + m)
    n = 2560
    x = torch.randn(m, n, generator=g).to(torch.bfloat16)
    w = (1.0 + 0.1 * torch.randn(n, generator=g)).to(torch.bfloat16)
    d = torch.randn(m, n, generator=g).to(torch.bfloat16)
    planes = torch.randn(4, m, n, generator=g)
    xd, wd = x.to(DEV), w.to(DEV)
    for kind, delta in (("bf16", d), ("planes", planes), ("none", None)):
        res, code, scale, normed = qlinear.add_norm_quant_fp8(
            xd, None if delta is None else delta.to(DEV), wd, 1e-6, keep_normed=True)
        if kind == "bf16":
            o_res, o_norm = O.add_rms_norm(bits16(x), bits16(d), bits16(w), 1e-6)
        elif kind == "planes":
            o_res, o_norm = O.add_rms_norm_partials(bits16(x), planes.numpy(), bits16(w), 1e-6)
        else:
            o_res, o_norm = None, O.rms_norm(bits16(x), bits16(w), 1e-6)
        if o_res is None:
            assert res is None
        else:
            assert np.array_equal(bits16(res), o_res), (kind, "residual")
        assert np.array_equal(bits16(normed), o_norm), (kind, "normed")
        oq, os_ = O.quantize_fp8_activation(o_norm)
        assert np.array_equal(code.view(torch.uint8).cpu().numpy(), oq), (kind, "codes")
        assert np.array_equal(scale.cpu().numpy().view(np.uint32), os_.view(np.uint32)), (kind, "scales")
    wq = qlinear.quantize_fp8(weights(1024, n, 7, edge=False).to(DEV))
    pre = qlinear.linear_fp8_w8a8_quantized(code, scale, wq)
    fused = qlinear.linear_fp8_w8a8(normed, wq, pre_quantize=False)
    assert torch.equal(pre, fused), "pre-quantized codes = the GEMM's own prologue"


@pytest.mark.parametrize("m,k", [(1, 2560), (3, 9728), (16, 256), (64, 4096)])
def test_quantize_fp8_activation_bit_exact(m, k):
    x = acts(m, k, 11 + m)
    x[0, :7] = torch.tensor([0.0, -0.0, 1e-30, 448.0, -3e4, 2.0 ** -10, 7.0], dtype=torch.bfloat16)
    if m > 1:
        x[1].zero_()
    q, s = qlinear.quantize_fp8_activation(x.to(DEV))
    oq, os_ = O.quantize_fp8_activation(bits16(x))
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), oq)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), os_.view(np.uint32))


SHAPES = [(256, 512), (6144, 2560), (2560, 9728), (2560, 4096)]
BATCHES = [1, 3, 8, 16, 17, 32, 64]


def _check(y, ref_deq, ref_exact, tag):
    yf = y.float().cpu().numpy()
    err = O.rel_l2(yf, ref_deq)
    assert np.isfinite(yf).all(), tag
    assert err <= 1e-2, f"{tag}: rel-L2 vs dequantize-then-matmul {err}"
    exact = O.rel_l2(yf, O.round_bf16(ref_exact.astype(np.float32)))
    assert exact <= 4e-3, f"{tag}: rel-L2 vs exact per-group product {exact}"


@pytest.mark.parametrize("n,k", SHAPES)
def test_linear_w4a16(n, k):
    w = weights(n, k, 5)
    q, s = qlinear.quantize_w4(w.to(DEV))
    oq, os_ = O.quantize_int4_g128(bits16(w))
    codes = O.unpack_int4_k32(oq)
    deq = O.dequantize(codes, os_, bits=4, scale_dtype="bf16")
    for m in BATCHES:
        x = acts(m, k, 100 + m)
        y = qlinear.linear_w4a16(x.to(DEV), (q, s))
        ref = O.linear_dequant(bits16(x), deq)
        exact = O.linear_exact_grouped(bits16(x), codes.astype(np.float64) - 8, O.bf16_to_f32(os_), 128)
        _check(y, ref, exact, f"w4 n={n} k={k} m={m}")
        assert not y[:, 0].float().abs().sum().item(), "zero weight row must give zero"


@pytest.mark.parametrize("n,k", SHAPES)
def test_linear_w8a16(n, k):
    w = weights(n, k, 6)
    q, s = qlinear.quantize_w8(w.to(DEV))
    oq, os_ = O.quantize_w8_per_channel(bits16(w))
    deq = O.dequantize(oq, os_[:, None], scale_dtype="bf16", storage="signed")
    for m in BATCHES:
        x = acts(m, k, 200 + m)
        y = qlinear.linear_w8a16(x.to(DEV), (q, s))
        ref = O.linear_dequant(bits16(x), deq)
        exact = O.linear_exact_grouped(bits16(x), oq, O.bf16_to_f32(os_)[:, None], k)
        _check(y, ref, exact, f"w8 n={n} k={k} m={m}")


@pytest.mark.parametrize("n,k", SHAPES)
def test_linear_fp8_w8a8(n, k):
    w = weights(n, k, 7)
    q, s = qlinear.quantize_fp8(w.to(DEV))
    oq, os_ = O.fp8_quantize(bits16(w), group=k)
    for m in BATCHES:
        x = acts(m, k, 300 + m)
        y = qlinear.linear_fp8_w8a8(x.to(DEV), (q, s))
        ref = O.linear_fp8_w8a8(bits16(x), oq, os_)
        yf = y.float().cpu().numpy()
        err = O.rel_l2(yf, ref)
        assert err <= 1e-2, f"fp8 n={n} k={k} m={m}: {err}"
        # the kernel computes the same products in fp32: far tighter than the contract
        assert O.rel_l2(yf, O.round_bf16(ref.astype(np.float32))) <= 4e-3


@pytest.mark.parametrize("tiled", [False, True])
def test_fp8_pre_quantized_activation_is_bitwise_the_fused_prologue(tiled):
    """From 2 tokens the FP8 activation is quantized by its own kernel and the GEMM stages the
    codes; the per-token scale and codes are those of the in-kernel prologue, so every output
    (plain, planes, SwiGLU; several plans) is bit-identical."""
    n, k = 2 * 1024, 2560
    w = weights(n, k, 11, edge=False).to(DEV)
    packed = qlinear.quantize_fp8(w)
    if tiled:
        packed = qlinear.prepare(packed)
    for m in (2, 5, 8, 16, 33, 64):
        print(f"fp8 pre-quantized tiled={tiled} m={m}", flush=True)
        x = acts(m, k, 900 + m).to(DEV)
        for cfg in (None, (4, 1, 1, 3), (4, 2, 2, 2)):
            try:
                fused = qlinear.linear_fp8_w8a8(x, packed, config=cfg, pre_quantize=False)
            except ValueError as exc:  # the plan's activation slice does not fit LDS
                assert "LDS" in str(exc)
                continue
            pre = qlinear.linear_fp8_w8a8(x, packed, config=cfg, pre_quantize=True)
            assert torch.equal(pre, fused), (tiled, m, cfg)
            for kw in ({"swiglu": True}, {"planes": True}):
                a = qlinear.linear_fp8_w8a8(x, packed, config=cfg, pre_quantize=False, **kw)
                b = qlinear.linear_fp8_w8a8(x, packed, config=cfg, pre_quantize=True, **kw)
                assert torch.equal(a, b), (tiled, m, cfg, kw)


CONFIGS = [(4, 1, 1, 1), (4, 4, 1, 3), (8, 2, 1, 5), (4, 2, 2, 2), (8, 8, 1, 2), (4, 1, 2, 4)]


@pytest.mark.parametrize("fmt", ["w4a16", "w8a16", "fp8"])
def test_configs_agree_and_planes_reduce_exactly(fmt):
    quant, linear, code = qlinear.FORMATS[fmt]
    n, k = 1024, 2560
    w = weights(n, k, 8).to(DEV)
    packed = quant(w)
    for m in (1, 5, 16, 33):
        x = acts(m, k, 400 + m).to(DEV)
        base = linear(x, packed).float()
        for cfg in CONFIGS:
            try:
                y = linear(x, packed, config=cfg)
            except ValueError as exc:  # the plan's activation slice does not fit LDS
                assert "LDS" in str(exc)
                continue
            assert (y.float() - base).abs().max().item() <= 2e-2 * base.abs().max().item() + 1e-6, (fmt, m, cfg)
            planes = linear(x, packed, config=cfg, planes=True)
            acc = torch.zeros_like(planes[0])
            for p in planes:
                acc += p
            assert torch.equal(acc.to(torch.bfloat16), y), (fmt, m, cfg, "planes summed in order == split path")
            again = linear(x, packed, config=cfg)
            assert torch.equal(again, y), "deterministic"


@pytest.mark.parametrize("fmt", ["w4a16", "w8a16", "fp8"])
def test_swiglu_epilogue(fmt):
    quant, linear, code = qlinear.FORMATS[fmt]
    inter, k = 512, 2560
    w = weights(2 * inter, k, 9, edge=False).to(DEV)
    packed = quant(w)
    for m in (1, 4, 16, 32):
        x = acts(m, k, 500 + m).to(DEV)
        gu = linear(x, packed)
        want = O.swiglu(bits16(gu))
        for cfg in (None, (4, 1, 1, 4), (4, 4, 1, 4), (4, 2, 2, 5)):
            got = linear(x, packed, config=cfg, swiglu=True)
            planes = linear(x, packed, config=cfg, planes=True) if cfg else None
            if planes is not None:
                ref = O.swiglu_partials(planes.cpu().numpy())
                ulp = np.abs(bits16(got).astype(np.int32) - ref.astype(np.int32)).max()
                assert ulp <= 1, (fmt, m, cfg, "fused SwiGLU vs planes + SwiGLU", ulp)
            err = O.rel_l2(got.float().cpu().numpy(), O.bf16_to_f32(want))
            assert err < 2e-2, (fmt, m, cfg, err)


def test_contract_violations_raise_before_launch():
    q, s = qlinear.quantize_w4(weights(64, 256, 0).to(DEV))
    with pytest.raises(ValueError):
        qlinear.linear_w4a16(acts(1, 128, 0).to(DEV), (q, s))
    with pytest.raises(ValueError):
        qlinear.linear_w4a16(acts(65, 256, 0).to(DEV), (q, s))
    with pytest.raises(ValueError):
        qlinear.linear_w4a16(acts(1, 256, 0), (q, s))  # CPU activation
    with pytest.raises(ValueError):
        qlinear.linear_w4a16(acts(1, 256, 0).to(DEV), (q, s), config=(4, 3, 1, 1))


@pytest.mark.parametrize("fmt", ["w4a16", "w8a16", "fp8"])
def test_tiled_weights_match_oracle_and_row_major_bitwise(fmt):
    """prepare() relays bytes exactly as the oracle's tile map; linears give identical bits."""
    quant, linear, code = qlinear.FORMATS[fmt]
    n, k = 4096, 2560
    w = weights(n, k, 10).to(DEV)
    packed = quant(w)
    tiled = qlinear.prepare(packed)
    raw = packed[0].view(torch.uint8).cpu().numpy() if fmt == "fp8" else packed[0].cpu().numpy()
    want = O.tile_rows(raw)
    assert np.array_equal(tiled.weight.cpu().view(torch.uint8).numpy().reshape(want.shape), want)
    same_kernel = {"skinny": False}  # tiled batches > 8 default to the skinny GEMM
    for m in (1, 8, 33):
        x = acts(m, k, 600 + m).to(DEV)
        for cfg in (None, (4, 4, 1, 2), (8, 2, 2, 1)):
            for sw in (False, True):
                try:
                    a = linear(x, packed, config=cfg, swiglu=sw)
                except ValueError as exc:
                    assert "LDS" in str(exc)
                    continue
                b = linear(x, tiled, config=cfg, swiglu=sw, **same_kernel)
                assert torch.equal(a, b), (fmt, m, cfg, sw)


@pytest.mark.parametrize("fmt", ["w4a16", "w8a16"])
@pytest.mark.parametrize("n,k,sw", [(2 * 2048, 2560, True), (2560, 9728, False), (4112, 1024, False)])
def test_skinny_gemm_matches_decode_kernel_and_oracle(fmt, n, k, sw):
    """The skinny GEMM (the default for tile-layout weights from 9 tokens): K slices with fp32
    planes where row groups are few (2560 x 9728), a partial last workgroup (257 tiles), the
    SwiGLU epilogue. Against the decode kernel on the same weights, within one bf16 rounding
    step (the same products, summed in another order), and against the oracle's
    dequantize-then-matmul (rel-L2 <= 1e-2); a zero weight row gives exactly zero."""
    print(f"skinny {fmt} n={n} k={k} swiglu={sw}", flush=True)
    quant, linear, _ = qlinear.FORMATS[fmt]
    w = weights(n, k, 40)
    packed = quant(w.to(DEV))
    tiled = qlinear.prepare(packed)
    q, s = packed
    if fmt == "w4a16":
        deq = O.dequantize(O.unpack_int4_k32(q.cpu().numpy()), bits16(s), bits=4, scale_dtype="bf16")
    else:
        deq = O.dequantize(q.cpu().numpy(), bits16(s)[:, None], bits=8, scale_dtype="bf16", storage="signed")
    for m in (9, 16, 17, 33, 64):
        x = acts(m, k, 700 + m).to(DEV)
        ys = linear(x, tiled, swiglu=sw)
        yd = linear(x, tiled, swiglu=sw, skinny=False)
        # K slices reduced by the row group's last workgroup (tickets) or by a second launch
        code = _lib.FMT_W4A16 if fmt == "w4a16" else _lib.FMT_W8A16
        for fused in (True, False):
            yu = qlinear._skinny(code, tiled.weight, tiled.scale, x, n, k, sw, fused_reduce=fused)
            assert torch.equal(ys, yu), (fmt, n, k, m, fused, "fused split-K reduction differs from the planes launch")
        want = yd.float()
        diff = (ys.float() - want).abs()
        rowmax = want.abs().amax(dim=1, keepdim=True)
        tol = (2.0 ** -6 if sw else 2.0 ** -7) * want.abs() + 2.0 ** -9 * rowmax
        assert (diff > tol).sum().item() == 0, (fmt, n, k, m, diff.max().item())
        ref = O.linear_dequant(bits16(x), deq)
        if sw:
            ref = O.bf16_to_f32(O.swiglu(O.f32_to_bf16(ref.astype(np.float32))))
        assert O.rel_l2(ys.float().cpu().numpy(), ref) <= 1e-2, (fmt, n, k, m)
        if not sw:
            assert not ys[:, 0].float().abs().sum().item(), "zero weight row must give zero"


@pytest.mark.parametrize("n,k,sw", [(2 * 9728, 2560, True), (2560, 9728, False), (4112, 2560, False)])
def test_fp8_skinny_gemm_matches_decode_kernel_and_oracle(n, k, sw):
    """FP8 W8A8 from 9 tokens runs the skinny GEMM on the activation's e4m3 codes (quantized per
    token by its own kernel): within one bf16 rounding step of the decode kernel on the same
    codes, rel-L2 <= 1e-2 against the oracle's W8A8 product, K slices reduced by the last
    workgroup bit-identical to the planes launch, and the same output from codes handed in."""
    print(f"fp8 skinny n={n} k={k} swiglu={sw}", flush=True)
    packed = qlinear.quantize_fp8(weights(n, k, 44).to(DEV))
    tiled = qlinear.prepare(packed)
    q, s = packed
    for m in (9, 16, 17, 33, 64):
        x = acts(m, k, 990 + m).to(DEV)
        ys = qlinear.linear_fp8_w8a8(x, tiled, swiglu=sw)
        yd = qlinear.linear_fp8_w8a8(x, tiled, swiglu=sw, pre_quantize=True).float()
        xq, sx = qlinear.quantize_fp8_activation(x)
        for fused in (True, False):
            yu = qlinear._skinny_fp8(tiled.weight, tiled.scale, xq.view(torch.uint8), sx, n, k, sw, fused_reduce=fused)
            assert torch.equal(ys, yu), (n, k, m, fused, "fused split-K reduction differs from the planes launch")
        assert torch.equal(ys, qlinear.linear_fp8_w8a8_quantized(xq, sx, tiled, swiglu=sw)), (n, k, m)
        diff = (ys.float() - yd).abs()
        rowmax = yd.abs().amax(dim=1, keepdim=True)
        tol = (2.0 ** -6 if sw else 2.0 ** -7) * yd.abs() + 2.0 ** -9 * rowmax
        assert (diff > tol).sum().item() == 0, (n, k, m, diff.max().item())
        ref = O.linear_fp8_w8a8(bits16(x), q.view(torch.uint8).cpu().numpy(), bits16(s))
        if sw:
            ref = O.bf16_to_f32(O.swiglu(O.f32_to_bf16(ref.astype(np.float32))))
        assert O.rel_l2(ys.float().cpu().numpy(), ref) <= 1e-2, (n, k, m)


@pytest.mark.parametrize("m", [33, 64])
@pytest.mark.parametrize("n,k,sw", [(2 * 9728, 2560, True), (2 * 8320, 2560, True), (2560, 9728, False)])
def test_skinny_token_blocks_bit_identical(m, n, k, sw):
    """W4A16 batches of 33-64 tokens run as two blocks of at most 32 tokens where that fills the
    GPU better: whole-K over more than 256 row groups, in one launch where the row groups are a
    multiple of 8 (gate_up 2 x 9728 rows: 304), else in two (2 x 8320 rows: 260); K-sliced
    (down: 40 row groups x 6 slices) in one launch whose blocks write their rows of the planes.
    Each token's sums are unchanged, so the output equals, bit for bit, the one-launch 64-token
    kernel (reached here with an 8-wave plan)."""
    print(f"skinny token blocks m={m} n={n} k={k}", flush=True)
    tiled = qlinear.prepare(qlinear.quantize_w4(weights(n, k, 41).to(DEV)))
    x = acts(m, k, 900 + m).to(DEV)
    ys = qlinear.linear_w4a16(x, tiled, swiglu=sw)  # default plan: token blocks
    lib = _lib.lib()
    mode = _lib.MODE_SWIGLU if sw else _lib.MODE_BF16
    plan = _lib.Plan()
    _lib.check(lib.qlx_plan_skinny(_lib.FMT_W4A16, mode, m, n, k, plan), "plan_skinny")
    assert plan.waves == 4 and plan.rw == 1 and (plan.splits == 1) == sw
    plan.waves = 8  # one launch of the 64-token instance, 8 tiles per workgroup, same K slices
    work = torch.empty((plan.splits, m, n), dtype=torch.float32, device=DEV)
    plan.workspace = work.data_ptr() if plan.splits > 1 else None
    y8 = torch.empty((m, n // 2 if sw else n), dtype=torch.bfloat16, device=DEV)
    _lib.call("qlx_linear_skinny", _lib.FMT_W4A16, _lib.ptr(tiled.weight), _lib.ptr(tiled.scale), _lib.ptr(x),
              _lib.ptr(y8), m, n, k, ctypes.byref(plan), _lib.stream(x.device))
    assert torch.equal(ys, y8), (m, n, k)

