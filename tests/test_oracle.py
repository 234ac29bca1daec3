"""CPU tests that pin the oracle, so that it can be trusted as the checker of the GPU path.

Each oracle function is checked against something it could not simply restate:
the golden vectors written from the reference's own functions (tests/golden/), the
reference's own test invariants (tests/test_engine.py:431-490), library routines (torch's
casts, transformers' Qwen3 modules), closed forms and brute force on tiny inputs. A few
tests plant a mistake in a copy of the oracle and check that the pinning test notices.
"""

import os

import numpy as np
import pytest
import torch

import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_quant.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN)


def bits16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


# ---- number formats -----------------------------------------------------------------

def test_bf16_rounding_matches_torch_on_ties_and_random():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(200000).astype(np.float32) * np.float32(1e3)
    # exact ties: low 16 bits = 0x8000 with odd and even upper halves
    ties = (rng.integers(0, 1 << 15, 4096, dtype=np.uint32) << 17 | 0x8000 | (rng.integers(0, 2, 4096, dtype=np.uint32) << 16))
    ties = (ties & 0x7FFFFFFF).astype(np.uint32).view(np.float32)
    for arr in (x, ties, np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38], np.float32)):
        want = bits16(torch.from_numpy(arr).to(torch.bfloat16))
        got = O.f32_to_bf16(arr)
        nan = np.isnan(arr)  # NaN payloads are implementation-specific: compare NaN-ness only
        assert np.array_equal(got[~nan], want[~nan])
        assert np.isnan(O.bf16_to_f32(got[nan])).all()


def test_e4m3_matches_torch_on_every_code_and_midpoint():
    vals = O.e4m3_to_f32(np.arange(256, dtype=np.uint8))
    fin = np.unique(vals[np.isfinite(vals)].astype(np.float64))
    mids = ((fin[1:] + fin[:-1]) / 2).astype(np.float32)
    rng = np.random.default_rng(1)
    cases = [fin.astype(np.float32), mids, np.nextafter(mids, np.float32(np.inf)),
             np.nextafter(mids, np.float32(-np.inf)),
             np.clip(rng.standard_normal(100000).astype(np.float32) * 100, -448, 448),
             (rng.standard_normal(100000) * 1e-3).astype(np.float32)]
    for arr in cases:
        want = torch.from_numpy(arr).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        assert np.array_equal(O.f32_to_e4m3(arr), want)
    # every finite code decodes to what torch decodes
    codes = np.arange(256, dtype=np.uint8)
    t = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    finite = np.isfinite(t)
    assert np.array_equal(O.e4m3_to_f32(codes)[finite], t[finite])


def test_fp16_scale_rounding_matches_torch():
    x = np.random.default_rng(2).random(100000).astype(np.float32) * np.float32(1e-3)
    assert np.array_equal(O.f32_to_f16(x), bits16(torch.from_numpy(x).to(torch.float16)))


# ---- reference quantize / layouts (golden vectors) -------------------------------------

def test_quantize_dequantize_match_golden(gold):
    for name in "abc":
        w = gold[f"{name}_w"]
        for bits in (8, 4):
            for group in (64, 128):
                key = f"{name}_q{bits}_g{group}"
                if key not in gold:
                    continue
                q, s, _ = O.quantize(w, group, bits)
                assert np.array_equal(q, gold[key]), key
                assert np.array_equal(s, gold[f"{name}_s{bits}_g{group}"]), key
                assert np.array_equal(O.dequantize(q, s, bits), gold[f"{name}_deq{bits}_g{group}"]), key


def test_layouts_match_golden(gold):
    assert np.array_equal(O.permutation(), gold["permutation"])
    for name in "abc":
        w = gold[f"{name}_w"]
        q, _, _ = O.quantize(w)
        assert np.array_equal(O.prepare_weight(q, 8, True), gold[f"{name}_prep8_tiled"])
        assert np.array_equal(O.prepare_weight(q, 8, False), gold[f"{name}_prep8_rowmajor"])
        assert np.array_equal(O.row_major(gold[f"{name}_prep8_tiled"]), gold[f"{name}_prep8_rowmajor"])
        q4, _, _ = O.quantize(w, bits=4)
        assert np.array_equal(O.prepare_weight(q4, 4, True), gold[f"{name}_prep4_tiled"])
        got = O.int8_prepare(gold[f"{name}_prep8_rowmajor"]).view(np.uint8)
        assert np.array_equal(got, gold[f"{name}_int8_prepared"])


def test_fp8_quantize_matches_golden(gold):
    for name in "abc":
        w = gold[f"{name}_w"]
        k = w.shape[1]
        for group in (128, k):
            code, s = O.fp8_quantize(w, group)
            assert np.array_equal(code, gold[f"{name}_fp8_g{group}"])
            assert np.array_equal(s, gold[f"{name}_fp8s_g{group}"])


def test_reference_invariants_int4():
    """tests/test_engine.py:454-471: codes in [1, 15], error bounds, rel-L2 in (0.02, 0.2)."""
    g = torch.Generator().manual_seed(1)
    w = bits16(torch.randn(32, 256, generator=g).to(torch.bfloat16))
    q, s, _ = O.quantize(w, bits=4)
    assert q.min() >= 1 and q.max() <= 15
    exact = O.bf16_to_f32(O.dequantize(q, s, 4))
    wf = O.bf16_to_f32(w)
    rel = np.linalg.norm(exact - wf) / np.linalg.norm(wf)
    assert 0.02 < rel < 0.2
    step = np.repeat(O.f16_to_f32(s), 64, axis=1)
    assert (np.abs(exact - wf) <= step * 0.5 + np.abs(exact) * 2 ** -8 + 1e-6).all()


def test_permutation_closed_form_and_planted_mistake(gold):
    """The permutation is a bijection of 0..63 with a closed form; a transposed (s, t) fails."""
    p = O.permutation()
    assert sorted(p.tolist()) == list(range(64))
    for pos in range(64):
        t, s, i = pos // 16, (pos // 4) % 4, pos % 4
        assert p[pos] == 16 * s + 2 * t + (0, 1, 8, 9)[i]
    wrong = np.array([16 * t + 2 * s + u for t in range(4) for s in range(4) for u in (0, 1, 8, 9)])
    assert not np.array_equal(wrong, gold["permutation"])


# ---- north-star formats ---------------------------------------------------------------

def test_int4_k32_pack_brute_force_and_round_trip():
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 16, (5, 64), dtype=np.uint8)
    words = O.pack_int4_k32(codes).view(np.uint32)
    for r in range(5):
        for k in range(64):
            assert (words[r, k // 8] >> (4 * (k % 8))) & 0xF == codes[r, k]
    assert np.array_equal(O.unpack_int4_k32(words), codes)


def test_int4_g128_is_reference_formula_with_bf16_scales():
    """quantize_int4_g128 = the reference quantizer at group 128 with the scale rounded to bf16."""
    g = torch.Generator().manual_seed(4)
    w32 = torch.randn(16, 512, generator=g) * 0.02
    w = bits16(w32.to(torch.bfloat16))
    words, s = O.quantize_int4_g128(w)
    codes = O.unpack_int4_k32(words)
    # brute force the closed form element by element
    wf = O.bf16_to_f32(w).reshape(16, 4, 128)
    amax = np.abs(wf).max(axis=2)
    for r in range(16):
        for grp in range(4):
            sc = np.float32(max(np.float32(amax[r, grp]) / np.float32(7.0), np.float32(1e-12)))
            sc = np.float32(sc * np.float32(1 + 2 ** -10))
            sb = O.f32_to_bf16(sc)
            assert s[r, grp] == sb
            sv = O.bf16_to_f32(sb)
            want = np.clip(np.rint(wf[r, grp] / sv), -7, 7) + 8
            assert np.array_equal(codes[r, grp * 128:(grp + 1) * 128], want.astype(np.uint8))


def test_w8_per_channel_and_fp8_activation_closed_forms():
    g = torch.Generator().manual_seed(5)
    w = bits16((torch.randn(8, 256, generator=g) * 0.02).to(torch.bfloat16))
    q, s = O.quantize_w8_per_channel(w)
    wf = O.bf16_to_f32(w)
    for r in range(8):
        sc = np.float32(np.float32(np.abs(wf[r]).max()) / np.float32(127.0)) * np.float32(1 + 2 ** -10)
        assert s[r] == O.f32_to_bf16(np.float32(sc))
        assert np.array_equal(q[r], np.clip(np.rint(wf[r] / O.bf16_to_f32(s[r])), -127, 127).astype(np.int8))
    x = bits16(torch.randn(3, 256, generator=g).to(torch.bfloat16))
    code, sx = O.quantize_fp8_activation(x)
    xf = O.bf16_to_f32(x)
    # per-token = fp8.quantize with group = K on each row, but keeping the fp32 scale
    for r in range(3):
        c2, s2 = O.fp8_quantize(x[r:r + 1], group=256)
        assert np.array_equal(code[r], c2[0])
        assert O.f32_to_bf16(sx[r:r + 1])[0] == s2[0, 0]
        assert sx[r] == np.float32(np.float32(np.abs(xf[r]).max()) / np.float32(448.0))
    # torch's own cast gives the same codes
    t = (torch.from_numpy(xf) / torch.from_numpy(sx)[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    assert np.array_equal(code, t.view(torch.uint8).numpy())


def test_tile_rows_brute_force_and_planted_mistake():
    rng = np.random.default_rng(6)
    data = rng.integers(0, 256, (32, 256), dtype=np.uint8)
    t = O.tile_rows(data).reshape(-1)
    for row in range(32):
        for byte in range(256):
            tile, r, step, j, c, b = row // 16, row % 16, byte // 128, (byte // 64) % 2, (byte // 16) % 4, byte % 16
            off = (tile * 2 + step) * 2048 + ((j * 4 + c) * 16 + r) * 16 + b
            assert t[off] == data[row, byte]
    swapped = np.ascontiguousarray(data.reshape(2, 16, 2, 2, 4, 16).transpose(0, 2, 3, 1, 4, 5)).reshape(-1)
    assert not np.array_equal(swapped, t), "a c/r transposition would be caught"


# ---- linear and epilogue oracles ------------------------------------------------------

def test_linear_oracles_agree_with_torch_fp64():
    g = torch.Generator().manual_seed(7)
    w = bits16((torch.randn(48, 256, generator=g) * 0.02).to(torch.bfloat16))
    x = bits16(torch.randn(3, 256, generator=g).to(torch.bfloat16))
    q, s, _ = O.quantize(w)
    deq = O.dequantize(q, s)
    want = (torch.from_numpy(O.bf16_to_f32(x)).double() @ torch.from_numpy(O.bf16_to_f32(deq)).double().T).numpy()
    assert np.allclose(O.linear_dequant(x, deq), want)
    exact = O.linear_exact_grouped(x, q.astype(np.float64) - 128, O.f16_to_f32(s), 64)
    assert O.rel_l2(exact, want) < 1e-2
    wq, ws = O.fp8_quantize(w, 256)
    fp = O.linear_fp8_w8a8(x, wq, ws)
    # the same product restated with torch's e4m3 casts (oracle/cpu_baseline.py's CPU path)
    from oracle import cpu_baseline
    xt = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
    wt = torch.from_numpy(wq).view(torch.float8_e4m3fn)
    st = torch.from_numpy(ws[:, 0].view(np.int16)).view(torch.bfloat16)
    tq = cpu_baseline.linear_fp8_w8a8(xt, wt, st).float().numpy()
    assert O.rel_l2(tq, fp) < 4e-3
    wx = O.bf16_to_f32(x).astype(np.float64) @ O.bf16_to_f32(w).astype(np.float64).T
    assert O.rel_l2(fp, wx) < 0.1  # e4m3 on both operands: a few percent from the bf16 product


def test_swiglu_and_rms_norm_match_transformers():
    from transformers.models.qwen3.configuration_qwen3 import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3MLP, Qwen3RMSNorm
    torch.manual_seed(3)
    cfg = Qwen3Config(hidden_size=256, intermediate_size=512, num_hidden_layers=1, num_attention_heads=4,
                      num_key_value_heads=2, head_dim=64, rms_norm_eps=1e-6)
    mlp = Qwen3MLP(cfg).to(torch.bfloat16)
    x = torch.randn(32, 256, dtype=torch.bfloat16)
    with torch.no_grad():
        gate, up = mlp.gate_proj(x), mlp.up_proj(x)
        want = mlp.act_fn(gate) * up
    got = O.swiglu(bits16(torch.cat([gate, up], dim=1)))
    ulps = np.abs(got.astype(np.int32) - bits16(want).astype(np.int32)).max()
    assert ulps <= 1
    torch.manual_seed(0)
    ref = Qwen3RMSNorm(2560, eps=1e-6).to(torch.bfloat16)
    ref.weight.data = torch.randn(2560, dtype=torch.bfloat16)
    xs = torch.randn(16, 2560, dtype=torch.bfloat16)
    with torch.no_grad():
        want = ref(xs)
    got = O.rms_norm(bits16(xs), bits16(ref.weight.data), 1e-6)
    ulps = np.abs(got.astype(np.int32) - bits16(want).astype(np.int32)).max()
    assert ulps <= 1


def test_plane_reduction_order_and_residual_rounding():
    planes = np.array([[[1e8, 1.0]], [[-1e8, 1.0]], [[1.0, 1e8]]], dtype=np.float32)
    # sequential plane order: (1e8 + -1e8) + 1 = 1, not 1e8 + (-1e8 + 1) = 0
    assert O.bf16_to_f32(O.reduce_partials(planes))[0, 0] == 1.0
    x = O.f32_to_bf16(np.array([[1.0, 1.0]], np.float32))
    r = O.residual_partials(x, planes)
    assert O.bf16_to_f32(r)[0, 0] == 2.0


def test_int8_activation_quantize_closed_form():
    g = torch.Generator().manual_seed(8)
    x = bits16(torch.randn(2, 128, generator=g).to(torch.bfloat16))
    q, s = O.int8_quantize_activation(x)
    xf = O.bf16_to_f32(x).reshape(2, 2, 64)
    nat = O.int8_natural()
    assert sorted(nat.tolist()) == list(range(64))
    for r in range(2):
        for grp in range(2):
            sc = np.float32(max(np.float32(np.abs(xf[r, grp]).max()) / np.float32(127), np.float32(1e-20)))
            assert s[r, grp] == sc
            for p in range(64):
                assert q[r, grp * 64 + p] == np.int8(np.rint(xf[r, grp, nat[p]] / sc))


def test_int8_second_component_closed_forms_and_bounds():
    """The INT8 activation's second component (cuda_int8.py:70-77): whole-number groups are
    taken exactly by the first component (residual 0: qr = 0, sr = 1e-20); otherwise the two
    components reconstruct every value to within half a step of the second scale, the second
    scale is the residual's max / 127, and each group's largest residual maps to +-127. A
    planted mistake (the residual taken with a fused multiply-add, i.e. the product unrounded)
    changes the codes of random data."""
    g = torch.Generator().manual_seed(31)
    # closed form: integers with a group maximum of 127 -> s = 1 exactly, nothing left over
    ints = torch.randint(-127, 128, (2, 128), generator=g).float()
    ints[:, 0] = 127.0
    ints[:, 64] = -127.0
    q, s, qr, sr = O.int8_quantize_activation(bits16(ints.to(torch.bfloat16)), components=2)
    assert np.all(s == np.float32(1.0)) and not qr.any() and np.all(sr == np.float32(1e-20))
    nat = O.int8_natural()
    assert np.array_equal(q.reshape(2, 2, 64), ints.numpy().astype(np.int8).reshape(2, 2, 64)[:, :, nat])
    # bounds on random data
    x = bits16(torch.randn(4, 256, generator=g).to(torch.bfloat16))
    q, s, qr, sr = O.int8_quantize_activation(x, components=2)
    q1, s1 = O.int8_quantize_activation(x)
    assert np.array_equal(q, q1) and np.array_equal(s, s1), "the first component is the plain quantize"
    xf = O.bf16_to_f32(x).reshape(4, 4, 64)[:, :, nat].astype(np.float64)
    qd = q.reshape(4, 4, 64).astype(np.float64)
    rd = qr.reshape(4, 4, 64).astype(np.float64)
    res = xf - qd * s[:, :, None].astype(np.float64)
    assert np.all(np.abs(res - rd * sr[:, :, None]) <= 0.5 * sr[:, :, None] * (1 + 1e-6) + 1e-7 * np.abs(xf))
    assert np.all(np.abs(rd).max(axis=2) == 127)
    assert np.allclose(sr, np.abs(res).max(axis=2) / 127, rtol=1e-5)
    # planted mistake: the residual with the product kept exact
    xf32 = O.bf16_to_f32(x).reshape(4, 4, 64)
    qf = np.rint(xf32 / s[:, :, None]).astype(np.float64)
    fused = (xf32.astype(np.float64) - qf * s[:, :, None].astype(np.float64)).astype(np.float32)
    sr_f = np.maximum(np.abs(fused).max(axis=2) / np.float32(127), np.float32(1e-20)).astype(np.float32)
    qr_f = np.rint(fused / sr_f[:, :, None]).astype(np.int8)[:, :, nat].reshape(4, 256)
    assert not (np.array_equal(qr_f, qr) and np.array_equal(sr_f, sr)), "an unrounded product must show"


def test_int8_w8a8_product_pinned_by_golden_weights_and_fp64(gold):
    """oracle.linear_w8a8_int8 (the INT8 W8A8 GEMM's checker) against an fp64 torch product in
    natural column order: activation s_x * rint(x / s_x) per 64-group (torch ops), weight
    (byte - 128) * fp16 scale from the golden quantize vectors, while the oracle is fed the
    golden fragment-ordered cuda_int8.Prepared bytes. Plus a closed form and a planted
    fragment-order mistake."""
    g = torch.Generator().manual_seed(23)
    for name, rows in (("a", 32), ("b", 64)):
        k = 256
        x = torch.randn(3, k, generator=g).to(torch.bfloat16)
        q8 = gold[f"{name}_q8_g64"] if f"{name}_q8_g64" in gold else None
        if q8 is None:  # b has prepared bytes only: requantize its weight with the pinned oracle
            q8, s8, _ = O.quantize(gold[f"{name}_w"])
        else:
            s8 = gold[f"{name}_s8_g64"]
        prepared = gold[f"{name}_int8_prepared"].view(np.int8)
        assert np.array_equal(prepared, O.int8_prepare(O.prepare_weight(q8, tiled=False)))
        xf = x.float().double().reshape(3, k // 64, 64)
        sx = torch.clamp(xf.abs().amax(dim=2, keepdim=True).float() / 127.0, min=1e-20).double()
        xhat = (torch.round(xf / sx) * sx).reshape(3, k)  # torch.round is half-even, as rint
        what = (torch.from_numpy(q8.astype(np.float64)) - 128.0) * torch.from_numpy(
            O.f16_to_f32(s8).astype(np.float64)).repeat_interleave(64, dim=1)
        want = (xhat @ what.T).numpy()
        got = O.linear_w8a8_int8(bits16(x), prepared, s8)
        assert np.allclose(got, want, rtol=1e-12, atol=1e-12), name
        # planted mistake: the activation codes left in natural order (no fragment permutation)
        wrong = prepared.reshape(rows, k // 64, 64)[:, :, np.argsort(O.int8_natural())].reshape(rows, k)
        assert not np.allclose(O.linear_w8a8_int8(bits16(x), wrong, s8), want, rtol=1e-6), name
    # closed form: every activation 127/128 -> s_x = 2^-7 exactly, codes 127, so the product is
    # 127/128 times the row sums of the dequantized weight
    q8, s8 = gold["a_q8_g64"], gold["a_s8_g64"]
    prepared = gold["a_int8_prepared"].view(np.int8)
    x = np.full((1, 256), O.f32_to_bf16(np.array([127.0 / 128.0], np.float32))[0], np.uint16)
    rowsum = ((q8.astype(np.float64) - 128.0) * np.repeat(O.f16_to_f32(s8).astype(np.float64), 64, axis=1)).sum(1)
    assert np.allclose(O.linear_w8a8_int8(x, prepared, s8)[0], 127.0 / 128.0 * rowsum, rtol=1e-12, atol=1e-15)
