"""numpy restatement of the reference's quantized-linear arithmetic (test oracle).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py; never by the product path.

Conventions: bf16 and fp16 values travel as ``uint16`` bit patterns, e4m3 as
``uint8`` bytes, so every comparison with the device is on bits. Citations are
``path:line`` inside the reference repository.
"""

import numpy as np

__all__ = [
    "f32_to_bf16", "bf16_to_f32", "round_bf16", "f32_to_f16", "f16_to_f32",
    "f32_to_e4m3", "e4m3_to_f32",
    "permutation", "quantize", "dequantize", "prepare_weight", "row_major",
    "fp8_quantize", "int8_natural", "int8_prepare", "int8_quantize_activation",
    "pack_int4_k32", "unpack_int4_k32", "tile_rows", "quantize_int4_g128", "quantize_w8_per_channel",
    "quantize_fp8_activation",
    "linear_dequant", "linear_exact_grouped", "linear_fp8_w8a8", "linear_w8a8_int8",
    "reduce_partials", "residual_partials", "rms_norm", "add_rms_norm",
    "add_rms_norm_partials", "silu_bf16", "swiglu", "swiglu_partials", "add_norm_quant",
    "rel_l2",
]

F32 = np.float32


# --------------------------------------------------------------------------------------
# Number formats. Round-to-nearest-even everywhere, as torch's casts do.
# --------------------------------------------------------------------------------------

def f32_to_bf16(x):
    """fp32 -> bf16 bits, RNE; NaN -> canonical quiet NaN (torch's ``.to(bfloat16)``).

    Same integer-add rounding the reference kernels use (cuda_fp8.py:64-68).
    Pinned: tests compare with torch's cast over random and tie values.
    """
    u = np.ascontiguousarray(x, dtype=F32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32)
    nan = np.isnan(np.asarray(x, dtype=F32))
    r = np.where(nan, ((u >> 16) & 0x8000) | 0x7FC0, r)
    return r.astype(np.uint16)


def bf16_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(F32)


def round_bf16(x):
    """fp32 value rounded to bf16 and back (the reference's ``.to(bf16).float()``)."""
    return bf16_to_f32(f32_to_bf16(x))


def f32_to_f16(x):
    """fp32 -> fp16 bits, RNE with subnormals (numpy's cast is IEEE)."""
    return np.asarray(x, dtype=F32).astype(np.float16).view(np.uint16)


def f16_to_f32(h):
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(F32)


def f32_to_e4m3(x):
    """fp32 -> OCP e4m3fn byte, RNE, as torch's ``.to(torch.float8_e4m3fn)``.

    Normal range: drop 20 mantissa bits with round-half-even by integer add;
    below 2**-6 the subnormal code is ``rint(|x| * 2**9)`` (0..8, where 8 is
    the smallest normal). Results past 448 become NaN (0x7F), as torch does;
    callers clamp to +-448 first (fp8.py:27). Pinned: tests compare with
    torch's cast over every e4m3 value, every rounding midpoint and random
    values.
    """
    f = np.ascontiguousarray(x, dtype=F32)
    u = f.view(np.uint32).astype(np.int64)
    sign = ((u >> 24) & 0x80).astype(np.uint8)
    a = u & 0x7FFFFFFF
    af = (a.astype(np.uint32)).view(F32)
    sub = a < (121 << 23)
    code_sub = np.rint(af.astype(F32) * F32(512.0)).astype(np.int64)
    ar = a + 0x7FFFF + ((a >> 20) & 1)
    code_norm = (ar >> 20) - (120 << 3)
    code = np.where(sub, code_sub, code_norm)
    code = np.where(code > 0x7E, 0x7F, code)
    code = np.where(a > 0x7F800000, 0x7F, code)
    return (code.astype(np.uint8) | sign)


def e4m3_to_f32(b):
    b = np.asarray(b, dtype=np.uint8).astype(np.int64)
    s = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 15
    m = b & 7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    val = np.where((e == 15) & (m == 7), np.nan, val)
    return (s * val).astype(F32)


# --------------------------------------------------------------------------------------
# Reference weight formats (engine/kernels/cuda_fp8.py).
# --------------------------------------------------------------------------------------

def permutation():
    """Natural column held at each permuted position of a 64-wide block.

    cuda_fp8.py:1117-1124: position 16t+4s+i holds natural 16s+2t+u, u in
    (0,1,8,9)[i]. Pinned by the golden vector ``permutation``.
    """
    order = [16 * s + 2 * t + u for t in range(4) for s in range(4) for u in (0, 1, 8, 9)]
    return np.array(order, dtype=np.int64)


def quantize(w_bits, group=64, bits=8, scale_dtype="f16", nudge=True, storage="offset"):
    """Symmetric absmax quantize of a bf16 ``[out, in]`` weight.

    cuda_fp8.py:1127-1151, step for step: s = max(amax/limit, 1e-12) in fp32;
    s = fp16(s * (1 + 2**-10)); q = clamp(rint(w / float(s)), +-limit);
    byte = q + offset as uint8 (limit/offset 127/128 for 8 bits, 7/8 for 4).
    NaN codes (0/0 when an all-zero group's fp16 scale underflows to 0) become
    byte 0, as the x86 and CUDA float->uint8 conversions give.

    Generalisations used by the north-star formats (defaults reproduce the
    reference): ``scale_dtype="bf16"`` rounds the scale to bf16 instead of
    fp16; ``storage="signed"`` stores q itself as int8 (no offset);
    ``storage="codes"`` stores q + offset as uint8 for packing.
    Pinned by the golden vectors ``*_q{8,4}_g{64,128}`` / ``*_s*``.
    """
    w = bf16_to_f32(w_bits)
    out, inner = w.shape
    if inner % group:
        raise ValueError(f"{inner} is not a multiple of {group}")
    limit, offset = (F32(127.0), F32(128.0)) if bits == 8 else (F32(7.0), F32(8.0))
    tiles = w.reshape(out, inner // group, group)
    with np.errstate(divide="ignore", invalid="ignore"):
        scale = np.maximum(np.abs(tiles).max(axis=2, keepdims=True) / limit, F32(1e-12)).astype(F32)
        if nudge:
            scale = (scale * F32(1.0 + 2.0 ** -10)).astype(F32)
        if scale_dtype == "f16":
            s_bits = f32_to_f16(scale)
            s_val = f16_to_f32(s_bits)
        elif scale_dtype == "bf16":
            s_bits = f32_to_bf16(scale)
            s_val = bf16_to_f32(s_bits)
        else:
            raise ValueError(scale_dtype)
        q = np.clip(np.rint(tiles / s_val), -limit, limit)
    if storage == "signed":
        data = np.where(np.isnan(q), 0, q).astype(np.int8).reshape(out, inner)
    else:
        biased = q + offset
        data = np.where(np.isnan(biased), 0, biased).astype(np.uint8).reshape(out, inner)
    return data, s_bits.reshape(out, inner // group), bits


def dequantize(data, s_bits, bits=8, scale_dtype="f16", storage="offset"):
    """bf16((byte - offset) * float(scale)), cuda_fp8.py:1154-1161 (``signed``: q * scale)."""
    rows, k = data.shape
    blocks = s_bits.shape[1]
    if storage == "signed":
        q = data.astype(F32)
    else:
        q = data.astype(F32) - (F32(128.0) if bits == 8 else F32(8.0))
    s = f16_to_f32(s_bits) if scale_dtype == "f16" else bf16_to_f32(s_bits)
    prod = (q.reshape(rows, blocks, k // blocks) * s[:, :, None]).astype(F32)
    return f32_to_bf16(prod.reshape(rows, k))


def prepare_weight(data, bits=8, tiled=True):
    """Byte layout of ``cuda_fp8.Prepared.weight`` (cuda_fp8.py:1164-1205).

    Columns of every 64-block are permuted by ``permutation()``; ``tiled`` then
    regroups a 16-row x 128-column group as [half][j][g][t][16 B] (8 bits) or
    folds j into nibbles, [half][g][t][16 B] with block 0 low and block 1 high
    (4 bits). Pinned by the golden vectors ``*_prep8_*`` and ``*_prep4_tiled``.
    """
    rows, k = data.shape
    if k % 128 or rows % 16:
        raise ValueError("rows must be a multiple of 16 and K of 128")
    perm = permutation()
    cols = (np.arange(k // 64)[:, None] * 64 + perm[None, :]).reshape(-1)
    w = data.view(np.uint8)[:, cols]
    if bits == 4:
        if not tiled:
            raise ValueError("4-bit weights are stored tiled")
        v = w.reshape(rows // 16, 2, 8, k // 128, 2, 4, 16)
        packed = v[:, :, :, :, 0] | (v[:, :, :, :, 1] << 4)
        return np.ascontiguousarray(packed.transpose(0, 3, 1, 2, 4, 5)).reshape(rows, k // 2)
    if tiled:
        w = w.reshape(rows // 16, 2, 8, k // 128, 2, 4, 16).transpose(0, 3, 1, 4, 2, 5, 6)
    return np.ascontiguousarray(w).reshape(rows, k)


def row_major(weight, tiled=True):
    """``Prepared.row_major`` (cuda_fp8.py:1207-1214): the fragment-permuted [rows, K] bytes."""
    rows, k = weight.shape
    if not tiled:
        return weight
    t = weight.reshape(rows // 16, k // 128, 2, 2, 8, 4, 16).transpose(0, 2, 4, 1, 3, 5, 6)
    return np.ascontiguousarray(t).reshape(rows, k)


def fp8_quantize(w_bits, group=128):
    """E4M3 weight quantize, fp8.py:20-28.

    s = max(amax/448, 1e-12) in fp32; code = e4m3(clamp(w/s, +-448)); the
    returned scale is bf16(s), so the division used the unrounded scale.
    Per-output-channel is ``group = K``. Pinned by golden ``*_fp8_g*``.
    """
    w = bf16_to_f32(w_bits)
    out, inner = w.shape
    if inner % group:
        raise ValueError(f"{inner} is not a multiple of {group}")
    tiles = w.reshape(out, inner // group, group)
    scale = np.maximum(np.abs(tiles).max(axis=2, keepdims=True) / F32(448.0), F32(1e-12)).astype(F32)
    code = f32_to_e4m3(np.clip(tiles / scale, F32(-448.0), F32(448.0)))
    return code.reshape(out, inner), f32_to_bf16(scale.reshape(out, inner // group))


# --------------------------------------------------------------------------------------
# INT8 W8A8 (engine/kernels/cuda_int8.py).
# --------------------------------------------------------------------------------------

def int8_natural():
    """Natural index held at INT8 fragment position p (cuda_int8.py:64, 102)."""
    p = np.arange(64)
    return (p // 16) * 4 + ((p % 16) // 4) * 16 + p % 4


def int8_prepare(row_major_bytes):
    """``cuda_int8.Prepared.weight`` (cuda_int8.py:100-108).

    Position p of every 64-block holds natural column ``int8_natural()[p]``,
    taken from the fragment-permuted row-major bytes, with the offset removed
    by ``^ 128`` (two's complement int8). Pinned by golden ``*_int8_prepared``.
    """
    rows, k = row_major_bytes.shape
    nat = int8_natural()
    old = ((nat % 8) // 2) * 16 + (nat // 16) * 4 + ((nat % 16) // 8) * 2 + nat % 2
    cols = (np.arange(k // 64)[:, None] * 64 + old[None, :]).reshape(-1)
    return (row_major_bytes[:, cols] ^ 128).astype(np.uint8).view(np.int8)


def int8_quantize_activation(x_bits, components=1):
    """Per-row, per-64-group INT8 activation quantize (cuda_int8.py:58-77).

    s = max(amax/127, 1e-20) in fp32; q = rint(x/s) (``nearbyint``, half-even)
    stored at fragment position p from natural ``int8_natural()[p]``. Returns
    (q int8 [M,K], s fp32 [M,K/64]). With ``components=2`` (cuda_int8.py:70-77) also the
    second component of what q leaves: residual = x - fp32(q * s) (the kernel is compiled
    without fp fusion, so the product is rounded before the subtraction), then
    sr = max(amax(residual)/127, 1e-20) and qr = rint(residual/sr) in the same positions:
    returns (q, s, qr, sr). Pinned by closed form and brute-force tests (the reference's
    version is a Triton kernel that cannot run here).
    """
    x = bf16_to_f32(x_bits)
    m, k = x.shape
    nat = int8_natural()
    g = x.reshape(m, k // 64, 64)
    s = np.maximum(np.abs(g).max(axis=2) / F32(127.0), F32(1e-20)).astype(F32)
    qf = np.rint(g / s[:, :, None]).astype(F32)
    q = qf.astype(np.int8)[:, :, nat]
    if components == 1:
        return q.reshape(m, k), s
    res = (g - (qf * s[:, :, None]).astype(F32)).astype(F32)
    sr = np.maximum(np.abs(res).max(axis=2) / F32(127.0), F32(1e-20)).astype(F32)
    qr = np.rint(res / sr[:, :, None]).astype(np.int8)[:, :, nat]
    return q.reshape(m, k), s, qr.reshape(m, k), sr


def linear_w8a8_int8(x_bits, prepared_i8, w_scale_f16):
    """INT8 W8A8 product as next_probe.py:79-91 states it: (q_x s_x) . (q_w s_w), fp64 here."""
    q, s = int8_quantize_activation(x_bits)
    m, k = q.shape
    n = prepared_i8.shape[0]
    qx = q.reshape(m, k // 64, 64).astype(np.float64)
    qw = prepared_i8.reshape(n, k // 64, 64).astype(np.float64)
    sw = f16_to_f32(w_scale_f16).astype(np.float64)
    dots = np.einsum("mgk,ngk->mng", qx, qw)
    return np.einsum("mng,mg,ng->mn", dots, s.astype(np.float64), sw)


# --------------------------------------------------------------------------------------
# North-star formats (the reference formula with documented substitutions).
# --------------------------------------------------------------------------------------

def pack_int4_k32(codes):
    """uint8 nibble codes [N, K] (0..15) -> int32 [N, K/8]: nibble i of word j is k = 8j+i."""
    n, k = codes.shape
    if k % 8:
        raise ValueError("K must be a multiple of 8")
    c = codes.astype(np.uint32).reshape(n, k // 8, 8)
    word = np.zeros((n, k // 8), dtype=np.uint32)
    for i in range(8):
        word |= (c[:, :, i] & 0xF) << (4 * i)
    return word.view(np.int32)


def unpack_int4_k32(words):
    w = np.asarray(words).view(np.uint32)
    n, kw = w.shape
    out = np.zeros((n, kw, 8), dtype=np.uint8)
    for i in range(8):
        out[:, :, i] = (w >> (4 * i)) & 0xF
    return out.reshape(n, kw * 8)


def tile_rows(data):
    """MI355X tile layout of a row-major weight (any dtype, viewed as bytes).

    Block (tile t, step s) -- rows 16t..16t+15, bytes 128s..128s+127 -- is stored as
    [j 2][c 4][r 16][16 bytes] holding row 16t + r, bytes 128s + 64j + 16c. Pinned by a
    brute-force per-byte check and by round trip in the tests.
    """
    b = np.ascontiguousarray(data).view(np.uint8)
    rows, width = b.shape
    v = b.reshape(rows // 16, 16, width // 128, 2, 4, 16)        # t, r, s, j, c, byte
    return np.ascontiguousarray(v.transpose(0, 2, 3, 4, 1, 5)).reshape(rows, width)


def quantize_int4_g128(w_bits, group=128):
    """W4A16: the reference quantizer (cuda_fp8.py:1140-1151) at group 128 with bf16
    scales, codes q+8 packed eight per int32 along K. Returns (int32 [N,K/8], bf16 [N,K/128])."""
    codes, s_bits, _ = quantize(w_bits, group=group, bits=4, scale_dtype="bf16", storage="codes")
    return pack_int4_k32(codes), s_bits


def quantize_w8_per_channel(w_bits):
    """W8A16 per output channel: the reference quantizer with group = K, bf16 scales,
    signed int8 storage. Returns (int8 [N,K], bf16 [N])."""
    k = w_bits.shape[1]
    data, s_bits, _ = quantize(w_bits, group=k, bits=8, scale_dtype="bf16", storage="signed")
    return data, s_bits[:, 0].copy()


def quantize_fp8_activation(x_bits):
    """Dynamic per-token e4m3 activation quantize.

    ``fp8_quantize`` applied to each row with group = K (fp8.py:25-27), but the
    scale stays fp32 as ``cuda_int8.quantize_activation`` keeps its (cuda_int8.py:67):
    s = max(amax/448, 1e-12); code = e4m3(clamp(x/s, +-448)). Returns
    (e4m3 uint8 [M,K], fp32 [M]). No reference function computes exactly this;
    it is pinned by the fp8_quantize golden vectors it reduces to (group = K)
    and by brute force.
    """
    x = bf16_to_f32(x_bits)
    s = np.maximum(np.abs(x).max(axis=1, keepdims=True) / F32(448.0), F32(1e-12)).astype(F32)
    code = f32_to_e4m3(np.clip(x / s, F32(-448.0), F32(448.0)))
    return code, s[:, 0].copy()


# --------------------------------------------------------------------------------------
# Linear-layer oracles.
# --------------------------------------------------------------------------------------

def linear_dequant(x_bits, w_deq_bits):
    """``F.linear(x, dequantize(W))`` (gpu_checks.py:141-144) in fp64; round with round_bf16."""
    x = bf16_to_f32(x_bits).astype(np.float64)
    w = bf16_to_f32(w_deq_bits).astype(np.float64)
    return x @ w.T


def linear_exact_grouped(x_bits, q_values, scale_values, group):
    """What the kernels compute (cuda_fp8.py:383-388): per group the exact fp32 partial of
    q * x, times the group scale, summed over groups -- here in fp64."""
    x = bf16_to_f32(x_bits).astype(np.float64)
    m, k = x.shape
    n = q_values.shape[0]
    q = q_values.astype(np.float64).reshape(n, k // group, group)
    xs = x.reshape(m, k // group, group)
    dots = np.einsum("mgk,ngk->mng", xs, q)
    return np.einsum("mng,ng->mn", dots, np.asarray(scale_values, np.float64).reshape(n, k // group))


def linear_fp8_w8a8(x_bits, w_code, w_scale_bits):
    """FP8 W8A8 as BASELINE states its CPU path: (x_q s_x) @ (w_q s_w)^T, in fp64 here."""
    xq, sx = quantize_fp8_activation(x_bits)
    xa = e4m3_to_f32(xq).astype(np.float64) * sx.astype(np.float64)[:, None]
    sw = bf16_to_f32(np.asarray(w_scale_bits).reshape(-1)).astype(np.float64)
    wa = e4m3_to_f32(w_code).astype(np.float64) * sw[:, None]
    return xa @ wa.T


# --------------------------------------------------------------------------------------
# Epilogues and plane consumers.
# --------------------------------------------------------------------------------------

def reduce_partials(planes):
    """bf16(sum_s P[s]) in plane order, fp32 (cuda_fp8.py:965-981)."""
    acc = np.zeros(planes.shape[1:], dtype=F32)
    for p in planes:
        acc = (acc + p.astype(F32)).astype(F32)
    return f32_to_bf16(acc)


def residual_partials(x_bits, planes):
    """bf16(x + bf16(sum_s P[s])) (cuda_small.py:43-55)."""
    delta = bf16_to_f32(reduce_partials(planes))
    return f32_to_bf16((bf16_to_f32(x_bits) + delta).astype(F32))


def rms_norm(x_bits, w_bits, eps):
    """bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w) (reference.py:13-16).

    The squares of bf16 values and their sum over a row are exact in fp64, so the mean is
    taken exactly, rounded to fp32, then eps is added and 1/sqrt taken in fp32 as torch's
    rsqrt(mean + eps) does. An fp32 sum in another order agrees to within one bf16 ulp (the
    reference's own bar, gpu_checks.py:451-492); the device kernel sums in fp64 too."""
    x = bf16_to_f32(x_bits)
    ms = (x.astype(np.float64) ** 2).sum(axis=-1, keepdims=True) / x.shape[-1]
    scale = (F32(1.0) / np.sqrt((ms.astype(F32) + F32(eps)).astype(F32))).astype(F32)
    y = round_bf16((x * scale).astype(F32))
    return f32_to_bf16((y * bf16_to_f32(w_bits)).astype(F32))


def add_rms_norm(x_bits, delta_bits, w_bits, eps):
    """(bf16(x + delta), rms_norm of it) (reference.py:19-23)."""
    r = f32_to_bf16((bf16_to_f32(x_bits) + bf16_to_f32(delta_bits)).astype(F32))
    return r, rms_norm(r, w_bits, eps)


def add_rms_norm_partials(x_bits, planes, w_bits, eps):
    """reference.py:26-28: the planes are reduced to bf16 first."""
    return add_rms_norm(x_bits, reduce_partials(planes), w_bits, eps)


def silu_bf16(g):
    """bf16(g / (1 + exp(-g))) for fp32 g (reference.py:77)."""
    g = np.asarray(g, dtype=F32)
    with np.errstate(over="ignore"):
        return round_bf16((g / (F32(1.0) + np.exp(-g).astype(F32))).astype(F32))


def swiglu(gate_up_bits):
    """bf16(bf16(silu(gate)) * up) over [rows, 2I] (reference.py:74-79)."""
    inter = gate_up_bits.shape[1] // 2
    gate = bf16_to_f32(gate_up_bits[:, :inter])
    up = bf16_to_f32(gate_up_bits[:, inter:])
    return f32_to_bf16((silu_bf16(gate) * up).astype(F32))


def swiglu_partials(planes):
    """Planes summed in order, rounded to bf16, then swiglu (reference.py:82-86, swiglu.py:37-53)."""
    return swiglu(reduce_partials(planes))


def add_norm_quant(x_bits, planes, w_bits, eps):
    """Residual + RMSNorm + INT8 activation quantize (cuda_int8.py:17-44).

    Returns (residual bf16 bits, q int8 fragment order, s fp32 [M, N/64])."""
    r, y = add_rms_norm_partials(x_bits, planes, w_bits, eps)
    q, s = int8_quantize_activation(y)
    return r, q, s


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
