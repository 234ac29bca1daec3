"""numpy restatement of the reference's QKV consumer and decode attention (test oracle).

TEST INFRASTRUCTURE ONLY: imported by tests/ and bench.py's cpu_baseline leg; never by the
product path.

Covers engine/kernels/rope.py (per-head RMSNorm + RoPE, K/V cache writes, INT8 cache) as the
reference's torch statement gives it (engine/kernels/reference.py:31-113), and
engine/kernels/attention.py (grouped-query decode attention) as the SDPA it is checked against
(bench/gpu_checks.py:45-86). bf16 values travel as uint16 bit patterns.

Pinning (tests/test_oracle_attention.py):
  head_norm_rope       bit-exact against transformers' Qwen3RMSNorm + apply_rotary_pos_emb with
                       Qwen3RotaryEmbedding's tables (the reference's own check,
                       tests/test_numerics.py:67-102); planted sign and partner mistakes fail.
  qkv_norm_rope_to_cache / kv_int8_quantize
                       cache slots against the reference's slot rule (reference.py:57-71),
                       INT8 closed forms (+-amax -> +-127, ties round up, zero head), the
                       half-step bound of gpu_checks.py:238-245.
  decode_attention     torch's scaled_dot_product_attention with the causal mask of
                       gpu_checks.py:66-75; closed forms (equal keys -> mean of values, one
                       dominant key -> its value); NaN beyond the live keys never read.
"""

import numpy as np

from .qlinear_oracle import F32, bf16_to_f32, f32_to_bf16, round_bf16

__all__ = ["head_norm_rope", "qkv_norm_rope_to_cache", "kv_int8_quantize", "decode_attention"]

HEAD_DIM = 128


def head_norm_rope(x_bits, w_bits, cos_bits, sin_bits, eps):
    """Per-head RMSNorm then RoPE (reference.py:31-46; rope.py:24-36).

    ``x_bits`` [rows, heads, 128]; ``cos_bits``/``sin_bits`` [rows, 128] (each row's table row).
    scale = 1/sqrt(mean(x^2) + eps) in fp32 from the exact sum of squares (fp64 holds every
    square of a bf16 value and their sum over a head exactly, so the order does not matter);
    n = bf16(bf16(x scale) w); y = bf16(bf16(n cos) + bf16(rotate_half(n) sin)).
    """
    x = bf16_to_f32(x_bits)
    ss = (x.astype(np.float64) ** 2).sum(-1, keepdims=True)
    mean = (ss / HEAD_DIM).astype(F32)
    scale = (F32(1.0) / np.sqrt((mean + F32(eps)).astype(F32))).astype(F32)
    n = round_bf16(round_bf16((x * scale).astype(F32)) * bf16_to_f32(w_bits))
    half = HEAD_DIM // 2
    rot = np.concatenate([-n[..., half:], n[..., :half]], axis=-1)
    c = bf16_to_f32(cos_bits)[:, None, :]
    s = bf16_to_f32(sin_bits)[:, None, :]
    y = round_bf16(round_bf16((n * c).astype(F32)) + round_bf16((rot * s).astype(F32)))
    return f32_to_bf16(y)


def kv_int8_quantize(y):
    """INT8 cache codes of fp32 values [..., 128] (rope.py:108-118): scale = max(amax, 1e-12) / 127
    per head row (fp32), code = clamp(floor(y / scale + 0.5), -127, 127)."""
    y = np.asarray(y, dtype=F32)
    amax = np.abs(y).max(-1)
    scale = (np.maximum(amax, F32(1e-12)).astype(F32) / F32(127.0)).astype(F32)
    code = np.floor((y / scale[..., None]).astype(F32) + F32(0.5))
    return np.clip(code, -127, 127).astype(np.int8), scale


def qkv_norm_rope_to_cache(qkv_bits, n_q, n_kv, qw_bits, kw_bits, cos_bits, sin_bits, positions, seq_len,
                           k_cache, v_cache, eps, k_scale=None, v_scale=None, k_copy=None, v_copy=None):
    """Return Q bits [rows, n_q*128]; write rotated K and raw V (or their INT8 codes and scales)
    into slot positions[r % seq_len] of sequence r // seq_len (reference.py:49-100; rope.py:
    125-166). ``qkv_bits`` [rows, width] holds Q, K, V heads back to back. Caches are numpy
    arrays [batch, n_kv, capacity, 128] updated in place; copies [batch, n_kv, seq_len, 128]."""
    qkv_bits = np.asarray(qkv_bits, dtype=np.uint16)
    rows = qkv_bits.shape[0]
    pos = np.asarray(positions)[:seq_len].astype(np.int64)
    tok = np.arange(rows) % seq_len
    cos_rows = np.asarray(cos_bits)[pos[tok]]
    sin_rows = np.asarray(sin_bits)[pos[tok]]
    q = qkv_bits[:, : n_q * HEAD_DIM].reshape(rows, n_q, HEAD_DIM)
    k = qkv_bits[:, n_q * HEAD_DIM: (n_q + n_kv) * HEAD_DIM].reshape(rows, n_kv, HEAD_DIM)
    v = qkv_bits[:, (n_q + n_kv) * HEAD_DIM: (n_q + 2 * n_kv) * HEAD_DIM].reshape(rows, n_kv, HEAD_DIM)
    q_out = head_norm_rope(q, qw_bits, cos_rows, sin_rows, eps).reshape(rows, n_q * HEAD_DIM)
    if n_kv:
        kr = head_norm_rope(k, kw_bits, cos_rows, sin_rows, eps)
        for r in range(rows):
            b, t, p = r // seq_len, r % seq_len, pos[r % seq_len]
            if k_scale is not None:
                kc, ks = kv_int8_quantize(bf16_to_f32(kr[r]))
                vc, vs = kv_int8_quantize(bf16_to_f32(v[r]))
                k_cache[b, :, p], k_scale[b, :, p] = kc, ks
                v_cache[b, :, p], v_scale[b, :, p] = vc, vs
            else:
                k_cache[b, :, p] = kr[r]
                v_cache[b, :, p] = v[r]
            if k_copy is not None:
                k_copy[b, :, t] = kr[r]
                v_copy[b, :, t] = v[r]
    return q_out


def decode_attention(q_bits, k, v, pos, tokens, group, k_scale=None, v_scale=None):
    """Exact (fp64) grouped-query attention of a decode pass: query row (b, t) head h attends
    to keys 0 .. pos + t of KV head h // group with softmax(q k / sqrt(128)) -- the SDPA the
    reference's kernel is checked against (gpu_checks.py:66-75). ``k``/``v`` bf16 bits
    [batch, n_kv, capacity, 128], or INT8 codes with fp32 scales [batch, n_kv, capacity]
    (dequantised to bf16(code * scale), attention.py:94-99). Returns float64
    [batch * tokens, n_kv * group * 128]."""
    batch, n_kv, _, d = k.shape
    live = pos + tokens
    if k_scale is not None:
        kd = bf16_to_f32(f32_to_bf16(k[:, :, :live].astype(F32) * k_scale[:, :, :live, None]))
        vd = bf16_to_f32(f32_to_bf16(v[:, :, :live].astype(F32) * v_scale[:, :, :live, None]))
    else:
        kd = bf16_to_f32(k[:, :, :live])
        vd = bf16_to_f32(v[:, :, :live])
    kd, vd = kd.astype(np.float64), vd.astype(np.float64)
    q = bf16_to_f32(np.asarray(q_bits)).astype(np.float64).reshape(batch, tokens, n_kv, group, d)
    out = np.empty((batch, tokens, n_kv, group, d))
    scale = d ** -0.5
    for t in range(tokens):
        n = pos + t + 1
        s = np.einsum("bhgd,bhkd->bhgk", q[:, t], kd[:, :, :n]) * scale
        s -= s.max(-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(-1, keepdims=True)
        out[:, t] = np.einsum("bhgk,bhkd->bhgd", p, vd[:, :, :n])
    return out.reshape(batch * tokens, n_kv * group * d)
