"""Pins of the QKV-consumer and decode-attention oracle (oracle/attention_oracle.py) on the CPU:
transformers' Qwen3 modules, torch's SDPA, closed forms and planted mistakes."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.attention_oracle as A
from oracle import bf16_to_f32, f32_to_bf16

EPS = 1e-6
THETA = 5_000_000.0


def bits16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def tables(n):
    """cos/sin bf16 rows for positions 0..n-1, built as transformers' Qwen3RotaryEmbedding does
    (and as the engine's table, engine/engine.py:350-358)."""
    from transformers.models.qwen3.configuration_qwen3 import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding
    cfg = Qwen3Config(hidden_size=2560, intermediate_size=9728, num_hidden_layers=1, num_attention_heads=32,
                      num_key_value_heads=8, head_dim=128, rms_norm_eps=EPS,
                      rope_parameters={"rope_type": "default", "rope_theta": THETA})
    rotary = Qwen3RotaryEmbedding(cfg)
    cos, sin = rotary(torch.zeros(1, n, 8, dtype=torch.float32), torch.arange(n).unsqueeze(0))
    return cos[0].to(torch.bfloat16), sin[0].to(torch.bfloat16)


def test_head_norm_rope_matches_transformers():
    """tests/test_numerics.py:67-102 of the reference: q_norm then apply_rotary_pos_emb."""
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm, apply_rotary_pos_emb
    torch.manual_seed(2)
    batch, heads, seq = 2, 8, 6
    q = torch.randn(batch, seq, heads, 128, dtype=torch.bfloat16) * 3
    norm = Qwen3RMSNorm(128, eps=EPS).to(torch.bfloat16)
    norm.weight.data = torch.randn(128, dtype=torch.bfloat16)
    cos, sin = tables(seq)
    with torch.no_grad():
        want, _ = apply_rotary_pos_emb(norm(q).transpose(1, 2), norm(q).transpose(1, 2),
                                       cos.unsqueeze(0), sin.unsqueeze(0))
    want = bits16(want.transpose(1, 2).reshape(batch * seq, heads, 128))
    rows = np.tile(np.arange(seq), batch)
    got = A.head_norm_rope(bits16(q.reshape(batch * seq, heads, 128)), bits16(norm.weight.data),
                           bits16(cos)[rows], bits16(sin)[rows], EPS)
    assert np.array_equal(got, want)

    # planted mistakes: rotate_half's sign, or the partner taken before normalisation
    x = bf16_to_f32(bits16(q.reshape(batch * seq, heads, 128)))
    scale = 1 / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + EPS)
    n = bf16_to_f32(f32_to_bf16(bf16_to_f32(f32_to_bf16((x * scale).astype(np.float32)))
                                * bf16_to_f32(bits16(norm.weight.data))))
    c, s = bf16_to_f32(bits16(cos)[rows])[:, None], bf16_to_f32(bits16(sin)[rows])[:, None]
    wrong_sign = np.concatenate([n[..., 64:], -n[..., :64]], -1)
    bad = f32_to_bf16(bf16_to_f32(f32_to_bf16(n * c)) + bf16_to_f32(f32_to_bf16(wrong_sign * s)))
    assert not np.array_equal(bad, want)
    raw_partner = np.concatenate([-x[..., 64:], x[..., :64]], -1)
    bad = f32_to_bf16(bf16_to_f32(f32_to_bf16(n * c)) + bf16_to_f32(f32_to_bf16(raw_partner * s)))
    assert not np.array_equal(bad, want)


def test_cache_slots_follow_positions_and_sequences():
    """Row r is token r % seq_len of sequence r // seq_len and lands in slot positions[token]
    (reference.py:57-71); other slots stay untouched; V is copied raw."""
    g = torch.Generator().manual_seed(5)
    n_q, n_kv, seq_len, batch, cap = 4, 2, 3, 2, 12
    qkv = bits16(torch.randn(batch * seq_len, (n_q + 2 * n_kv) * 128, generator=g).to(torch.bfloat16))
    qw = bits16(torch.randn(128, generator=g).to(torch.bfloat16))
    kw = bits16(torch.randn(128, generator=g).to(torch.bfloat16))
    cos, sin = tables(cap)
    pos = np.array([7, 2, 9], np.int32)
    kc = np.full((batch, n_kv, cap, 128), 0x1234, np.uint16)
    vc = kc.copy()
    q = A.qkv_norm_rope_to_cache(qkv, n_q, n_kv, qw, kw, bits16(cos), bits16(sin), pos, seq_len, kc, vc, EPS)
    assert q.shape == (batch * seq_len, n_q * 128)
    for r in range(batch * seq_len):
        b, t = divmod(r, seq_len)
        v = qkv[r, (n_q + n_kv) * 128:].reshape(n_kv, 128)
        assert np.array_equal(vc[b, :, pos[t]], v)
        k = A.head_norm_rope(qkv[r, n_q * 128:(n_q + n_kv) * 128].reshape(1, n_kv, 128), kw,
                             bits16(cos)[pos[t]][None], bits16(sin)[pos[t]][None], EPS)[0]
        assert np.array_equal(kc[b, :, pos[t]], k)
    untouched = np.ones(cap, bool)
    untouched[pos] = False
    assert (kc[:, :, untouched] == 0x1234).all() and (vc[:, :, untouched] == 0x1234).all()


def test_int8_cache_quantize_closed_forms():
    y = np.zeros((3, 128), np.float32)
    y[0, 5], y[0, 9] = 127.0, -127.0     # scale 1: +-amax -> +-127
    y[0, 11] = 2.5                       # exact tie: floor(2.5 + 0.5) = 3 (round half up, not even)
    y[0, 12] = -2.5                      # floor(-2.5 + 0.5) = -2
    y[1] = 0.0                           # zero head: scale 1e-12 / 127, codes 0
    y[2] = np.linspace(-3, 3, 128, dtype=np.float32)
    code, scale = A.kv_int8_quantize(y)
    assert scale[0] == np.float32(1.0) and code[0, 5] == 127 and code[0, 9] == -127
    assert code[0, 11] == 3 and code[0, 12] == -2
    assert scale[1] == np.float32(np.float32(1e-12) / np.float32(127)) and not code[1].any()
    err = np.abs(code[2].astype(np.float32) * scale[2] - y[2])
    assert (err <= scale[2] * 0.5 + 1e-6).all()  # the half-step bound of gpu_checks.py:238-245
    assert np.array_equal(A.kv_int8_quantize(-y)[0][2], -code[2])


def sdpa(q_bits, k_bits, v_bits, pos, tokens, group):
    """torch's SDPA with the causal mask of bench/gpu_checks.py:66-75 (fp32, CPU)."""
    batch, n_kv, _, d = k_bits.shape
    live = pos + tokens
    q = torch.from_numpy(bf16_to_f32(q_bits)).view(batch, tokens, n_kv * group, d).transpose(1, 2)
    k = torch.from_numpy(bf16_to_f32(k_bits[:, :, :live])).repeat_interleave(group, 1)
    v = torch.from_numpy(bf16_to_f32(v_bits[:, :, :live])).repeat_interleave(group, 1)
    mask = torch.arange(live)[None, :] <= pos + torch.arange(tokens)[:, None]
    out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask)
    return out.transpose(1, 2).reshape(batch * tokens, -1).numpy().astype(np.float64)


@pytest.mark.parametrize("batch,tokens,pos", [(1, 1, 0), (2, 1, 37), (1, 3, 20), (2, 2, 61)])
def test_decode_attention_matches_sdpa(batch, tokens, pos):
    g = torch.Generator().manual_seed(47 + pos)
    n_kv, group, cap = 2, 4, 64
    q = bits16(torch.randn(batch * tokens, n_kv * group * 128, generator=g).to(torch.bfloat16))
    k = bits16(torch.randn(batch, n_kv, cap, 128, generator=g).to(torch.bfloat16))
    v = bits16(torch.randn(batch, n_kv, cap, 128, generator=g).to(torch.bfloat16))
    # keys past the last live one hold NaN: the oracle must never read them
    k[:, :, pos + tokens:] = 0x7FC0
    v[:, :, pos + tokens:] = 0x7FC0
    got = A.decode_attention(q, k, v, pos, tokens, group)
    want = sdpa(q, k, v, pos, tokens, group)
    assert np.isfinite(got).all()
    assert np.abs(got - want).max() < 1e-5


def test_decode_attention_closed_forms():
    g = torch.Generator().manual_seed(9)
    n_kv, group, cap, pos = 1, 4, 16, 9
    q = bits16(torch.randn(2, n_kv * group * 128, generator=g).to(torch.bfloat16))
    v = bits16(torch.randn(1, n_kv, cap, 128, generator=g).to(torch.bfloat16))
    # equal keys: uniform softmax, each token averages its live values (token t sees pos + t + 1)
    k = np.tile(bits16(torch.randn(128, generator=g).to(torch.bfloat16)), (1, n_kv, cap, 1))
    got = A.decode_attention(q, k, v, pos, 2, group).reshape(2, group, 128)
    vf = bf16_to_f32(v[0, 0]).astype(np.float64)
    for t in range(2):
        assert np.allclose(got[t], vf[: pos + t + 1].mean(0)[None], atol=1e-12)
    # one key aligned with every query row and far larger than the rest: its value comes back
    k = np.zeros((1, n_kv, cap, 128), np.uint16)
    qf = np.zeros((1, n_kv * group * 128), np.float32)
    qf[0, ::128] = 8.0
    kk = np.zeros((1, n_kv, cap, 128), np.float32)
    kk[0, 0, 4, 0] = 64.0  # score 8 * 64 / sqrt(128) = 45 against 0 for every other key
    got = A.decode_attention(f32_to_bf16(qf), f32_to_bf16(kk), v, pos, 1, group).reshape(group, 128)
    assert np.allclose(got, vf[4][None], atol=1e-12)


def test_decode_attention_int8_dequantises_to_bf16():
    g = torch.Generator().manual_seed(61)
    batch, n_kv, group, cap, pos = 1, 2, 4, 40, 30
    q = bits16(torch.randn(batch, n_kv * group * 128, generator=g).to(torch.bfloat16))
    kf = torch.randn(batch, n_kv, cap, 128, generator=g)
    vf = torch.randn(batch, n_kv, cap, 128, generator=g)
    ks = (kf.abs().amax(-1) / 127).numpy()
    vs = (vf.abs().amax(-1) / 127).numpy()
    k8 = np.clip(np.round(kf.numpy() / ks[..., None]), -127, 127).astype(np.int8)
    v8 = np.clip(np.round(vf.numpy() / vs[..., None]), -127, 127).astype(np.int8)
    got = A.decode_attention(q, k8, v8, pos, 1, group, ks, vs)
    kd = f32_to_bf16(k8.astype(np.float32) * ks[..., None])
    vd = f32_to_bf16(v8.astype(np.float32) * vs[..., None])
    assert np.abs(got - sdpa(q, kd, vd, pos, 1, group)).max() < 1e-5
