"""Per-head RMSNorm + RoPE with K and V written straight into the cache: drop-in for the
reference's ``kernels.rope`` (engine/kernels/rope.py:221-329).

One HIP launch (``qlx_qkv_norm_rope``, csrc/rope.hip) reads the fused QKV projection in
place -- bf16 by row stride and column offset, or its unreduced fp32 split-K planes --
normalises each 128-value Q and K head with its gain, rotates it by the cos/sin row of the
token's absolute position, returns Q and writes the rotated K and the raw V into the cache
slot the position names. The roundings are the reference's (engine/kernels/reference.py:31-46).
The INT8 cache layout (``k_scale``/``v_scale``) and the bf16 copies for prefill's SDPA
(``k_copy``/``v_copy``) follow rope.py:96-122.
"""

import ctypes

import torch

from . import _lib

_HEAD_DIM = 128


def _check_cache(k_cache, v_cache, k_scale, v_scale, k_copy, v_copy):
    quant = k_scale is not None
    if quant != (k_cache.dtype == torch.int8) or (v_scale is not None) != quant:
        raise ValueError("scales must be given exactly when the cache is INT8")
    if (k_copy is None) != (v_copy is None):
        raise ValueError("give both bf16 copies or neither")
    want = torch.int8 if quant else torch.bfloat16
    if k_cache.dtype != want or v_cache.dtype != want:
        raise ValueError("K and V caches must both be bfloat16 (or both INT8 with scales)")
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape or k_cache.shape[3] != _HEAD_DIM:
        raise ValueError("caches must be [batch, n_kv, capacity, 128] and alike")
    _lib.require_device(k_cache, v_cache, k_scale, v_scale, k_copy, v_copy)
    if quant and (k_scale.dtype != torch.float32 or k_scale.shape != k_cache.shape[:3]
                  or v_scale.shape != k_cache.shape[:3] or v_scale.dtype != torch.float32):
        raise ValueError("cache scales must be fp32 [batch, n_kv, capacity]")


def _launch(source, planes, n_q, n_kv, q_col, k_col, v_col, q_weight, k_weight, cos, sin, positions, seq_len,
            k_cache, v_cache, eps, out, k_scale=None, v_scale=None, k_copy=None, v_copy=None):
    if planes is not None:
        if planes.dim() != 3 or planes.dtype != torch.float32:
            raise ValueError("planes must be fp32 [splits, rows, width]")
        _lib.require_device(planes)
        splits, rows, stride = planes.shape
        device = planes.device
    else:
        if source.dim() != 2 or source.dtype != torch.bfloat16 or source.stride(1) != 1:
            raise ValueError("qkv must be a bfloat16 [rows, width] matrix with unit column stride")
        if source.device.type != "cuda":
            raise ValueError("norm_rope needs tensors on a ROCm GPU (no CPU path)")
        splits, (rows, stride) = 0, (source.shape[0], source.stride(0))
        if source.data_ptr() % 16 or stride % 8:
            raise ValueError("qkv rows must start on 16-byte boundaries")
        device = source.device
    if cos.dtype != torch.bfloat16 or sin.dtype != torch.bfloat16 or cos.shape != sin.shape or cos.dim() != 2 \
            or cos.shape[1] != _HEAD_DIM:
        raise ValueError("cos/sin must be bfloat16 [positions, 128] tables of one shape")
    if positions.dtype not in (torch.int32, torch.int64) or positions.dim() != 1 or positions.numel() < seq_len:
        raise ValueError("positions must be a 1-D int32/int64 tensor with at least seq_len entries")
    if seq_len < 1 or rows % seq_len:
        raise ValueError("rows must be a whole number of sequences of seq_len tokens")
    _lib.require_device(cos, sin, positions, q_weight, k_weight, out)
    for w in (q_weight, k_weight):
        if w is not None and (w.dtype != torch.bfloat16 or w.numel() != _HEAD_DIM):
            raise ValueError("head norm weights must be bfloat16 [128]")
    capacity = 0
    if n_kv:
        _check_cache(k_cache, v_cache, k_scale, v_scale, k_copy, v_copy)
        if k_cache.shape[0] * seq_len < rows or k_cache.shape[1] != n_kv:
            raise ValueError("caches must hold every sequence of the pass and n_kv heads")
        if k_copy is not None and (k_copy.dtype != torch.bfloat16 or k_copy.shape != v_copy.shape
                                   or tuple(k_copy.shape) != (k_cache.shape[0], n_kv, seq_len, _HEAD_DIM)):
            raise ValueError("bf16 copies must be [batch, n_kv, seq_len, 128]")
        capacity = k_cache.shape[2]
    a = _lib.RopeArgs()
    a.qkv = source.data_ptr() if planes is None else None
    a.planes = planes.data_ptr() if planes is not None else None
    a.stride, a.splits, a.rows = stride, splits, rows
    a.n_q, a.n_kv, a.q_col, a.k_col, a.v_col = n_q, n_kv, q_col, k_col, v_col
    a.seq_len, a.capacity, a.table_rows = seq_len, capacity, cos.shape[0]
    a.pos_int64 = int(positions.dtype == torch.int64)
    a.eps = float(eps)
    a.q_norm_w = q_weight.data_ptr() if q_weight is not None else None
    a.k_norm_w = k_weight.data_ptr() if k_weight is not None else None
    a.cos, a.sin, a.positions = cos.data_ptr(), sin.data_ptr(), positions.data_ptr()
    a.q_out = out.data_ptr() if out is not None else None
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache), ("k_scale", k_scale), ("v_scale", v_scale),
                    ("k_copy", k_copy), ("v_copy", v_copy)):
        setattr(a, name, t.data_ptr() if (t is not None and n_kv) else None)
    _lib.call("qlx_qkv_norm_rope", ctypes.byref(a), _lib.stream(device))


def qkv_norm_rope_to_cache(
    qkv, n_q, n_kv, q_weight, k_weight, cos, sin, positions, seq_len,
    k_cache, v_cache, eps, k_scale=None, v_scale=None, k_copy=None, v_copy=None,
):
    """Return Q and write K/V in one launch (rope.py:221-240). ``qkv`` holds Q, K and V heads
    back to back; ``k_scale``/``v_scale`` select the INT8 cache, ``k_copy``/``v_copy`` also
    receive the bf16 K/V of this pass."""
    rows = qkv.shape[0]
    out = torch.empty((rows, n_q * _HEAD_DIM), dtype=torch.bfloat16, device=qkv.device)
    _launch(qkv, None, n_q, n_kv, 0, n_q * _HEAD_DIM, (n_q + n_kv) * _HEAD_DIM, q_weight, k_weight, cos, sin,
            positions, seq_len, k_cache, v_cache, eps, out, k_scale, v_scale, k_copy, v_copy)
    return out


def qkv_planes_norm_rope_to_cache(
    planes, n_q, n_kv, q_weight, k_weight, cos, sin, positions, seq_len,
    k_cache, v_cache, eps, k_scale=None, v_scale=None, k_copy=None, v_copy=None,
):
    """``qkv_norm_rope_to_cache`` over fp32 split-K planes ``[splits, rows, width]`` (rope.py:
    200-218): each value is the slice-order sum of the planes rounded once to bf16."""
    rows = planes.shape[1]
    out = torch.empty((rows, n_q * _HEAD_DIM), dtype=torch.bfloat16, device=planes.device)
    _launch(None, planes, n_q, n_kv, 0, n_q * _HEAD_DIM, (n_q + n_kv) * _HEAD_DIM, q_weight, k_weight, cos, sin,
            positions, seq_len, k_cache, v_cache, eps, out, k_scale, v_scale, k_copy, v_copy)
    return out


def q_norm_rope(qkv, n_heads, weight, cos, sin, positions, seq_len, eps):
    """Q from the first ``n_heads * 128`` columns of ``qkv``, normed and rotated (rope.py:243-263)."""
    rows = qkv.shape[0]
    out = torch.empty((rows, n_heads * _HEAD_DIM), dtype=qkv.dtype, device=qkv.device)
    _launch(qkv, None, n_heads, 0, 0, 0, 0, weight, None, cos, sin, positions, seq_len, None, None, eps, out)
    return out


def kv_norm_rope_to_cache(qkv, k_offset, n_heads, weight, cos, sin, positions, seq_len, k_cache, v_cache, eps):
    """Norm and rotate K (at column ``k_offset``), copy V (right after it), and write both to
    the slots ``positions`` names (rope.py:266-297)."""
    _launch(qkv, None, 0, n_heads, 0, k_offset, k_offset + n_heads * _HEAD_DIM, None, weight, cos, sin, positions,
            seq_len, k_cache, v_cache, eps, None)
