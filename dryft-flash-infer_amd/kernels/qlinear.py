"""The north-star quantized formats: W8A16 per channel, W4A16 group 128, FP8 W8A8.

Each format is the reference's quantizer (engine/kernels/cuda_fp8.py:1127-1151,
engine/kernels/fp8.py:20-28) with documented substitutions, and each linear is a drop-in
for the ``cuda_fp8.matmul`` call the engine makes per projection
(engine/engine.py:881-884):

* W8A16: ``cuda_fp8.quantize(w, group=K, bits=8)`` with bf16 scales and signed int8
  storage -> ``(int8 [N, K], bf16 [N])``.
* W4A16: ``cuda_fp8.quantize(w, group=128, bits=4)`` with bf16 scales; codes ``q + 8``
  packed eight per int32 along K, nibble i of word j holding k = 8j + i ->
  ``(int32 [N, K/8], bf16 [N, K/128])``.
* FP8 W8A8: ``fp8.quantize(w, group=K)`` -> ``(e4m3 [N, K], bf16 [N])``; the activation
  is quantized per token inside the linear: ``s = max(amax/448, 1e-12)`` (fp32),
  ``e4m3(clamp(x/s, +-448))``.

``prepare(packed)`` relays a packed weight into the MI355X tile layout at load time (the
role of ``cuda_fp8.prepare``, engine/kernels/cuda_fp8.py:1220-1224); every linear accepts
either the row-major packed tuple or the prepared ``Tiled`` weight.

All work runs in the gfx950 library; tensors must be on the GPU.
"""

import ctypes

import torch

from . import _lib, _linear


class Tiled:
    """A packed weight relaid into 16-row x 128-byte tiles (``qlx_tile_rows``).

    ``weight`` holds the same bytes as the packed codes, in tile order; ``scale`` is
    unchanged; ``rows`` and ``k`` are the logical shape; ``fmt`` names the format.
    """

    __slots__ = ("weight", "scale", "rows", "k", "fmt")

    def __init__(self, weight, scale, rows, k, fmt):
        self.weight, self.scale, self.rows, self.k, self.fmt = weight, scale, rows, k, fmt

    def bytes_moved(self):
        return self.weight.numel() * self.weight.element_size() + self.scale.numel() * self.scale.element_size()


def prepare(packed, fmt=None):
    """Relay ``(codes, scales)`` of any north-star format into the tile layout."""
    q, s = packed
    _lib.require_device(q, s)
    rows = q.shape[0]
    row_bytes = q.shape[1] * q.element_size()
    if fmt is None:
        fmt = "w4a16" if q.dtype == torch.int32 else ("fp8" if q.dtype == torch.float8_e4m3fn else "w8a16")
    k = row_bytes * 2 if fmt == "w4a16" else row_bytes
    if rows % 16 or row_bytes % 128:
        raise ValueError(f"tiles need rows % 16 == 0 and 128-byte rows (got {rows} x {row_bytes} B)")
    out = torch.empty_like(q)
    _lib.call("qlx_tile_rows", _lib.ptr(q), _lib.ptr(out), rows, row_bytes, _lib.stream(q.device))
    return Tiled(out, s, rows, k, fmt)


def _unpack(packed, fmt):
    """(codes, scales, rows, k, tiled) of a packed tuple or a Tiled weight."""
    if isinstance(packed, Tiled):
        if packed.fmt != fmt:
            raise ValueError(f"a {packed.fmt} weight cannot feed a {fmt} linear")
        return packed.weight, packed.scale, packed.rows, packed.k, 1
    q, s = packed
    rows = q.shape[0]
    k = q.shape[1] * 8 if fmt == "w4a16" else q.shape[1]
    return q, s, rows, k, 0


def _bf16_2d(t, what):
    if t.dtype != torch.bfloat16 or t.dim() != 2:
        raise ValueError(f"{what} must be a 2-D bfloat16 tensor")
    _lib.require_device(t)


# ---- quantize / pack ------------------------------------------------------------------

def quantize_w8(weight):
    """bf16 ``[N, K]`` -> (int8 ``[N, K]``, bf16 per-channel scales ``[N]``)."""
    _bf16_2d(weight, "weight")
    n, k = weight.shape
    if k % 8:
        raise ValueError(f"K={k} must be a multiple of 8")
    q = torch.empty((n, k), dtype=torch.int8, device=weight.device)
    s = torch.empty((n, 1), dtype=torch.bfloat16, device=weight.device)
    _lib.call("qlx_quantize_weight", _lib.ptr(weight), _lib.ptr(q), _lib.ptr(s), n, k, k, 8,
              _lib.SCALE_BF16, 1, _lib.STORE_SIGNED, _lib.stream(weight.device))
    return q, s.view(n)


def quantize_w4(weight, group=128):
    """bf16 ``[N, K]`` -> (int32 k32 words ``[N, K/8]``, bf16 scales ``[N, K/group]``)."""
    _bf16_2d(weight, "weight")
    n, k = weight.shape
    if k % group or group % 8:
        raise ValueError(f"{k} is not a multiple of {group}")
    q = torch.empty((n, k // 8), dtype=torch.int32, device=weight.device)
    s = torch.empty((n, k // group), dtype=torch.bfloat16, device=weight.device)
    _lib.call("qlx_quantize_weight", _lib.ptr(weight), _lib.ptr(q), _lib.ptr(s), n, k, group, 4,
              _lib.SCALE_BF16, 1, _lib.STORE_K32, _lib.stream(weight.device))
    return q, s


def quantize_fp8(weight):
    """bf16 ``[N, K]`` -> (e4m3 ``[N, K]`` as ``torch.float8_e4m3fn``, bf16 scales ``[N]``)."""
    _bf16_2d(weight, "weight")
    n, k = weight.shape
    if k % 8:
        raise ValueError(f"K={k} must be a multiple of 8")
    q = torch.empty((n, k), dtype=torch.uint8, device=weight.device)
    s = torch.empty((n, 1), dtype=torch.bfloat16, device=weight.device)
    _lib.call("qlx_quantize_fp8_weight", _lib.ptr(weight), _lib.ptr(q), _lib.ptr(s), n, k, k,
              _lib.stream(weight.device))
    return q.view(torch.float8_e4m3fn), s.view(n)


def quantize_fp8_activation(x):
    """bf16 ``[M, K]`` -> (e4m3 ``[M, K]``, fp32 per-token scales ``[M]``)."""
    _bf16_2d(x, "activation")
    m, k = x.shape
    if k % 8:
        raise ValueError(f"K={k} must be a multiple of 8")
    q = torch.empty((m, k), dtype=torch.uint8, device=x.device)
    s = torch.empty((m,), dtype=torch.float32, device=x.device)
    _lib.call("qlx_quantize_fp8_act", _lib.ptr(x), _lib.ptr(q), _lib.ptr(s), m, k, _lib.stream(x.device))
    return q.view(torch.float8_e4m3fn), s


def dequantize_w8(packed):
    q, s = packed
    n, k = q.shape
    out = torch.empty((n, k), dtype=torch.bfloat16, device=q.device)
    _lib.call("qlx_dequantize", _lib.ptr(q), _lib.ptr(s), _lib.ptr(out), n, k, 1, 8,
              _lib.SCALE_BF16, _lib.STORE_SIGNED, _lib.stream(q.device))
    return out


def dequantize_w4(packed):
    q, s = packed
    n, k = q.shape[0], q.shape[1] * 8
    out = torch.empty((n, k), dtype=torch.bfloat16, device=q.device)
    _lib.call("qlx_dequantize", _lib.ptr(q), _lib.ptr(s), _lib.ptr(out), n, k, s.shape[1], 4,
              _lib.SCALE_BF16, _lib.STORE_K32, _lib.stream(q.device))
    return out


def dequantize_fp8(packed):
    """bf16(e4m3 code * bf16 scale) per output channel."""
    q, s = packed
    return (q.float() * s.float()[:, None]).to(torch.bfloat16)


def dequantize(packed, fmt):
    """The bf16 weight a north-star ``(codes, scales)`` pair stands for."""
    return {"w8a16": dequantize_w8, "w4a16": dequantize_w4, "fp8": dequantize_fp8}[fmt](packed)


# ---- linears ---------------------------------------------------------------------------

def _check_x(x, k):
    _bf16_2d(x, "activation")
    if x.shape[1] != k:
        raise ValueError("activation width does not match the weight")
    if not 1 <= x.shape[0] <= 64:
        raise ValueError(f"batch {x.shape[0]} exceeds 64 rows")


def _mode(swiglu=False, planes=False):
    return _lib.MODE_SWIGLU if swiglu else (_lib.MODE_PLANES if planes else _lib.MODE_BF16)


def _skinny(fmt, q, s, x, n, k, swiglu, fused_reduce=None):
    """The skinny GEMM (``qlx_linear_skinny``): the activation streams through LDS per K step.
    K slices write fp32 planes that the row group's last workgroup reduces in slice order
    (``fused_reduce``: split-K tickets) or a second launch reduces (bit-identical)."""
    m = x.shape[0]
    if fused_reduce is None:
        fused_reduce = True
    mode = _lib.MODE_SWIGLU if swiglu else _lib.MODE_BF16
    plan = _lib.Plan()
    _lib.check(_lib.lib().qlx_plan_skinny(fmt, mode, m, n, k, plan), "plan_skinny")
    out = torch.empty((m, n // 2 if swiglu else n), dtype=torch.bfloat16, device=x.device)
    work = None
    if plan.splits > 1:  # fp32 planes, reduced in slice order inside the call
        work = torch.empty((plan.splits, m, n), dtype=torch.float32, device=x.device)
        plan.workspace = work.data_ptr()
        if fused_reduce:  # one counter per row group: n / 16 always suffices
            plan.tickets = _lib.tickets(x.device, n // 16).data_ptr()
    _lib.call("qlx_linear_skinny", fmt, _lib.ptr(q), _lib.ptr(s), _lib.ptr(x), _lib.ptr(out), m, n, k,
              ctypes.byref(plan), _lib.stream(x.device))
    return out


#: From this many tokens the skinny GEMM is the default (tile-layout W4A16/W8A16
#: weights, library plan): at 16-64 tokens it is 1.5-7.5x faster than the decode kernel.
SKINNY_FROM = 9


def _use_skinny(skinny, x, tiled, planes, config):
    if skinny is None:
        return bool(tiled) and not planes and config is None and x.shape[0] >= SKINNY_FROM
    if skinny and (not tiled or planes or config is not None):
        raise ValueError("the skinny GEMM takes tile-layout weights, bf16 or SwiGLU output, its own plan")
    return bool(skinny)


def linear_w8a16(x, packed, config=None, planes=False, swiglu=False, skinny=None):
    """``x @ deq(W).T`` for W8A16 per-channel weights; bf16 ``[M, N]`` (SwiGLU: ``[M, N/2]``).
    ``skinny`` (None: from 9 tokens on tile-layout weights) runs the skinny GEMM, whose
    activation streams through LDS per K step; False forces the decode kernel."""
    q, s, n, k, tiled = _unpack(packed, "w8a16")
    _check_x(x, k)
    _lib.require_device(q, s)
    if s.numel() != n:
        raise ValueError("W8A16 scales are one bf16 per output channel")
    if _use_skinny(skinny, x, tiled, planes, config):
        return _skinny(_lib.FMT_W8A16, q, s, x, n, k, swiglu)
    return _linear.run(_lib.FMT_W8A16, "qlx_linear_w8a16", x, n, k,
                       (_lib.ptr(q), _lib.ptr(s), _lib.ptr(x)), (tiled,), mode=_mode(swiglu, planes), config=config)


def linear_w4a16(x, packed, config=None, planes=False, swiglu=False, skinny=None):
    """``x @ deq(W).T`` for W4A16 group-128 weights (``skinny``: as in ``linear_w8a16``)."""
    q, s, n, k, tiled = _unpack(packed, "w4a16")
    _check_x(x, k)
    _lib.require_device(q, s)
    if q.dtype != torch.int32 or tuple(s.shape) != (n, k // 128):
        raise ValueError("W4A16 weights are int32 [N, K/8] with bf16 scales [N, K/128]")
    if _use_skinny(skinny, x, tiled, planes, config):
        return _skinny(_lib.FMT_W4A16, q, s, x, n, k, swiglu)
    return _linear.run(_lib.FMT_W4A16, "qlx_linear_w4a16", x, n, k,
                       (_lib.ptr(q), _lib.ptr(s), _lib.ptr(x)), (tiled,), mode=_mode(swiglu, planes), config=config)


#: From this many tokens the FP8 activation is quantized by its own kernel before the GEMM;
#: one token's row is cheaper to read inside every workgroup.
FP8_QUANTIZE_FROM = 2


def _skinny_fp8(q, s, xq, sx, n, k, swiglu, fused_reduce=None):
    """The FP8 W8A8 skinny GEMM (``qlx_linear_skinny_fp8``) on codes quantized beforehand; K
    slices reduced as in ``_skinny``."""
    m = xq.shape[0]
    if fused_reduce is None:
        fused_reduce = True
    mode = _lib.MODE_SWIGLU if swiglu else _lib.MODE_BF16
    plan = _lib.Plan()
    _lib.check(_lib.lib().qlx_plan_skinny(_lib.FMT_FP8, mode, m, n, k, plan), "plan_skinny")
    out = torch.empty((m, n // 2 if swiglu else n), dtype=torch.bfloat16, device=xq.device)
    work = None
    if plan.splits > 1:
        work = torch.empty((plan.splits, m, n), dtype=torch.float32, device=xq.device)
        plan.workspace = work.data_ptr()
        if fused_reduce:
            plan.tickets = _lib.tickets(xq.device, n // 16).data_ptr()
    _lib.call("qlx_linear_skinny_fp8", _lib.ptr(q), _lib.ptr(s), _lib.ptr(xq), _lib.ptr(sx), _lib.ptr(out), m, n, k,
              ctypes.byref(plan), _lib.stream(xq.device))
    return out


def linear_fp8_w8a8(x, packed, config=None, planes=False, swiglu=False, pre_quantize=None, skinny=None):
    """``(x_q s_x) @ (W_q s_w).T`` with the activation quantized per token (``pre_quantize``:
    None = by its own kernel from 2 tokens, else inside the GEMM; the codes are the same).
    ``skinny`` (None: from 9 tokens on tile-layout weights) runs the skinny GEMM on the
    quantized codes; False forces the decode kernel."""
    q, s, n, k, tiled = _unpack(packed, "fp8")
    _check_x(x, k)
    _lib.require_device(q, s)
    if s.numel() != n:
        raise ValueError("FP8 W8A8 weight scales are one bf16 per output channel")
    if skinny is None and pre_quantize is not None:  # a decode-kernel variant was asked for
        skinny = False
    if _use_skinny(skinny, x, tiled, planes, config):
        if pre_quantize is False:
            raise ValueError("the FP8 skinny GEMM takes the activation quantized beforehand")
        xq, sx = quantize_fp8_activation(x)
        return _skinny_fp8(q, s, xq, sx, n, k, swiglu)
    if pre_quantize is None:
        pre_quantize = x.shape[0] >= FP8_QUANTIZE_FROM and k % 128 == 0
    if pre_quantize:
        xq, sx = quantize_fp8_activation(x)
        return _linear.run(_lib.FMT_FP8, "qlx_linear_fp8_w8a8_q", x, n, k,
                           (_lib.ptr(q), _lib.ptr(s), _lib.ptr(xq), _lib.ptr(sx)), (tiled,),
                           mode=_mode(swiglu, planes), config=config)
    return _linear.run(_lib.FMT_FP8, "qlx_linear_fp8_w8a8", x, n, k,
                       (_lib.ptr(q), _lib.ptr(s), _lib.ptr(x)), (tiled,), mode=_mode(swiglu, planes), config=config)


def linear_fp8_w8a8_quantized(xq, sx, packed, config=None, planes=False, swiglu=False, skinny=None):
    """FP8 W8A8 linear of an activation quantized beforehand: e4m3 codes ``xq`` [m, k] with
    fp32 per-token scales ``sx`` [m] (``quantize_fp8_activation`` or ``add_norm_quant_fp8``).
    ``skinny`` as for ``linear_fp8_w8a8``."""
    q, s, n, k, tiled = _unpack(packed, "fp8")
    if xq.ndim != 2 or xq.shape[1] != k or xq.element_size() != 1:
        raise ValueError("codes must be one byte each, [m, k] with k the weight's width")
    if sx.dtype != torch.float32 or sx.numel() != xq.shape[0]:
        raise ValueError("token scales are fp32 [m]")
    if not 1 <= xq.shape[0] <= 64:
        raise ValueError(f"batch {xq.shape[0]} exceeds 64 rows")
    _lib.require_device(q, s, xq, sx)
    if _use_skinny(skinny, xq, tiled, planes, config):
        return _skinny_fp8(q, s, xq.view(torch.uint8), sx, n, k, swiglu)
    return _linear.run(_lib.FMT_FP8, "qlx_linear_fp8_w8a8_q", xq, n, k,
                       (_lib.ptr(q), _lib.ptr(s), _lib.ptr(xq), _lib.ptr(sx)), (tiled,),
                       mode=_mode(swiglu, planes), config=config)


def add_norm_quant_fp8(residual, delta, weight, eps, keep_normed=False):
    """Residual + RMSNorm with the reference's bf16 casts, then the FP8 per-token activation of
    the normed row, in one launch: the FP8 W8A8 counterpart of ``cuda_int8.add_norm_quant``
    (engine/kernels/cuda_int8.py:17-55). ``delta`` is bf16 [m, n], fp32 planes [splits, m, n] or
    None (plain RMSNorm). Returns (residual out or None, codes e4m3 [m, n], scales fp32 [m]) and,
    with ``keep_normed``, the normed bf16 row too."""
    _bf16_2d(residual, "residual")
    m, n = residual.shape
    if n % 8:
        raise ValueError(f"width {n} is not a multiple of 8")
    planes = delta is not None and delta.ndim == 3
    if planes and delta.dtype != torch.float32:
        raise ValueError("planes are fp32 [splits, rows, n]")
    if delta is not None and tuple(delta.shape[-2:]) != (m, n):
        raise ValueError("delta does not match the residual")
    _lib.require_device(residual, weight, *(() if delta is None else (delta,)))
    res = torch.empty_like(residual) if delta is not None else None
    normed = torch.empty_like(residual) if keep_normed else None
    code = torch.empty((m, n), dtype=torch.uint8, device=residual.device)
    scale = torch.empty(m, dtype=torch.float32, device=residual.device)
    _lib.call("qlx_add_norm_quant_fp8", _lib.ptr(residual),
              None if (delta is None or planes) else _lib.ptr(delta), _lib.ptr(delta) if planes else None,
              delta.shape[0] if planes else 0, _lib.ptr(weight), None if res is None else _lib.ptr(res),
              None if normed is None else _lib.ptr(normed), _lib.ptr(code), _lib.ptr(scale), m, n, float(eps),
              _lib.stream(residual.device))
    out = (res, code.view(torch.float8_e4m3fn), scale)
    return out + (normed,) if keep_normed else out


def splits(fmt, m, n, k, config=None, swiglu=False):
    """How many fp32 planes a linear of this shape and config reduces."""
    return _linear.splits_for(fmt, _mode(swiglu), m, n, k, config)


FORMATS = {
    "w8a16": (quantize_w8, linear_w8a16, _lib.FMT_W8A16),
    "w4a16": (quantize_w4, linear_w4a16, _lib.FMT_W4A16),
    "fp8": (quantize_fp8, linear_fp8_w8a8, _lib.FMT_FP8),
}


def weight_bytes(packed):
    """Bytes a linear streams for its weight (codes + scales)."""
    if isinstance(packed, Tiled):
        return packed.bytes_moved()
    q, s = packed
    return q.numel() * q.element_size() + s.numel() * s.element_size()
