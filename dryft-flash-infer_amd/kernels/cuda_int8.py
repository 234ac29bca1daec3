"""Drop-in for the reference's ``kernels.cuda_int8`` (engine/kernels/cuda_int8.py) on MI355X.

INT8 W8A8: the ``cuda_fp8`` INT8 weights re-permuted into fragment order and made signed
(``^ 128``); activations quantized per row and 64-group with fp32 scales
(s = max(amax/127, 1e-20), q = rint(x/s)); per group the int8 dot product is taken on
the ``v_mfma_i32_16x16x64_i8`` matrix cores and accumulated as
acc = fma(float(dot) * s_x, s_w, acc) (cuda_int8.py:198-199), the optional residual
component after it. ``mode`` 0 gives bf16, 2 the SwiGLU epilogue (gate rows then up rows).
"""

import torch

from . import _lib, _linear


def quantize_activation(x, components=1):
    """``x`` bf16 [M, K] -> (q, s, r, rs): int8 in fragment order and fp32 [M, K/64] scales;
    with ``components=2`` also the quantized residual, else r, rs alias q, s."""
    if components not in (1, 2):
        raise ValueError("components is 1 or 2")
    if x.dtype != torch.bfloat16 or x.dim() != 2:
        raise ValueError("activation must be a 2-D bfloat16 tensor")
    m, k = x.shape
    if k % 64:
        raise ValueError(f"K={k} is not a multiple of 64")
    _lib.require_device(x)
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    s = torch.empty((m, k // 64), dtype=torch.float32, device=x.device)
    r = torch.empty_like(q) if components == 2 else q
    rs = torch.empty_like(s) if components == 2 else s
    _lib.call("qlx_quantize_act_int8", _lib.ptr(x), _lib.ptr(q), _lib.ptr(s),
              _lib.ptr(r) if components == 2 else None, _lib.ptr(rs) if components == 2 else None,
              m, k, _lib.stream(x.device))
    return q, s, r, rs


class Prepared:
    """INT8 weights in fragment order (cuda_int8.py:100-108), from a ``cuda_fp8.Prepared``."""

    def __init__(self, source):
        if getattr(source, "bits", 8) != 8:
            raise ValueError("W8A8 needs 8-bit weights")
        self.rows, self.k = source.rows, source.k
        rm = source.row_major()
        self.weight = torch.empty((self.rows, self.k), dtype=torch.int8, device=rm.device)
        _lib.call("qlx_int8_prepare", _lib.ptr(rm), _lib.ptr(self.weight), self.rows, self.k,
                  _lib.stream(rm.device))
        self.scale = source.scale


def _reduce_partials(planes):
    out = torch.empty(planes.shape[1:], dtype=torch.bfloat16, device=planes.device)
    _lib.call("qlx_reduce_planes", _lib.ptr(planes), _lib.ptr(out), planes[0].numel(), planes.shape[0],
              _lib.stream(planes.device))
    return out


def matmul_quantized(activation, prepared, config=(4, 1), components=1, mode=0):
    """``activation`` = (q, s, r, rs) from ``quantize_activation``; returns bf16
    ``[m, n]`` (mode 0) or ``[m, n/2]`` (mode 2, SwiGLU)."""
    x, sx, r, sr = activation
    m, k = x.shape
    if k != prepared.k:
        raise ValueError("activation width does not match the weight")
    if m > 64:
        raise ValueError(f"batch {m} exceeds 64 rows")
    warps, splits = config
    if mode == 2 and splits != 1:
        raise ValueError('SwiGLU requires no split K')
    if mode not in (0, 2):
        raise ValueError("mode is 0 (bf16) or 2 (SwiGLU)")
    _lib.require_device(x, sx, prepared.weight)
    lib_mode = _lib.MODE_SWIGLU if mode == 2 else _lib.MODE_BF16
    base = _linear.make_plan(_lib.FMT_INT8, lib_mode, m, prepared.rows, k)
    cfg = (base.waves, base.kw, base.rw, max(1, int(splits)))
    two = components == 2
    return _linear.run(_lib.FMT_INT8, "qlx_linear_int8", x, prepared.rows, k,
                       (_lib.ptr(prepared.weight), _lib.ptr(prepared.scale), _lib.ptr(x), _lib.ptr(sx),
                        _lib.ptr(r) if two else None, _lib.ptr(sr) if two else None),
                       mode=lib_mode, config=cfg, fit=True, comp=2 if two else 1)


def matmul(x, prepared, config=(4, 1), components=1, mode=0):
    activation = x if isinstance(x, tuple) else quantize_activation(x, components)
    return matmul_quantized(activation, prepared, config, components, mode)


def add_norm_quant(residual, delta, weight, eps):
    """Residual + RMSNorm with the reference's bf16 casts, then packed INT8 activations.

    ``delta`` is bf16 [m, n] or fp32 planes [splits, m, n] (cuda_int8.py:17-55)."""
    m, n = residual.shape
    if n % 64:
        raise ValueError(f"width {n} is not a multiple of 64")
    _lib.require_device(residual, delta, weight)
    out = torch.empty_like(residual)
    q = torch.empty_like(residual, dtype=torch.int8)
    scale = torch.empty((m, n // 64), device=residual.device, dtype=torch.float32)
    planes = delta.ndim == 3
    if planes and delta.dtype != torch.float32:
        raise ValueError("planes are fp32 [splits, rows, n]")
    _lib.call("qlx_add_norm_quant_int8", _lib.ptr(residual), None if planes else _lib.ptr(delta),
              _lib.ptr(delta) if planes else None, delta.shape[0] if planes else 0, _lib.ptr(weight),
              _lib.ptr(out), _lib.ptr(q), _lib.ptr(scale), m, n, float(eps), _lib.stream(residual.device))
    return out, (q, scale, q, scale)
