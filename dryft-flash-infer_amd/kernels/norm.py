"""Drop-in for the reference's ``kernels.norm`` plane consumers (engine/kernels/norm.py).

RMSNorm with ``Qwen3RMSNorm``'s cast placement -- the normalised value rounds to bf16
before the weight multiply (norm.py:1-10) -- and the residual add fused in front of it,
the delta given in bf16 or as fp32 split-K planes reduced in slice order.
"""

import torch

from . import _lib


def _add_norm(x, delta, planes, weight, eps):
    rows, n = x.shape
    _lib.require_device(x, weight, delta, planes)
    residual = torch.empty_like(x)
    out = torch.empty_like(x)
    _lib.call("qlx_add_rms_norm", _lib.ptr(x), _lib.ptr(delta) if delta is not None else None,
              _lib.ptr(planes) if planes is not None else None, planes.shape[0] if planes is not None else 0,
              _lib.ptr(weight), _lib.ptr(residual), _lib.ptr(out), rows, n, float(eps), _lib.stream(x.device))
    return residual, out


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    from .cuda_small import rms_norm as _rms
    return _rms(x, weight, eps)


def add_rms_norm(x, delta, weight, eps):
    """``(bf16(x + delta), rms_norm of it)``."""
    return _add_norm(x, delta, None, weight, eps)


def add_rms_norm_partials(x, partials, weight, eps):
    """``add_rms_norm`` where ``delta`` arrives as fp32 planes ``[splits, rows, n]``."""
    return _add_norm(x, None, partials, weight, eps)


def add_rms_norm_separate(x, delta, weight, eps):
    return add_rms_norm(x, delta, weight, eps)


def add_rms_norm_partials_separate(x, partials, weight, eps):
    return add_rms_norm_partials(x, partials, weight, eps)
