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
    """RMSNorm over the last dimension of a contiguous ``[rows, n]`` tensor (norm.py:98-104): the
    add-norm kernel with neither delta nor planes, and no residual written."""
    rows, n = x.shape
    _lib.require_device(x, weight)
    out = torch.empty_like(x)
    _lib.call("qlx_add_rms_norm", _lib.ptr(x), None, None, 0, _lib.ptr(weight), None, _lib.ptr(out),
              rows, n, float(eps), _lib.stream(x.device))
    return out


def add_rms_norm(x, delta, weight, eps):
    """``(bf16(x + delta), rms_norm of it)``."""
    return _add_norm(x, delta, None, weight, eps)


def add_rms_norm_partials(x, partials, weight, eps):
    """``add_rms_norm`` where ``delta`` arrives as fp32 planes ``[splits, rows, n]``."""
    return _add_norm(x, None, partials, weight, eps)


def add_rms_norm_separate(x, delta, weight, eps):
    """The reference's two-kernel form (norm.py:141-144: a bf16 residual add, then ``rms_norm``
    of it, chosen there for short decode matrices). Both steps round exactly as the fused kernel
    does, so the one launch of ``add_rms_norm`` gives the same bits for a launch fewer: on MI355X
    the fused kernel is the faster one at every row count (one workgroup per row, every load
    issued before any is used)."""
    return _add_norm(x, delta, None, weight, eps)


def add_rms_norm_partials_separate(x, partials, weight, eps):
    """The reference's sequential form (norm.py:147-154: the fp32 planes summed in slice order,
    the bf16 casts of the projection and the residual, then ``rms_norm``): the same roundings in
    the same order as ``add_rms_norm_partials``, which does them in one launch."""
    return _add_norm(x, None, partials, weight, eps)
