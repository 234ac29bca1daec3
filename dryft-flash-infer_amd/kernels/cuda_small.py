"""Drop-in for the reference's ``kernels.cuda_small`` (engine/kernels/cuda_small.py).

The small decode kernels between projections, with the reference's bf16 rounding
placement: split-K residual sum, RMSNorm and the split-K SwiGLU (cuda_small.py:43-110).
Planes are summed in slice order in fp32.
"""

import torch

from . import _lib

_ready = None


def ready() -> bool:
    global _ready
    if _ready is None:
        try:
            _lib.lib()
            _ready = True
        except Exception as exc:
            print(f"cuda_small: unavailable ({type(exc).__name__}: {exc})"[:300])
            _ready = False
    return _ready


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    rows, n = x.shape
    _lib.require_device(x, weight)
    out = torch.empty_like(x)
    _lib.call("qlx_add_rms_norm", _lib.ptr(x), None, None, 0, _lib.ptr(weight), None, _lib.ptr(out),
              rows, n, float(eps), _lib.stream(x.device))
    return out


def residual_partials(x: torch.Tensor, partials: torch.Tensor) -> torch.Tensor:
    """``bf16(x + bf16(sum of planes))`` for planes ``[splits, rows, n]``."""
    _lib.require_device(x, partials)
    residual = torch.empty_like(x)
    _lib.call("qlx_residual_planes", _lib.ptr(x), _lib.ptr(partials), _lib.ptr(residual), x.numel(),
              partials.shape[0], _lib.stream(x.device))
    return residual


def add_rms_norm_partials_separate(x, partials, weight, eps):
    residual = residual_partials(x, partials)
    return residual, rms_norm(residual, weight, eps)


def swiglu_partials(partials: torch.Tensor) -> torch.Tensor:
    from .swiglu import swiglu_partials as _sp
    return _sp(partials)
