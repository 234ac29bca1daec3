"""Drop-in for the reference's ``kernels.swiglu`` (engine/kernels/swiglu.py).

SwiGLU over a fused ``[gate | up]`` projection: bf16(bf16(silu(g)) * u), silu rounding to
bf16 before the product (swiglu.py:21-22); from fp32 split-K planes, gate and up are
summed in slice order and rounded to bf16 first (swiglu.py:49-53).
"""

import torch

from . import _lib


def swiglu(gate_up: torch.Tensor) -> torch.Tensor:
    """``[rows, 2 * inter]`` fused projection output to ``[rows, inter]``."""
    rows, width = gate_up.shape
    inter = width // 2
    _lib.require_device(gate_up)
    out = torch.empty((rows, inter), dtype=gate_up.dtype, device=gate_up.device)
    _lib.call("qlx_swiglu", _lib.ptr(gate_up), None, 0, _lib.ptr(out), rows, inter, _lib.stream(gate_up.device))
    return out


def swiglu_partials(partials: torch.Tensor) -> torch.Tensor:
    """Sequentially reduce FP32 [splits, rows, 2*I] planes and apply SwiGLU."""
    splits, rows, width = partials.shape
    inter = width // 2
    _lib.require_device(partials)
    out = torch.empty((rows, inter), device=partials.device, dtype=torch.bfloat16)
    _lib.call("qlx_swiglu", None, _lib.ptr(partials), splits, _lib.ptr(out), rows, inter,
              _lib.stream(partials.device))
    return out
