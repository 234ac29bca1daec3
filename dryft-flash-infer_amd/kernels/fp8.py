"""Drop-in for the reference's ``kernels.fp8`` (engine/kernels/fp8.py) on MI355X.

E4M3 weights with bf16 scales per ``group`` values along K, bf16 activations and outputs.
``quantize`` is bit-exact with the reference's (fp8.py:20-28); ``fp8_matmul`` runs the
gfx950 GEMM (e4m3 -> bf16 exactly, bf16 MFMA, the group scale applied to each 64-block's
fp32 partial, split-K reduced in slice order) instead of the reference's Triton kernels.
``fp8.quantize(w, group=K)`` is the per-output-channel weight of the FP8 W8A8 format.
"""

import torch

from . import _lib, _linear

#: One scale per this many input values (fp8.py:16).
GROUP = 128
_E4M3_MAX = 448.0

#: The reference's Triton race entries (BLOCK_N, num_warps, num_stages, k_splits)
#: (fp8.py:163-167); here only k_splits has a meaning.
CONFIGS = [
    (32, 4, 4, 1), (64, 8, 4, 1), (128, 8, 4, 1),
    (32, 4, 4, 2), (32, 4, 4, 4), (32, 4, 4, 8),
    (64, 8, 4, 2), (64, 8, 4, 4), (16, 4, 4, 4),
]


def quantize(weight: torch.Tensor, group: int = GROUP):
    """``[out, in]`` bfloat16 to E4M3 plus ``[out, in / group]`` bf16 scales."""
    if weight.dim() != 2 or weight.dtype != torch.bfloat16:
        raise ValueError("weight must be a 2-D bfloat16 tensor")
    out, inner = weight.shape
    if inner % group:
        raise ValueError(f"{inner} is not a multiple of {group}")
    if group % 8:
        raise ValueError(f"group {group} must be a multiple of 8")
    _lib.require_device(weight)
    q = torch.empty((out, inner), dtype=torch.uint8, device=weight.device)
    s = torch.empty((out, inner // group), dtype=torch.bfloat16, device=weight.device)
    _lib.call("qlx_quantize_fp8_weight", _lib.ptr(weight), _lib.ptr(q), _lib.ptr(s), out, inner, group,
              _lib.stream(weight.device))
    return q.view(torch.float8_e4m3fn), s


def fp8_matmul(x: torch.Tensor, packed, config=None) -> torch.Tensor:
    """``x @ weight.T`` where ``packed`` is ``(e4m3 weight, group scales)``."""
    weight, scale = packed
    batch, k = x.shape
    n = weight.shape[0]
    groups = scale.shape[1]
    group = k // groups
    if group * groups != k or weight.shape[1] != k:
        raise ValueError("quantization groups must cover K exactly")
    if x.dtype != torch.bfloat16:
        raise ValueError("activation must be bfloat16")
    if batch > 64:
        raise ValueError(f"batch {batch} exceeds 64 rows")
    _lib.require_device(x, weight, scale)
    cfg = None
    if config is not None:
        base = _linear.make_plan(_lib.FMT_FP8WO, _lib.MODE_BF16, batch, n, k)
        cfg = (base.waves, base.kw, base.rw, max(1, int(config[3])))
    return _linear.run(_lib.FMT_FP8WO, "qlx_linear_fp8wo", x, n, k,
                       (_lib.ptr(weight), _lib.ptr(scale.contiguous()), _lib.ptr(x)), (group,),
                       config=cfg, fit=True)


def bytes_moved(packed) -> int:
    weight, scale = packed
    return weight.numel() + scale.numel() * scale.element_size()
