"""MI355X (gfx950) quantized decode linear layers behind the reference's operator API.

Mirrors the module surface of the reference's ``engine/kernels`` package for the
quantized linear path (engine/kernels/__init__.py:11-75): ``cuda_fp8``, ``fp8``,
``cuda_int8``, ``cuda_small``, ``swiglu``, ``norm``, ``gemm`` (the per-shape race) and
``timing``, ``rope`` (QKV head norm + RoPE + cache write) and ``attention``
(``DecodeAttention``) keep their names and signatures; ``qlinear`` adds the north-star
formats and ``decode_stack`` the one-launch decode-step executor. Every op runs in the hand-written HIP
library ``libqlinear.so``; there is no CPU or Triton fallback, and ops raise if the
library is missing or the tensors are not on the GPU.
"""

from . import _lib, attention, cuda_fp8, cuda_int8, cuda_small, decode_tuning, fp8, gemm, norm, qlinear, rope, swiglu, timing  # noqa: F401
from .attention import DecodeAttention  # noqa: F401
from .rope import (  # noqa: F401
    kv_norm_rope_to_cache, q_norm_rope, qkv_norm_rope_to_cache, qkv_planes_norm_rope_to_cache,
)
from .norm import (  # noqa: F401
    add_rms_norm, add_rms_norm_partials, add_rms_norm_partials_separate, add_rms_norm_separate, rms_norm,
)
# As in the reference, the package attribute ``swiglu`` is the function (the module stays
# importable as ``kernels.swiglu`` through sys.modules).
from .swiglu import swiglu, swiglu_partials  # noqa: F401,E402

HAVE_TRITON = False  # the reference's flag (kernels/__init__.py:13): these ops never use Triton

__all__ = [
    "HAVE_TRITON", "cuda_fp8", "fp8", "cuda_int8", "cuda_small", "qlinear", "norm", "swiglu", "gemm", "timing",
    "add_rms_norm", "add_rms_norm_partials", "add_rms_norm_separate", "add_rms_norm_partials_separate",
    "rms_norm", "swiglu_partials", "DecodeAttention", "attention", "rope",
    "kv_norm_rope_to_cache", "q_norm_rope", "qkv_norm_rope_to_cache", "qkv_planes_norm_rope_to_cache",
]
