"""MI355X (gfx950) quantized decode linear layers behind the reference's operator API.

Mirrors the module surface of the reference's ``engine/kernels`` package for the
quantized linear path (engine/kernels/__init__.py:11-75): ``cuda_fp8``, ``fp8``,
``cuda_int8``, ``cuda_small``, ``swiglu`` and ``norm`` keep their names and signatures,
and ``qlinear`` adds the north-star formats. Every op runs in the hand-written HIP
library ``libqlinear.so``; there is no CPU or Triton fallback.
"""

from . import _lib, qlinear  # noqa: F401

__all__ = ["qlinear"]
