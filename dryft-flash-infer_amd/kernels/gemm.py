"""Per-shape choice of the decode linear kernel (engine/kernels/gemm.py:134-261).

``pick_matmul`` races the incumbent, torch's ``F.linear`` on the bf16 weight (hipBLASLt on
ROCm), against the gfx950 8-/4-bit kernels of ``cuda_fp8`` over every config of the
reference's race list, under the reference's rules:

* a candidate must first agree with ``F.linear`` on one layer's weight, max-abs over
  max-ref below 0.08 for 8-bit and 0.3 for 4-bit weights (gemm.py:181-198);
* it is timed with ``timing.time_calls`` over every layer's weight, in a HIP graph;
* it replaces the incumbent only if it is faster by more than 3 % (gemm.py:248-250).

The reference also races Triton and CUDA bf16 GEMV families; they do not exist on this
build (no Triton, and the bf16 path is hipBLASLt's), so ``family="bf16"`` keeps the
incumbent. The returned ``fn`` is ``functools.partial(cuda_fp8.matmul, config=cfg)`` for the
8-bit family, as the engine expects (it reads ``fn.keywords["config"]``).
"""

import functools

import torch
import torch.nn.functional as F

from .timing import time_calls


def pick_matmul(batch: int, every, reps: int = 3, trials: int = 3, packed=None,
                use_graph=True, family=None, quick=False):
    """Choose how to run this projection shape during decode.

    ``every``: the bf16 weight [out, in] of every layer; ``packed``: the matching
    ``cuda_fp8.Prepared`` operands, or None. ``family``: "bf16" keeps the incumbent, "fp8"
    races the 8-bit kernels only, None races both. ``quick`` tries one config only.
    Returns ``(fn, transpose, note)``: call ``fn(x, w)`` (``transpose`` is False for
    ``F.linear``, "fp8" for the quantized kernels, whose ``w`` is the Prepared operand).
    """
    weight = every[0]
    device, dtype = weight.device, weight.dtype
    x = torch.randn(batch, weight.shape[1], dtype=dtype, device=device)
    reference = F.linear(x, weight)
    scale = reference.float().abs().max().item() or 1.0
    moved = weight.numel() * weight.element_size()

    def clock(fn, operands):
        return time_calls(lambda w: fn(x, w), operands, reps=reps, trials=trials, use_graph=use_graph)

    def agrees(out, tolerance=0.02):
        return (out.float() - reference.float()).abs().max().item() / scale < tolerance

    incumbent = clock(F.linear, every)
    best = (F.linear, False, incumbent)
    if family == "fp8":
        if packed is None:
            raise ValueError("an FP8-only race needs FP8 operands")
        best = (None, None, float("inf"))

    if packed is not None and family != "bf16":
        from . import cuda_fp8

        if cuda_fp8.ready():
            for cfg in (cuda_fp8.CONFIGS[:1] if quick else cuda_fp8.CONFIGS):
                if not cuda_fp8.applicable(cfg, batch):
                    continue
                runner = functools.partial(cuda_fp8.matmul, config=cfg)
                try:
                    if not agrees(runner(x, packed[0]), tolerance=0.08 if packed[0].bits == 8 else 0.3):
                        continue
                except Exception:  # the reference treats any failure as "candidate unavailable"
                    continue
                elapsed = clock(runner, packed)
                if elapsed < best[2]:
                    best = (runner, "fp8", elapsed)

    fn, transpose, elapsed = best
    if fn is None:
        raise RuntimeError("no FP8 kernel passed for this shape")
    if family != "fp8" and fn is not F.linear and elapsed > incumbent * 0.97:
        fn, transpose, elapsed = F.linear, False, incumbent
    if transpose == "fp8":
        real = packed[0].bytes_moved()
        return fn, "fp8", (f"fp8 {real / (elapsed * 1e-3) / 1e12:.2f} TB/s"
                           f" ({moved / (elapsed * 1e-3) / 1e12:.2f} effective)")
    return fn, transpose, f"hipblaslt {moved / (elapsed * 1e-3) / 1e12:.2f} TB/s"
