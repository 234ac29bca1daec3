"""Per-shape choice of the decode linear on MI355X.

``pick_matmul(batch, every, reps=3, trials=3, packed=None, use_graph=True, family=None,
quick=False) -> (fn, transpose, note)`` keeps the contract of
engine/kernels/gemm.py:134-261, which the engine consumes (engine/engine.py:540-634):

* a candidate counts only if it agrees with ``F.linear(x, W)`` on one layer's bf16 weight:
  max |difference| / max |reference| below 0.08 for 8-bit weights, 0.3 for 4-bit ones;
* a quantized winner replaces the incumbent (``F.linear``, hipBLASLt on ROCm) only if it
  is more than 3 % faster, unless ``family == "fp8"`` (quantized kernels only);
* ``transpose`` is False for ``F.linear`` on ``every`` and ``"fp8"`` for the quantized
  kernels, whose operand is ``packed[i]``; for the reference's format ``fn`` is
  ``functools.partial(cuda_fp8.matmul, config=cfg)`` (the engine reads
  ``fn.keywords["config"]`` to route split-K planes).

What is raced is this build's own set of paths for the operand's format, each timed over
a cache-defeating rotation (``timing.time_calls``):

* the reference's format (``cuda_fp8.Prepared``): the distinct MI355X plans its configs
  resolve to -- only split-K survives the mapping, so configs that resolve to one plan
  are timed once;
* the north-star formats (``cuda_fp8.FormatPrepared`` or ``qlinear.Tiled``): the library's
  default path for the batch (decode kernel to 8 tokens, skinny GEMM from 9, FP8
  activation quantized once from 2 tokens), the decode kernel at twice and four times its
  planned split-K, the skinny GEMM at any batch (W8A16/W4A16), and for FP8 both
  placements of the activation quantization.
"""

import dataclasses
import functools
import math

import torch
import torch.nn.functional as F

from . import _lib, _linear
from .timing import time_calls

#: Agreement bounds of the contract, by weight bits.
TOLERANCE = {8: 0.08, 4: 0.3}
#: A quantized kernel must beat the incumbent by this factor to replace it.
MARGIN = 0.97


@dataclasses.dataclass
class Candidate:
    label: str
    fn: object         # fn(x, operand)
    operands: list     # one operand per layer
    transpose: object  # False: F.linear on the bf16 weight; "fp8": a quantized operand
    bits: int = 16


def north_matmul(x, operand, *, config=None, skinny=None, pre_quantize=None):
    """``x @ W^T`` for a north-star operand (``cuda_fp8.FormatPrepared`` or ``qlinear.Tiled``)
    on one chosen path: ``config`` a ``(waves, kw, rw, splits)`` plan of the decode kernel,
    ``skinny`` the skinny GEMM, ``pre_quantize`` the FP8 activation's quantization placement."""
    from . import qlinear
    tiles = getattr(operand, "tiles", operand)
    kwargs = {"config": config}
    if tiles.fmt == "fp8":
        kwargs["pre_quantize"] = pre_quantize
    else:
        kwargs["skinny"] = skinny
    return qlinear.FORMATS[tiles.fmt][1](x, tiles, **kwargs)


def _reference_candidates(batch, packed, quick):
    from . import cuda_fp8
    if not cuda_fp8.ready():
        return
    resolved = set()
    for cfg in cuda_fp8.CONFIGS:
        if not cuda_fp8.applicable(cfg, batch):
            continue
        try:
            plan = cuda_fp8._plan_config(packed[0], batch, cfg, _lib.MODE_BF16)
        except ValueError:
            continue
        if plan in resolved:
            continue
        resolved.add(plan)
        yield Candidate(f"cuda_fp8 {cfg}", functools.partial(cuda_fp8.matmul, config=cfg), packed, "fp8",
                        packed[0].bits)
        if quick:
            return


def _north_candidates(batch, packed, quick):
    tiles = getattr(packed[0], "tiles", packed[0])
    fmt = tiles.fmt
    bits = 4 if fmt == "w4a16" else 8
    variants = [("default", {})]
    if not quick:
        lib_fmt = {"w8a16": _lib.FMT_W8A16, "w4a16": _lib.FMT_W4A16, "fp8": _lib.FMT_FP8}[fmt]
        plan = _linear.make_plan(lib_fmt, _lib.MODE_BF16, batch, tiles.rows, tiles.k)
        steps = tiles.k // (256 if fmt == "w4a16" else 128)
        for mul in (2, 4):
            if plan.splits * mul <= steps:
                variants.append((f"decode split-K {plan.splits * mul}",
                                 {"config": (plan.waves, plan.kw, plan.rw, plan.splits * mul), "skinny": False}))
        if fmt == "fp8":
            variants += [("activation quantized in the GEMM", {"pre_quantize": False}),
                         ("activation quantized once", {"pre_quantize": True})]
        else:
            variants += [("decode kernel", {"skinny": False}), ("skinny GEMM", {"skinny": True})]
    for label, kwargs in variants:
        if fmt == "fp8":
            kwargs.pop("skinny", None)
        yield Candidate(f"{fmt} {label}", functools.partial(north_matmul, **kwargs), packed, "fp8", bits)


def _candidates(batch, every, packed, family, quick):
    if family != "fp8":
        yield Candidate("hipblaslt", F.linear, every, False)
    if packed is None or family == "bf16":
        return
    if getattr(packed[0], "fmt", "ref") == "ref" and not hasattr(packed[0], "tiles"):
        yield from _reference_candidates(batch, packed, quick)
    else:
        yield from _north_candidates(batch, packed, quick)


@torch.no_grad()
def pick_matmul(batch: int, every, reps: int = 3, trials: int = 3, packed=None, use_graph=True, family=None,
                quick=False):
    """Choose how to run this projection shape during decode.

    ``every``: the bf16 weight ``[out, in]`` of every layer; ``packed``: the matching quantized
    operands (``cuda_fp8.prepare`` results or ``qlinear.Tiled``), or None. ``family``: "bf16"
    keeps the incumbent, "fp8" races the quantized kernels only, None races both; ``quick``
    races one quantized candidate. Returns ``(fn, transpose, note)``: call ``fn(x, w)`` with
    ``w`` from ``every`` (``transpose`` False) or from ``packed`` (``transpose`` "fp8")."""
    if family == "fp8" and packed is None:
        raise ValueError("an FP8-only race needs FP8 operands")
    weight = every[0]
    x = torch.randn(batch, weight.shape[1], dtype=weight.dtype, device=weight.device)
    want = F.linear(x, weight).float()
    peak = want.abs().max().item() or 1.0

    timed = []  # (milliseconds, candidate)
    incumbent = math.inf
    for cand in _candidates(batch, every, packed, family, quick):
        if cand.transpose == "fp8":
            try:
                got = cand.fn(x, cand.operands[0]).float()
            except (ValueError, RuntimeError):  # a path that does not take this shape
                continue
            if not (got - want).abs().max().item() / peak < TOLERANCE[cand.bits]:
                continue
        ms = time_calls(lambda op, fn=cand.fn: fn(x, op), cand.operands, reps=reps, trials=trials,
                        use_graph=use_graph)
        if cand.transpose is False:
            incumbent = ms
        timed.append((ms, cand))
    if not timed:
        raise RuntimeError("no FP8 kernel passed for this shape")
    ms, best = min(timed, key=lambda t: t[0])
    if best.transpose == "fp8" and family != "fp8" and ms > incumbent * MARGIN:
        ms, best = next(t for t in timed if t[1].transpose is False)
    bf16_bytes = weight.numel() * weight.element_size()
    if best.transpose is False:
        return best.fn, False, f"hipblaslt {bf16_bytes / (ms * 1e-3) / 1e12:.2f} TB/s"
    moved = best.operands[0].bytes_moved()
    return best.fn, "fp8", (f"{best.label} {moved / (ms * 1e-3) / 1e12:.2f} TB/s"
                            f" ({bf16_bytes / (ms * 1e-3) / 1e12:.2f} effective)")
