"""Drop-in for the reference's ``kernels.cuda_fp8`` on MI355X (gfx950).

Same names, signatures, weight formats and error behaviour as
engine/kernels/cuda_fp8.py: INT8 (or INT4) weights with one fp16 scale per 64 values,
stored offset by 128 (8) as bytes; ``prepare`` relays them into the reference's own
layouts -- the fragment-permuted row-major form or the 16-row x 128-byte tiles -- byte
for byte, and the MI355X GEMM consumes those layouts directly (bf16 MFMA, the group
scale applied to the fp32 partial of each 64-block, split-K planes summed in slice
order). Quantize, relayout, GEMM and the reduce all run in ``libqlinear.so``; there is
no CPU path, so every function needs GPU tensors.

A ``config`` is the reference's race entry ``(warps, splitk[, stage, nshare, ring])``.
``splitk`` keeps its meaning (K slices, reduced in slice order); the other fields pick
NVIDIA kernel variants and have no MI355X counterpart: the library plans the workgroup
shape itself (``qlx_plan_linear``).

The same signatures also carry the MI355X north-star formats, so an engine that calls
``prepare(quantize(w, bits=bits))`` and then ``matmul`` / ``matmul_partials`` /
``gate_up_swiglu`` / ``matmul_add_norm`` reaches them without changing a call site:

* ``quantize(..., fmt=...)`` or the module default ``FORMAT`` (environment variable
  ``QLX_WEIGHT_FORMAT``) selects ``"ref"`` (the reference's format, the default),
  ``"w8a16"`` (int8 per output channel, bf16 scales), ``"w4a16"`` (int4 group 128, bf16
  scales, eight codes per int32 along K), ``"fp8"`` (e4m3 per output channel with the
  activation quantized per token: FP8 W8A8), or ``"auto"`` (w8a16 for 8 bits, w4a16 for 4);
* ``prepare`` then relays the codes into the MI355X tile layout and returns a
  ``FormatPrepared`` with the attributes the engine reads (``bits``, ``k``, ``rows``,
  ``bytes_moved()``);
* the linears dispatch on it: ``matmul``/``gate_up_swiglu`` take the library's planned
  path for the batch (decode kernel, skinny GEMM from 9 tokens, FP8 activation quantized
  once from 2 tokens), ``matmul_partials``/``splits`` honour the config's split-K.
"""

import os

import torch

from . import _lib, _linear

#: Weight layout selected by ``prepare`` when ``tiled`` is None (engine/kernels/cuda_fp8.py:42-44).
TILED = True
#: Weight format ``quantize`` produces when the call names none (see the module docstring).
FORMAT = os.environ.get("QLX_WEIGHT_FORMAT", "ref")
FORMATS = ("ref", "w8a16", "w4a16", "fp8", "auto")
#: Values per scale (engine/kernels/cuda_fp8.py:57).
GROUP = 64
_FUSED_ROWS = 2560   # the hidden width; matmul_add_norm normalises rows of this length
RING_DEPTH = 2

# The reference's race lists (engine/kernels/cuda_fp8.py:1404-1423), kept as selectors.
_BASE = [(8, 1), (8, 2), (8, 4), (4, 4), (4, 8), (4, 16)]
_RING_BASE = [(8, 2), (8, 4), (8, 16), (4, 4), (4, 8)]
CONFIGS = [(w, k, 1, 1, 0) for w, k in _BASE] + [(w, k, 1, 1, RING_DEPTH) for w, k in _RING_BASE]
SWIGLU_CONFIGS = [(w, 1, 1, 1, r) for r in (0, RING_DEPTH) for w in (4, 8)]
ADD_NORM_CONFIGS = (4, 8)

_ready = None


def ready() -> bool:
    """Whether the gfx950 library loads. False (with a message) instead of raising."""
    global _ready
    if _ready is None:
        try:
            _lib.lib()
            _ready = True
        except Exception as exc:  # the reference prints and returns False (cuda_fp8.py:1104-1114)
            print(f"cuda_fp8: unavailable ({type(exc).__name__}: {exc})"[:400])
            _ready = False
    return _ready


def _permutation(device) -> torch.Tensor:
    """Natural column index held at each permuted position of a 64-wide block."""
    order = [16 * s + 2 * t + u for t in range(4) for s in range(4) for u in (0, 1, 8, 9)]
    return torch.tensor(order, dtype=torch.int64, device=device)


def _resolve(fmt, bits):
    fmt = FORMAT if fmt is None else fmt
    if fmt not in FORMATS:
        raise ValueError(f"unknown weight format {fmt!r} (one of {FORMATS})")
    if fmt == "auto":
        fmt = "w4a16" if bits == 4 else "w8a16"
    if fmt != "ref" and bits != (4 if fmt == "w4a16" else 8):
        raise ValueError(f"format {fmt} stores {4 if fmt == 'w4a16' else 8}-bit codes, not {bits}")
    return fmt


def quantize(weight: torch.Tensor, group: int = GROUP, bits: int = 8, *, fmt=None):
    """``[out, in]`` bfloat16 -> offset bytes ``[out, in]`` plus ``[out, in/group]`` fp16 scales.

    Symmetric absmax with the fp16 scale nudged up one fp16 ulp (cuda_fp8.py:1127-1151);
    bits 8 stores -127..127 offset by 128, bits 4 stores -7..7 offset by 8, one per byte.
    Returns ``(bytes, scales, bits)``.

    With a north-star ``fmt`` (or ``FORMAT``) the result is ``(codes, scales, bits, fmt)`` in
    that format (``qlinear.quantize_w8/w4/fp8``); ``group`` must then be the default or the
    format's own (128 for w4a16, K for the per-channel formats).
    """
    if bits not in (8, 4):
        raise ValueError("weights are 8 or 4 bits")
    if weight.dim() != 2 or weight.dtype != torch.bfloat16:
        raise ValueError("weight must be a 2-D bfloat16 tensor")
    fmt = _resolve(fmt, bits)
    if fmt != "ref":
        from . import qlinear
        own = 128 if fmt == "w4a16" else weight.shape[1]
        if group not in (GROUP, own):
            raise ValueError(f"format {fmt} uses group {own}, not {group}")
        q, s = qlinear.FORMATS[fmt][0](weight)
        return q, s, bits, fmt
    out, inner = weight.shape
    if inner % group:
        raise ValueError(f"{inner} is not a multiple of {group}")
    _lib.require_device(weight)
    q = torch.empty((out, inner), dtype=torch.uint8, device=weight.device)
    s = torch.empty((out, inner // group), dtype=torch.float16, device=weight.device)
    _lib.call("qlx_quantize_weight", _lib.ptr(weight), _lib.ptr(q), _lib.ptr(s), out, inner, group, bits,
              _lib.SCALE_F16, 1, _lib.STORE_OFFSET, _lib.stream(weight.device))
    return q, s, bits


def dequantize(packed) -> torch.Tensor:
    """The bfloat16 weight the kernel effectively multiplies by: bf16((byte - offset) * scale)."""
    if len(packed) > 3 and packed[3] != "ref":
        from . import qlinear
        return qlinear.dequantize(packed[:2], packed[3])
    weight, scale = packed[0], packed[1]
    bits = packed[2] if len(packed) > 2 else 8
    rows, k = weight.shape
    _lib.require_device(weight, scale)
    out = torch.empty((rows, k), dtype=torch.bfloat16, device=weight.device)
    _lib.call("qlx_dequantize", _lib.ptr(weight), _lib.ptr(scale.to(torch.float16).contiguous()), _lib.ptr(out),
              rows, k, scale.shape[1], bits, _lib.SCALE_F16, _lib.STORE_OFFSET, _lib.stream(weight.device))
    return out


class Prepared:
    """An offset INT8/INT4 weight in the reference's layout plus fp16 block scales.

    ``tiled`` stores the weight as ``[rows/16][K/128][half][j][g][t][16 B]`` (8 bits) or
    ``[rows/16][K/128][half][g][t][16 B]`` with block j in nibble j (4 bits); otherwise
    8-bit weights are row-major with each 64-block's columns permuted
    (engine/kernels/cuda_fp8.py:1164-1217).
    """

    __slots__ = ("weight", "scale", "rows", "k", "groups", "tiled", "bits")
    fmt = "ref"

    def __init__(self, packed: torch.Tensor, scale: torch.Tensor, tiled: bool = None, bits: int = 8):
        rows, k = packed.shape
        if k % 128:
            raise ValueError(f"K={k} is not a multiple of 128")
        if rows % 16:
            raise ValueError(f"rows={rows} is not a multiple of 16")
        if tuple(scale.shape) != (rows, k // GROUP):
            raise ValueError("scales do not match a 64-wide blocking")
        self.tiled = TILED if tiled is None else tiled
        self.bits = bits
        if bits == 4 and not self.tiled:
            raise ValueError("4-bit weights are stored tiled")
        _lib.require_device(packed, scale)
        width = k // 2 if bits == 4 else k
        self.weight = torch.empty((rows, width), dtype=torch.uint8, device=packed.device)
        _lib.call("qlx_prepare_ref", _lib.ptr(packed.view(torch.uint8).contiguous()), _lib.ptr(self.weight),
                  rows, k, bits, int(self.tiled), _lib.stream(packed.device))
        self.scale = scale.to(torch.float16).contiguous()
        self.rows, self.k = rows, k
        self.groups = k // 128

    def row_major(self) -> torch.Tensor:
        """The fragment-permuted ``[rows, K]`` weight regardless of storage layout."""
        if self.bits != 8:
            raise ValueError("4-bit weights have no 8-bit row-major form")
        if not self.tiled:
            return self.weight
        out = torch.empty_like(self.weight)
        _lib.call("qlx_row_major_ref", _lib.ptr(self.weight), _lib.ptr(out), self.rows, self.k,
                  _lib.stream(self.weight.device))
        return out

    def bytes_moved(self) -> int:
        return self.weight.numel() + self.scale.numel() * 2


class FormatPrepared(Prepared):
    """A north-star weight (``quantize(..., fmt=...)``) relaid into the MI355X tile layout.

    Carries the attributes the engine reads from ``Prepared`` (``weight``, ``scale``,
    ``rows``, ``k``, ``groups``, ``tiled``, ``bits``, ``bytes_moved()``) plus ``fmt`` and
    ``tiles``, the ``qlinear.Tiled`` weight the linears consume."""

    __slots__ = ("fmt", "tiles")

    def __init__(self, codes, scale, bits, fmt):  # noqa: super().__init__ relays the reference format
        from . import qlinear
        self.tiles = qlinear.prepare((codes, scale), fmt)
        self.fmt = fmt
        self.weight, self.scale = self.tiles.weight, self.tiles.scale
        self.rows, self.k = self.tiles.rows, self.tiles.k
        self.groups = self.k // 128
        self.tiled = True
        self.bits = bits

    def row_major(self):
        raise ValueError(f"row_major() serves the reference's 8-bit format, not {self.fmt}")

    def bytes_moved(self) -> int:
        return self.tiles.bytes_moved()


def prepare(packed, tiled: bool = None) -> Prepared:
    """``packed`` is ``(uint8 weight, fp16 scales[, bits])`` from ``quantize``, or a
    north-star ``(codes, scales, bits, fmt)``."""
    weight, scale = packed[0], packed[1]
    bits = packed[2] if len(packed) > 2 else 8
    if len(packed) > 3 and packed[3] != "ref":
        if tiled is False:
            raise ValueError(f"{packed[3]} weights are consumed in the MI355X tile layout")
        return FormatPrepared(weight, scale, bits, packed[3])
    return Prepared(weight, scale, tiled, bits)


def _splitk(prepared, config):
    splitk = config[1]
    if splitk == "pairs":
        splitk = -(-prepared.groups // 2)
    return max(1, min(int(splitk), prepared.groups))


def _plan_config(prepared, batch, config, mode):
    """The reference config's split-K on the library's planned workgroup shape."""
    if batch > 64:
        raise ValueError(f"batch {batch} exceeds 64 rows")
    base = _linear.make_plan(_fmt(prepared), mode, batch, prepared.rows, prepared.k)
    splitk = 1 if mode == _lib.MODE_SWIGLU else _splitk(prepared, config)
    return (base.waves, base.kw, base.rw, splitk)


_LIB_FMT = {"w8a16": _lib.FMT_W8A16, "w4a16": _lib.FMT_W4A16, "fp8": _lib.FMT_FP8}


def _fmt(prepared):
    if prepared.fmt != "ref":
        return _LIB_FMT[prepared.fmt]
    return _lib.FMT_REF8 if prepared.bits == 8 else _lib.FMT_REF4


def _run(x, prepared, config, mode):
    batch, k = x.shape
    if k != prepared.k:
        raise ValueError("activation width does not match the weight")
    if x.dtype != torch.bfloat16:
        raise ValueError("activation must be bfloat16")
    _lib.require_device(x, prepared.weight)
    if prepared.fmt != "ref":
        from . import qlinear
        linear = qlinear.FORMATS[prepared.fmt][1]
        if mode == _lib.MODE_PLANES:
            return linear(x, prepared.tiles, config=_plan_config(prepared, batch, config, mode), planes=True)
        return linear(x, prepared.tiles, swiglu=mode == _lib.MODE_SWIGLU)
    cfg = _plan_config(prepared, batch, config, mode)
    return _linear.run(_fmt(prepared), "qlx_linear_ref", x, prepared.rows, prepared.k,
                       (_lib.ptr(prepared.weight), _lib.ptr(prepared.scale), _lib.ptr(x)),
                       (prepared.bits, int(prepared.tiled)), mode=mode, config=cfg, fit=True)


def splits(prepared: Prepared, batch: int, config=(4, 1)) -> int:
    """How many fp32 planes ``matmul_partials`` returns for this shape and config."""
    cfg = _plan_config(prepared, batch, config, _lib.MODE_PLANES)
    return _linear.splits_for(_fmt(prepared), _lib.MODE_PLANES, batch, prepared.rows, prepared.k, cfg, fit=True)


def matmul_partials(x: torch.Tensor, prepared: Prepared, config=(4, 1)) -> torch.Tensor:
    """``x @ W.T`` as fp32 split-K planes ``[splits, B, N]``; sum them to finish."""
    return _run(x, prepared, config, _lib.MODE_PLANES)


def matmul(x: torch.Tensor, prepared: Prepared, config=(4, 1)) -> torch.Tensor:
    """``x @ W.T`` in bfloat16, ``x`` of shape ``[B, K]`` with ``B <= 64``."""
    return _run(x, prepared, config, _lib.MODE_BF16)


def gate_up_swiglu(x: torch.Tensor, prepared: Prepared, config=(4, 1)) -> torch.Tensor:
    """``silu(gate) * up`` from a fused ``[gate; up]`` weight, never writing 2*I.

    Gate row i pairs with up row I + i; the result is bf16(bf16(silu(bf16 g)) * bf16 u)
    (engine/kernels/cuda_fp8.py:483-499). As in the reference the config's split-K is not
    used (cuda_fp8.py:1389); a batch too wide for one slice is split and reduced in order.
    """
    return _run(x, prepared, config, _lib.MODE_SWIGLU)


def add_norm_scratch(batch: int, rows: int, device):
    """The delta buffer and ticket counter ``matmul_add_norm`` takes, per call site."""
    return (torch.empty((batch, rows), dtype=torch.bfloat16, device=device),
            torch.zeros(1, dtype=torch.int32, device=device))


def matmul_add_norm(x: torch.Tensor, prepared: Prepared, residual: torch.Tensor,
                    norm_weight: torch.Tensor, eps: float, scratch, warps: int = 8):
    """``residual + x @ W.T`` in bfloat16 and its RMSNorm, in one launch: returns
    ``(new_residual, normed)``.

    Delta = bf16(x @ W.T) lands in ``scratch``'s buffer; the workgroup that completes the
    last row block (``scratch``'s counter) then forms r = bf16(residual + delta) and
    y = bf16(bf16(r * rsqrt(mean r^2 + eps)) * w) for every row, the rounding of
    engine/kernels/cuda_fp8.py:1339-1374 (``qlx_linear_add_norm``). ``warps`` is the
    reference's block shape and has no MI355X counterpart (the library plans the launch).
    """
    batch, k = x.shape
    n = prepared.rows
    if k != prepared.k or n % 16 or n != _FUSED_ROWS:
        raise ValueError("the fused add-norm serves the hidden-width projections")
    if tuple(residual.shape) != (batch, n) or residual.dtype != torch.bfloat16:
        raise ValueError("residual must be bfloat16 [batch, rows]")
    if batch > 16:
        raise ValueError("the fused add-norm serves up to sixteen rows")
    if x.dtype != torch.bfloat16:
        raise ValueError("activation must be bfloat16")
    delta, counter = scratch
    if tuple(delta.shape) != (batch, n) or delta.dtype != torch.bfloat16:
        raise ValueError("scratch does not match this batch")
    if counter.dtype != torch.int32 or counter.numel() < 1:
        raise ValueError("scratch's counter is one int32")
    _lib.require_device(x, residual, norm_weight, delta, counter, prepared.weight)
    return _linear.run_add_norm(_fmt(prepared), (prepared.weight, prepared.scale), x, n, k, prepared.tiled,
                                residual, norm_weight, eps, delta, counter)


def applicable(config, batch: int, swiglu: bool = False) -> bool:
    """Whether a config is worth racing for this batch: sharing needs tiles to split."""
    nshare = config[3] if len(config) > 3 else 1
    if swiglu and config[1] != 1:
        return False
    return nshare == 1 or -(-batch // 8) >= nshare


class _ReduceModule:
    """``_module_for(...).kernel("reduce_partials")`` compatibility: the plane reduce."""

    def kernel(self, name):
        if name != "reduce_partials":
            raise KeyError(name)

        def launch(grid, block, planes, out, width, splits):
            _lib.call("qlx_reduce_planes", _lib.ptr(planes), _lib.ptr(out), int(width), int(splits),
                      _lib.stream(out.device))
        return launch


def _module_for(nt: int = 1, nshare: int = 1, tiled: bool = None, bits: int = 8):
    return _ReduceModule()
