"""Write golden input/output vectors for the quantize and layout functions.

Run once, in the build container only (the reference is not present on the
GPU box and never travels there):

    python tests/golden/make_golden.py /root/reference

It imports the reference's pure-torch functions on the CPU and records what
they return for small seeded inputs, so the CPU oracle under ``oracle/`` can
be pinned byte-for-byte:

* ``kernels.cuda_fp8.quantize`` / ``dequantize`` (engine/kernels/cuda_fp8.py:1127-1161)
  for bits 8 and 4, group 64 and 128, including degenerate groups (all zero,
  tiny values whose fp16 scale underflows, large values);
* ``kernels.cuda_fp8._permutation`` and ``Prepared`` in its tiled and row-major
  8-bit layouts and its 4-bit nibble layout, plus ``Prepared.row_major``
  (engine/kernels/cuda_fp8.py:1117-1124, 1164-1224);
* ``kernels.fp8.quantize`` for group 128 and group K (engine/kernels/fp8.py:20-28);
* ``kernels.cuda_int8.Prepared`` (engine/kernels/cuda_int8.py:100-108).

The reference's own tests pin these only partly (tests/test_engine.py:431-490
checks two explicit index equalities, a round trip and value ranges); these
vectors pin every byte. Only data is written: bf16/fp16 as uint16 bit
patterns, e4m3 as uint8 bytes, all in ``.npz`` files read with
``allow_pickle=False``.
"""

import os
import sys

import numpy as np
import torch


def _bits16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def _weights(rows, k, seed):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(rows, k, generator=g) * 0.02).to(torch.bfloat16)
    w[0].zero_()                                               # all-zero groups
    w[1] = (torch.randn(k, generator=g) * 1e-9).to(torch.bfloat16)   # fp16 scale underflows
    w[2] = (torch.randn(k, generator=g) * 300.0).to(torch.bfloat16)  # large values
    w[3, : k // 2] = 0.0                                       # half-zero row
    w[4, 5] = 1.0                                              # a lone outlier
    return w


def main(ref_root):
    sys.path.insert(0, os.path.join(ref_root, "engine"))
    import importlib
    cuda_fp8 = importlib.import_module("kernels.cuda_fp8")
    fp8 = importlib.import_module("kernels.fp8")
    cuda_int8 = importlib.import_module("kernels.cuda_int8")

    here = os.path.dirname(os.path.abspath(__file__))
    out = {}
    out["permutation"] = cuda_fp8._permutation("cpu").numpy()
    for name, rows, k, seed in (("a", 32, 256, 1), ("b", 64, 256, 0), ("c", 16, 384, 7)):
        w = _weights(rows, k, seed)
        out[f"{name}_w"] = _bits16(w)
        for bits in (8, 4):
            for group in (64, 128):
                if k % group:
                    continue
                q, s, b = cuda_fp8.quantize(w, group=group, bits=bits)
                out[f"{name}_q{bits}_g{group}"] = q.numpy().copy()
                out[f"{name}_s{bits}_g{group}"] = _bits16(s)
                out[f"{name}_deq{bits}_g{group}"] = _bits16(cuda_fp8.dequantize((q, s, b)))
            q, s, b = cuda_fp8.quantize(w, bits=bits)
            if bits == 8:
                tiled = cuda_fp8.prepare((q, s, b), tiled=True)
                flat = cuda_fp8.prepare((q, s, b), tiled=False)
                out[f"{name}_prep8_tiled"] = tiled.weight.numpy().copy()
                out[f"{name}_prep8_rowmajor"] = flat.weight.numpy().copy()
                out[f"{name}_prep8_scale"] = _bits16(tiled.scale)
                assert torch.equal(tiled.row_major(), flat.weight)
                i8 = cuda_int8.Prepared(tiled)
                out[f"{name}_int8_prepared"] = i8.weight.numpy().copy()
            else:
                four = cuda_fp8.prepare((q, s, b), tiled=True)
                out[f"{name}_prep4_tiled"] = four.weight.numpy().copy()
        for group in (128, k):
            e, s = fp8.quantize(w, group=group)
            out[f"{name}_fp8_g{group}"] = e.view(torch.uint8).numpy().copy()
            out[f"{name}_fp8s_g{group}"] = _bits16(s)
    path = os.path.join(here, "reference_quant.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
