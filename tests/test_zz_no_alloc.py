"""qlx_linear_skinny_noalloc (the skinny GEMM whose planes and tickets live in the library's
static device array) against qlx_linear_skinny with caller-allocated workspace, through the
C ABI: bit-identical outputs on two calls in a row, the second smaller, for W4A16 and W8A16,
bf16 and SwiGLU outputs, with tickets (<= 32 tokens) and the planes launch (33-64 tokens);
and the size limit rejected before any launch."""

import ctypes

import pytest
import torch

from kernels import _lib, qlinear

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def noalloc(fmt, tiles, x, swiglu=False):
    m, k = x.shape
    n = tiles.rows
    y = torch.empty((m, n // 2 if swiglu else n), dtype=torch.bfloat16, device=DEV)
    lib_fmt = _lib.FMT_W4A16 if fmt == "w4a16" else _lib.FMT_W8A16
    _lib.call("qlx_linear_skinny_noalloc", lib_fmt, _lib.ptr(tiles.weight), _lib.ptr(tiles.scale), _lib.ptr(x),
              _lib.ptr(y), m, n, k, _lib.MODE_SWIGLU if swiglu else _lib.MODE_BF16, _lib.stream(x.device))
    return y


@pytest.mark.parametrize("fmt", ["w4a16", "w8a16"])
def test_noalloc_matches_the_allocating_entry_point(fmt):
    g = torch.Generator(device=DEV).manual_seed(77)
    quant = qlinear.FORMATS[fmt][0]
    # (n, k, m, swiglu): down-shaped K slices at 64 then 16 tokens, then a smaller projection
    cases = [(2560, 9728, 64, False), (2560, 9728, 16, False), (1024, 2560, 9, True), (512, 2048, 40, False)]
    tiles = {}
    for n, k, m, swiglu in cases:
        key = (n, k)
        if key not in tiles:
            w = (torch.randn(n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
            tiles[key] = qlinear.prepare(quant(w), fmt)
        x = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16)
        print(f"noalloc {fmt} n={n} k={k} m={m} swiglu={swiglu}", flush=True)
        want = qlinear._skinny(_lib.FMT_W4A16 if fmt == "w4a16" else _lib.FMT_W8A16, tiles[key].weight,
                               tiles[key].scale, x, n, k, swiglu)
        got = noalloc(fmt, tiles[key], x, swiglu)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (fmt, n, k, m, swiglu)


def test_noalloc_rejects_rows_past_its_tickets():
    """Rejected on the host before any launch (the pointers are never dereferenced). The
    planner's K slices keep planes under ~4 MB (about 240 workgroups x m x 16 rows x 4 bytes),
    so the 8 MiB plane limit is not reachable through qlx_plan_skinny; the row limit is."""
    lib = _lib.lib()
    p = ctypes.c_void_p(1 << 20)
    rc = lib.qlx_linear_skinny_noalloc(_lib.FMT_W4A16, p, p, p, p, 16, 16 * 16385, 256, _lib.MODE_BF16, None)
    assert rc == _lib.QLX_EINVAL and "exceeds" in _lib.last_error()
    # FP8 has its own skinny entry point: rejected before the shared array is cleared
    rc = lib.qlx_linear_skinny_noalloc(_lib.FMT_FP8, p, p, p, p, 16, 2560, 2560, _lib.MODE_BF16, None)
    assert rc == _lib.QLX_EINVAL and "serves W4A16 and W8A16" in _lib.last_error()
