"""Decode-step executor: a chain of quantized projections run by one cooperative launch.

The reference replays a captured graph of per-projection launches whose weight loads
overlap the previous kernel through programmatic dependent launch
(engine/kernels/cuda_fp8.py:47-50, 150-169; engine/kernels/cuda_jit.py:218-262). On MI355X
the chain runs inside one launch (``qlx_stack_run``): each workgroup issues its first
weight loads for the next projection before waiting for the previous one to finish.

    chain = DecodeStack("fp8", m=1)
    chain.add(tiled_qkv, x_hidden, y_qkv)
    chain.add(tiled_gate_up, x_normed, y_act, swiglu=True)
    chain.add(tiled_down, y_act, y_out)            # reads what gate_up wrote
    chain.build()
    chain.run()                                     # on torch.cuda.current_stream()

Inputs and outputs are caller-owned bf16 tensors that stay in place between runs (the
descriptors hold their addresses), like the static buffers of a captured decode graph.
"""

import ctypes

import torch

from . import _lib
from .qlinear import Tiled

_FMTS = {"w8a16": _lib.FMT_W8A16, "w4a16": _lib.FMT_W4A16, "fp8": _lib.FMT_FP8}

#: Sleeps (about 50 ns each) a workgroup waits for the previous projection before giving up
#: and flagging the run as failed; far above any real projection's time.
SPIN_LIMIT = 1 << 20


class DecodeStack:
    """An ordered chain of projections of one format, for m = 1..16 tokens."""

    def __init__(self, fmt, m, groups_per_cu=2):
        if fmt not in _FMTS:
            raise ValueError(f"the decode executor serves {sorted(_FMTS)}, not {fmt!r}")
        if not 1 <= m <= 16:
            raise ValueError(f"the decode executor serves m = 1..16 (got {m})")
        self.fmt, self.m, self.groups_per_cu = fmt, m, groups_per_cu
        self.calls, self._keep = [], []
        self.desc = None

    def add(self, weight, x, y, swiglu=False):
        """Append y = x @ W^T (or the SwiGLU of [gate; up] rows) to the chain."""
        if not isinstance(weight, Tiled) or weight.fmt != self.fmt:
            raise ValueError(f"the chain takes {self.fmt} weights in tile layout (qlinear.prepare)")
        _lib.require_device(weight.weight, weight.scale, x, y)
        out_n = weight.rows // 2 if swiglu else weight.rows
        if x.dtype != torch.bfloat16 or y.dtype != torch.bfloat16:
            raise ValueError("activations and outputs are bf16")
        if tuple(x.shape) != (self.m, weight.k) or tuple(y.shape) != (self.m, out_n):
            raise ValueError(f"x must be [{self.m}, {weight.k}] and y [{self.m}, {out_n}], got "
                             f"{tuple(x.shape)} and {tuple(y.shape)}")
        self.calls.append(_lib.StackCall(weight.weight.data_ptr(), weight.scale.data_ptr(), x.data_ptr(),
                                         y.data_ptr(), weight.rows, weight.k,
                                         _lib.MODE_SWIGLU if swiglu else _lib.MODE_BF16, 0))
        self._keep += [weight, x, y]
        self.desc = None
        return self

    def build(self):
        """Plan the chain and upload its descriptors (call after the last ``add``)."""
        if not self.calls:
            raise ValueError("empty chain")
        device = self._keep[0].weight.device
        lib = _lib.lib()
        arr = (_lib.StackCall * len(self.calls))(*self.calls)
        fmt = _FMTS[self.fmt]
        ws, tk = ctypes.c_longlong(0), ctypes.c_int(0)
        grid, lds = ctypes.c_int(0), ctypes.c_int(0)
        with torch.cuda.device(device):
            _lib.check(lib.qlx_stack_build(fmt, self.m, arr, len(self.calls), self.groups_per_cu, None, None, None,
                                           None, ws, tk, grid, lds), "qlx_stack_build")
            self.workspace = torch.empty(max(ws.value, 1), dtype=torch.float32, device=device)
            self.tickets = torch.zeros(max(tk.value, 1), dtype=torch.int32, device=device)
            self.sync = torch.zeros(4, dtype=torch.int32, device=device)
            size = lib.qlx_stack_desc_size()
            host = torch.empty(size * len(self.calls), dtype=torch.uint8)
            plans = (_lib.Plan * len(self.calls))()
            _lib.check(lib.qlx_stack_build(fmt, self.m, arr, len(self.calls), self.groups_per_cu,
                                           ctypes.c_void_p(host.data_ptr()), plans, _lib.ptr(self.workspace),
                                           _lib.ptr(self.tickets), ws, tk, grid, lds), "qlx_stack_build")
            self.desc = host.to(device)
        #: (waves, kw, rw, splits) per projection: qlinear's linears with this config give the same bits
        self.configs = [(p.waves, p.kw, p.rw, p.splits) for p in plans]
        self.grid, self.lds = grid.value, lds.value
        self.device = device
        return self

    def run(self, spin_limit=SPIN_LIMIT):
        """Run the whole chain once on the current stream."""
        if self.desc is None:
            self.build()
        _lib.call("qlx_stack_run", _FMTS[self.fmt], _lib.ptr(self.desc), len(self.calls), self.grid, self.lds,
                  _lib.ptr(self.sync), int(spin_limit), _lib.stream(self.device))

    def failed(self):
        """True if a wait of any run so far gave up (outputs of that run are undefined).
        Synchronizes with the device."""
        return bool(self.sync[2].item())

    def reset(self):
        """Clear the error flag and the split-K tickets (a run whose wait gave up may leave
        tickets counted; a normal run leaves everything zero)."""
        self.sync.zero_()
        self.tickets.zero_()

    def bytes_moved(self):
        return sum(w.bytes_moved() for w in self._keep[0::3])
