"""Decode-step executor: a chain of quantized projections run by one launch.

The reference replays a captured graph of per-projection launches whose weight loads
overlap the previous kernel through programmatic dependent launch
(engine/kernels/cuda_fp8.py:47-50, 150-169; engine/kernels/cuda_jit.py:218-262). On MI355X
the chain runs inside one launch (``qlx_stack_run``): workgroups stream each projection's
weights while its input is still being produced, and wait only for the words they need.

    chain = DecodeStack("fp8", m=1)
    chain.add(tiled_qkv, x_hidden, y_qkv)
    chain.add(tiled_gate_up, x_normed, y_act, swiglu=True)
    chain.add(tiled_down, y_act, y_out)            # reads what gate_up writes
    chain.build()
    chain.run()                                     # on torch.cuda.current_stream()

Inputs and outputs are caller-owned bf16 tensors that stay in place between runs (the
descriptors hold their addresses), like the static buffers of a captured decode graph. An
input is either memory no projection of the chain writes, or an earlier projection's output
tensor -- whole, or its first columns (``y_qkv[:, :4096]``, the attention's query part) -- or,
with ``add_normed``, a residual add + RMSNorm of them computed inside the same launch.
"""

import ctypes

import torch

from . import _lib
from .qlinear import Tiled

_FMTS = {"w8a16": _lib.FMT_W8A16, "w4a16": _lib.FMT_W4A16, "fp8": _lib.FMT_FP8}

#: Microseconds a run may wait in total before its waits give up and flag it as failed; far
#: above any real chain's time.
BUDGET_US = 2_000_000


class DecodeStack:
    """An ordered chain of projections of one format, for m = 1..16 tokens, run by workgroups
    of ``waves`` (4 or 8) waves, ``groups_per_cu`` of them per CU."""

    def __init__(self, fmt, m, waves=8, groups_per_cu=1):
        if fmt not in _FMTS:
            raise ValueError(f"the decode executor serves {sorted(_FMTS)}, not {fmt!r}")
        if not 1 <= m <= 16:
            raise ValueError(f"the decode executor serves m = 1..16 (got {m})")
        self.fmt, self.m, self.waves, self.groups_per_cu = fmt, m, waves, groups_per_cu
        self.calls, self._keep = [], []
        self.norms, self.attns = [], []
        self.desc = None

    def add(self, weight, x, y, swiglu=False, kw=0):
        """Append y = x @ W^T (or the SwiGLU of [gate; up] rows) to the chain. ``kw`` forces
        the waves per 16-row tile (1, 2, 4, 8; 0 lets the planner choose)."""
        if not isinstance(weight, Tiled) or weight.fmt != self.fmt:
            raise ValueError(f"the chain takes {self.fmt} weights in tile layout (qlinear.prepare)")
        _lib.require_device(weight.weight, weight.scale, y)
        if x.device.type != "cuda":
            raise ValueError("quantized linear ops need tensors on a ROCm GPU (no CPU path)")
        if not x.is_contiguous():  # only the first columns of an earlier output, rows n_out apart
            earlier = [t for t in self._keep[2::3] if t is not None and t.data_ptr() == x.data_ptr()]
            if not earlier or x.stride() != (earlier[0].shape[1], 1):
                raise ValueError("a strided input must be the first columns of an earlier output of the chain")
        out_n = weight.rows // 2 if swiglu else weight.rows
        if x.dtype != torch.bfloat16 or y.dtype != torch.bfloat16:
            raise ValueError("activations and outputs are bf16")
        if tuple(x.shape) != (self.m, weight.k) or tuple(y.shape) != (self.m, out_n):
            raise ValueError(f"x must be [{self.m}, {weight.k}] and y [{self.m}, {out_n}], got "
                             f"{tuple(x.shape)} and {tuple(y.shape)}")
        self.calls.append(_lib.StackCall(weight.weight.data_ptr(), weight.scale.data_ptr(), x.data_ptr(),
                                         y.data_ptr(), weight.rows, weight.k,
                                         _lib.MODE_SWIGLU if swiglu else _lib.MODE_BF16, int(kw)))
        self.norms.append(_lib.NormInput())
        self.attns.append(_lib.StackAttention())
        self._keep += [weight, x, y]
        self.desc = None
        return self

    def add_attention(self, qkv, n_q, n_kv, q_norm_w, k_norm_w, cos, sin, positions, k_cache, v_cache, out, eps,
                      splits=4, scale=None):
        """Append an attention stage for one token (m = 1, batch 1): the per-head RMSNorm + RoPE
        of ``qkv`` (the output tensor of an earlier projection: n_q query heads, n_kv key heads,
        n_kv value heads of 128 values) as ``qkv_norm_rope_to_cache`` does (rope.py:125-166), the
        key and value written into the bf16 caches ``[1, n_kv, capacity, 128]`` at the token's
        position ``positions[0]`` (an int32 device tensor), and grouped-query attention over keys
        0 .. position as ``DecodeAttention`` computes it (attention.py:37-178), into ``out``
        (bf16 ``[1, n_q * 128]``, which later projections may read, e.g. o). ``splits`` items per KV
        head share the keys; their partials are merged in the same launch."""
        if self.m != 1:
            raise ValueError("an attention stage takes one token (m = 1)")
        if n_q != 4 * n_kv:
            raise ValueError("the attention stage serves 4 query heads per KV head")
        width = (n_q + 2 * n_kv) * 128
        earlier = [t for t in self._keep[2::3] if t is not None and t.data_ptr() == qkv.data_ptr()]
        if not earlier or tuple(qkv.shape) != (1, width) or qkv.dtype != torch.bfloat16:
            raise ValueError(f"qkv must be the bf16 [1, {width}] output tensor of an earlier projection")
        cap = k_cache.shape[2]
        for name, t in (("k_cache", k_cache), ("v_cache", v_cache)):
            if t.dtype != torch.bfloat16 or tuple(t.shape) != (1, n_kv, cap, 128) or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous bf16 [1, {n_kv}, capacity, 128] tensor")
        for name, t in (("q_norm_w", q_norm_w), ("k_norm_w", k_norm_w)):
            if t.dtype != torch.bfloat16 or tuple(t.shape) != (128,):
                raise ValueError(f"{name} must be bf16 [128]")
        if cos.dtype != torch.bfloat16 or cos.dim() != 2 or cos.shape[1] != 128 or sin.shape != cos.shape:
            raise ValueError("cos and sin must be bf16 [table_rows, 128]")
        if positions.dtype != torch.int32 or positions.numel() < 1:
            raise ValueError("positions must be an int32 device tensor holding the token's position")
        if out.dtype != torch.bfloat16 or tuple(out.shape) != (1, n_q * 128) or not out.is_contiguous():
            raise ValueError(f"out must be a contiguous bf16 [1, {n_q * 128}] tensor")
        if not 1 <= splits <= 64:
            raise ValueError("splits must be 1..64")
        _lib.require_device(qkv, q_norm_w, k_norm_w, cos, sin, positions, k_cache, v_cache, out)
        scale = 128 ** -0.5 if scale is None else scale
        for kind, x, y, k in ((1, qkv.data_ptr(), None, width), (2, None, out.data_ptr(), 0)):
            self.calls.append(_lib.StackCall(None, None, x, y, n_q * 128, k, _lib.MODE_BF16, 0))
            self.norms.append(_lib.NormInput())
            self.attns.append(_lib.StackAttention(kind, n_q, n_kv, int(splits), cap, cos.shape[0], q_norm_w.data_ptr(),
                                                  k_norm_w.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                                  positions.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                                                  float(eps), float(scale)))
        self._keep += [None, qkv, None, None, None, out]
        self._extra = getattr(self, "_extra", []) + [q_norm_w, k_norm_w, cos, sin, positions, k_cache, v_cache]
        self.desc = None
        return self

    def add_normed(self, weight, resid, y, norm_w, eps, delta=None, resid_out=None, normed_out=None,
                   swiglu=False):
        """Append a projection of bf16(bf16(r * rsqrt(mean(r^2) + eps)) * norm_w) with
        r = bf16(resid + delta) (r = resid without delta), the residual add + RMSNorm run inside
        the launch (norm.py:53-80, 125-154). ``resid`` is memory the chain does not write or an
        earlier stage's ``resid_out``; ``delta`` the output tensor of an earlier projection;
        ``resid_out`` / ``normed_out`` (optional) receive r and the normed input. FP8 W8A8
        quantizes the normed input per token inside the same stage. A whole decode layer:

            chain.add_normed(qkv, h_in, y_qkv, w_in, eps, resid_out=h0)          # rmsnorm(h_in)
            chain.add(o, y_qkv[:, :4096], y_o)
            chain.add_normed(gate_up, h0, y_act, w_post, eps, delta=y_o, resid_out=h1, swiglu=True)
            chain.add(down, y_act, y_down)
            chain.add_normed(next_qkv, h1, ..., delta=y_down, resid_out=h2)      # the next layer
        """
        if not isinstance(weight, Tiled) or weight.fmt != self.fmt:
            raise ValueError(f"the chain takes {self.fmt} weights in tile layout (qlinear.prepare)")
        shape = (self.m, weight.k)
        tensors = [resid, norm_w] + [t for t in (delta, resid_out, normed_out) if t is not None]
        _lib.require_device(weight.weight, weight.scale, y, *tensors)
        for name, t in (("resid", resid), ("delta", delta), ("resid_out", resid_out), ("normed_out", normed_out)):
            if t is not None and (t.dtype != torch.bfloat16 or tuple(t.shape) != shape or not t.is_contiguous()):
                raise ValueError(f"{name} must be a contiguous bf16 [{self.m}, {weight.k}] tensor")
        if norm_w.dtype != torch.bfloat16 or tuple(norm_w.shape) != (weight.k,):
            raise ValueError(f"norm_w must be bf16 [{weight.k}]")
        out_n = weight.rows // 2 if swiglu else weight.rows
        if y.dtype != torch.bfloat16 or tuple(y.shape) != (self.m, out_n):
            raise ValueError(f"y must be bf16 [{self.m}, {out_n}]")
        ptr = lambda t: None if t is None else t.data_ptr()
        self.calls.append(_lib.StackCall(weight.weight.data_ptr(), weight.scale.data_ptr(), None, y.data_ptr(),
                                         weight.rows, weight.k, _lib.MODE_SWIGLU if swiglu else _lib.MODE_BF16, 0))
        self.norms.append(_lib.NormInput(ptr(resid), ptr(delta), ptr(norm_w), ptr(resid_out), ptr(normed_out),
                                         float(eps), 0))
        self.attns.append(_lib.StackAttention())
        self._keep += [weight, resid, y]
        self._extra = getattr(self, "_extra", []) + tensors
        self.desc = None
        return self

    def build(self):
        """Plan the chain and upload its descriptors (call after the last ``add``)."""
        if not self.calls:
            raise ValueError("empty chain")
        device = next(w for w in self._keep[0::3] if w is not None).weight.device
        lib = _lib.lib()
        arr = (_lib.StackCall * len(self.calls))(*self.calls)
        norms = (_lib.NormInput * len(self.norms))(*self.norms)
        attns = (_lib.StackAttention * len(self.attns))(*self.attns)
        fmt = _FMTS[self.fmt]
        arena_bytes, launch = ctypes.c_longlong(0), _lib.StackLaunch()
        with torch.cuda.device(device):
            opts = (self.waves, self.groups_per_cu)
            _lib.check(lib.qlx_stack_build_step(fmt, self.m, arr, len(self.calls), norms, attns, *opts, None, None,
                                                None, arena_bytes, launch), "qlx_stack_build_step")
            self.arena = torch.zeros(max(arena_bytes.value, 256), dtype=torch.uint8, device=device)
            self.error = torch.zeros(1, dtype=torch.int32, device=device)
            host = torch.empty(lib.qlx_stack_desc_size() * len(self.calls), dtype=torch.uint8)
            plans = (_lib.Plan * len(self.calls))()
            _lib.check(lib.qlx_stack_build_step(fmt, self.m, arr, len(self.calls), norms, attns, *opts,
                                                ctypes.c_void_p(host.data_ptr()), plans, _lib.ptr(self.arena),
                                                arena_bytes, launch), "qlx_stack_build_step")
            self.desc = host.to(device)
        #: (waves, kw, rw, most K pieces of one row block) per projection
        self.configs = [(p.waves, p.kw, p.rw, p.splits) for p in plans]
        self.launch = launch
        self.grid, self.lds = launch.grid, launch.lds_bytes
        self.device = device
        return self

    def run(self, budget_us=BUDGET_US):
        """Run the whole chain once on the current stream. Capturable: the run's epoch (the tag
        of what it publishes) is kept in the arena and advanced by the kernel, so every replay
        of a captured run is a new run. Runs of one chain must not overlap (one stream)."""
        if self.desc is None:
            self.build()
        _lib.call("qlx_stack_run", _FMTS[self.fmt], _lib.ptr(self.desc), len(self.calls), ctypes.byref(self.launch),
                  _lib.ptr(self.arena), _lib.ptr(self.error), int(budget_us), _lib.stream(self.device))

    def failed(self):
        """True if a wait of any run so far gave up (that run's outputs are undefined).
        Synchronizes with the device."""
        return bool(self.error.item())

    #: The kinds of wait, by bit of the error word: an activation from an earlier projection, a
    #: piece's partial sums.
    WAIT_SITES = ("input", "partial")

    def failed_waits(self):
        """The kind of the first wait that gave up (a list; empty if none did)."""
        e = int(self.error.item())
        return [name for i, name in enumerate(self.WAIT_SITES) if e >> i & 1]

    def reset(self):
        """Clear the error flag (nothing else outlives a failed run)."""
        self.error.zero_()

    def bytes_moved(self):
        return sum(w.bytes_moved() for w in self._keep[0::3] if w is not None)
