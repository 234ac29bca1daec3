"""Grouped-query decode attention over the KV cache: drop-in for the reference's
``kernels.attention`` (engine/kernels/attention.py:181-318).

``DecodeAttention`` keeps the reference's constructor, call and ``tuned`` race. The work is
``qlx_decode_attention`` (csrc/attention.hip): a workgroup per (sequence x KV head, split) runs
S^T = K Q^T and P V on bf16 MFMA for all ``tokens x group`` query rows of its KV head, and with
several splits a small second kernel merges them, like the reference's split and merge kernels.
The live length is read from ``pos`` on the device and shared among the splits, so the grids
are fixed and the call captures into a HIP graph.
"""

import ctypes
import sys

import torch

from . import _lib

#: Workgroups a launch aims for: one per compute unit of an MI355X.
_WORKGROUP_TARGET = 256
#: Fewest keys a split should hold at full capacity (four waves of one 32-key block).
_MIN_SPLIT_KEYS = 128
_MAX_SPLITS = 64


def plan_splits(capacity: int, batch: int, n_kv: int) -> tuple[int, int]:
    """How many workgroups share each KV head, and the longest chunk one of them reads.

    Doubles the split count while the grid is below one workgroup per CU and a split would
    still hold ``_MIN_SPLIT_KEYS`` keys at full capacity (the reference's rule,
    attention.py:181-196, with MI355X's 256 CUs). The kernel divides the *live* length among
    the splits, so the chunk returned is the one a full cache gives.
    """
    splits = 1
    while (splits < _MAX_SPLITS and batch * n_kv * splits < _WORKGROUP_TARGET
           and capacity >= _MIN_SPLIT_KEYS * 2 * splits):
        splits *= 2
    length = ((capacity + splits - 1) // splits + 31) // 32 * 32
    return splits, length


class DecodeAttention:
    """Persistent output and split workspace, sized once so the call can be captured.

    ``tokens`` is how many query positions one pass carries (1 for plain decoding, the
    confirmed token plus its draft when speculating); token t sits at ``pos + t`` and sees keys
    ``0 .. pos + t``. ``config`` picks the split count: an int, or the reference's
    ``(splits, block_n, warps)`` tuple, of which only ``splits`` applies here (blocks are 32 keys
    per wave, four waves per workgroup).
    """

    def __init__(self, batch, n_kv, group, head_dim, capacity, device, tokens=1, config=None, quant=False):
        if head_dim != 128:
            raise ValueError("decode attention supports head_dim 128")
        if tokens * group > 64:
            raise ValueError("decode attention supports tokens x group <= 64 query rows per KV head")
        self.batch, self.n_kv, self.group, self.head_dim = batch, n_kv, group, head_dim
        self.capacity, self.tokens, self.quant = capacity, tokens, quant
        self.n_q = n_kv * group
        self.scale = head_dim ** -0.5
        self.splits, self.split_len = plan_splits(capacity, batch, n_kv)
        if config is not None:
            splits = config if isinstance(config, int) else config[0]
            if splits not in (1, 2, 4, 8, 16, 32, 64):
                raise ValueError("attention splits must be a power of two up to 64")
            self.splits = splits
            self.split_len = ((capacity + splits - 1) // splits + 31) // 32 * 32
        self.direct = self.splits == 1
        self.device = torch.device(device)
        size = ctypes.c_size_t()
        _lib.call("qlx_attention_workspace", batch, n_kv, group, tokens, self.splits, ctypes.byref(size))
        self.workspace = torch.empty(max(size.value, 1), dtype=torch.uint8, device=self.device)
        self.out = torch.empty(batch * tokens, self.n_q * head_dim, dtype=torch.bfloat16, device=self.device)

    def __call__(self, q, k_cache, v_cache, pos, k_scale=None, v_scale=None):
        """``q`` is ``[batch * tokens, n_q * head_dim]``; caches ``[batch, n_kv, capacity, d]``.

        With ``quant`` the caches are INT8 and ``k_scale``/``v_scale`` the fp32
        ``[batch, n_kv, capacity]`` scales. Returns the persistent output buffer.
        """
        if self.quant != (k_scale is not None) or (k_scale is None) != (v_scale is None):
            raise ValueError("scales must be given exactly when the cache is quantised")
        shape = (self.batch, self.n_kv, self.capacity, self.head_dim)
        if tuple(k_cache.shape) != shape or tuple(v_cache.shape) != shape:
            raise ValueError(f"caches must be {list(shape)}")
        want = torch.int8 if self.quant else torch.bfloat16
        if k_cache.dtype != want or v_cache.dtype != want:
            raise ValueError(f"caches must be {want}")
        if self.quant and (k_scale.dtype != torch.float32 or tuple(k_scale.shape) != shape[:3]
                           or v_scale.dtype != torch.float32 or tuple(v_scale.shape) != shape[:3]):
            raise ValueError("cache scales must be fp32 [batch, n_kv, capacity]")
        if q.dtype != torch.bfloat16 or tuple(q.shape) != (self.batch * self.tokens, self.n_q * self.head_dim):
            raise ValueError(f"q must be bfloat16 [{self.batch * self.tokens}, {self.n_q * self.head_dim}]")
        if pos.dtype != torch.int32 or pos.numel() < 1:
            raise ValueError("pos must be an int32 device tensor holding token 0's position")
        _lib.require_device(q, k_cache, v_cache, k_scale, v_scale, pos)
        _lib.call("qlx_decode_attention", _lib.ptr(q), _lib.ptr(k_cache), _lib.ptr(v_cache), _lib.ptr(k_scale),
                  _lib.ptr(v_scale), _lib.ptr(pos), _lib.ptr(self.out), _lib.ptr(self.workspace),
                  self.workspace.numel(), self.batch, self.n_kv, self.group, self.head_dim, self.tokens,
                  self.capacity, self.splits, float(self.scale), _lib.stream(q.device))
        return self.out

    @torch.no_grad()
    def tuned(self, keys, values, first_position, last_position, use_graph=True, key_scales=None,
              value_scales=None):
        """Pick the split count once, before decode is captured (the reference's contract,
        engine/kernels/attention.py:227-280: every layer's cache at both ends of generation, a
        candidate agrees with this object within 0.04 and is finite, the planned object stays
        unless another is more than 5 % faster; returns the chosen object).

        Every split count is built and checked for agreement first. Each one admitted then gets
        one timed program -- all layers' caches at both positions, extended to a 1 GiB rotation
        so the Infinity Cache cannot serve the keys, captured as one HIP graph -- and the
        programs run in rounds, each round in a rotated order, so a clock or thermal drift over
        the race touches every candidate alike. The statistic is the median over rounds.
        """
        from .timing import rotation

        device = self.out.device
        gen = torch.Generator(device=device).manual_seed(0)
        q = torch.randn(self.batch * self.tokens, self.n_q * self.head_dim, generator=gen, device=device)
        q = q.to(torch.bfloat16)
        ends = [torch.tensor([p], dtype=torch.int32, device=device) for p in sorted({first_position, last_position})]
        scales = zip(key_scales, value_scales) if self.quant else ((None, None) for _ in keys)
        caches = [(k, v, ks, vs) for (k, v), (ks, vs) in zip(zip(keys, values), scales)]
        if not caches:
            raise ValueError("tuned needs at least one layer's cache")

        def first_layer(attn):
            k, v, ks, vs = caches[0]
            return [attn(q, k, v, p, ks, vs).clone() for p in ends]

        planned = first_layer(self)
        pool = [self] + [DecodeAttention(self.batch, self.n_kv, self.group, self.head_dim, self.capacity, device,
                                         tokens=self.tokens, config=s, quant=self.quant)
                         for s in (1, 2, 4, 8, 16, 32, 64) if s != self.splits]
        admitted = []
        for attn in pool:
            outs = first_layer(attn)
            if all(bool(torch.isfinite(o).all()) and float((o.float() - w.float()).abs().max()) <= 0.04
                   for o, w in zip(outs, planned)):
                admitted.append(attn)
        if self not in admitted:  # cannot happen: the planned object is its own reference
            admitted.insert(0, self)

        work = rotation([(cache, p) for cache in caches for p in ends])
        programs = []
        for attn in admitted:
            def sweep(attn=attn):
                for (k, v, ks, vs), p in work:
                    attn(q, k, v, p, ks, vs)
            sweep()  # creates nothing lazily, but runs every operand once before a capture
            if use_graph:
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    sweep()
                graph.replay()
                programs.append(graph.replay)
            else:
                programs.append(sweep)
        torch.cuda.synchronize()

        rounds = 5
        samples = [[] for _ in admitted]
        for r in range(rounds):
            order = [(i + r) % len(admitted) for i in range(len(admitted))]
            marks = [torch.cuda.Event(enable_timing=True) for _ in range(len(order) + 1)]
            marks[0].record()
            for j, i in enumerate(order):
                programs[i]()
                marks[j + 1].record()
            marks[-1].synchronize()
            for j, i in enumerate(order):
                samples[i].append(marks[j].elapsed_time(marks[j + 1]) / len(work))
        medians = [sorted(v)[len(v) // 2] for v in samples]
        fastest = min(range(len(admitted)), key=medians.__getitem__)
        mine = admitted.index(self)
        choice = fastest if medians[fastest] < 0.95 * medians[mine] else mine
        chosen = admitted[choice]
        print(f"engine: attention splits={chosen.splits} ({medians[choice] * 1e3:.1f} us per call; planned "
              f"{self.splits}: {medians[mine] * 1e3:.1f} us; {len(admitted)}/{len(pool)} split counts agree)",
              file=sys.stderr)
        return chosen
