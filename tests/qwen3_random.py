"""A seeded random-init Qwen3-4B-shaped model for the greedy-decode parity check.

Every op of a decode step runs through the gfx950 library (the drop-in path): RMSNorm and the
residual add + RMSNorm, the quantized projections (SwiGLU fused into gate_up), the q/k head
norm + RoPE + KV-cache write, and decode attention over the cache. The reference side is torch:
the reference engine's CPU-expressible linear path, dequantize-then-``F.linear``
(engine/kernels/cuda_fp8.py:1154-1161 followed by F.linear, as bench/gpu_checks.py:141-144 checks
it), here in fp32 on the GPU (for FP8 W8A8: (x_q s_x)(w_q s_w)^T with the dynamic per-token
activation scale); its head norm + RoPE as the reference's torch statement
(engine/kernels/reference.py:31-46) with bf16 cos/sin tables built as the engine builds them
(engine/engine.py:350-358); fp32 softmax attention; Qwen3RMSNorm. Prefill (512 prompt tokens)
is out of the product's scope: it runs the reference side and fills the cache both sides read.

The comparison is the reference harness's rule (bench/harness.py:136-152): the emitted
tokens are replayed teacher-forced through the reference model; at every step the gap
between the reference's best logit and the logit of the emitted token is measured, and
whether the emitted token is the reference's argmax.

Model shape: hidden 2560, intermediate 9728, 32 query / 8 key-value
heads of 128, 36 layers, vocab 151936, tied embedding / lm_head, RMSNorm eps 1e-6, RoPE
theta 5e6. Norm weights are 1 + 0.1 N(0, 1) as the reference's tests draw them
(tests/test_engine.py:47-51); projections and the embedding are N(0, 0.02).
"""

import torch

HIDDEN, INTER, HEADS, KV_HEADS, HEAD_DIM = 2560, 9728, 32, 8, 128
VOCAB, LAYERS, EPS, THETA = 151936, 36, 1e-6, 5e6
#: KV-cache slots per sequence: the 512-token prompt and 64 decode steps fit.
CAPACITY = 640


# ---- reference linears (torch fp32) ------------------------------------------------------

def unpack_w4(q, s):
    """bf16(q * s) of W4A16 k32 words: nibble i of word j is k = 8 j + i, code = q + 8."""
    n, kw = q.shape
    shifts = torch.arange(8, device=q.device, dtype=torch.int32) * 4
    codes = (q.unsqueeze(-1) >> shifts) & 0xF
    vals = (codes - 8).reshape(n, kw * 8).float()
    return (vals * s.float().repeat_interleave(128, dim=1)).to(torch.bfloat16)


def dequantize(fmt, packed):
    """The reference's dequantized bf16 weight (cuda_fp8.py:1154-1161 with the north-star formats)."""
    q, s = packed
    if fmt == "w8a16":
        return (q.float() * s.float()[:, None]).to(torch.bfloat16)
    if fmt == "w4a16":
        return unpack_w4(q, s)
    raise ValueError(fmt)


def fp8_act(x):
    """Per-token e4m3 activation quantize: s = max(amax/448, 1e-12), code = e4m3(clamp(x/s))."""
    xf = x.float()
    s = torch.clamp(xf.abs().amax(dim=1, keepdim=True) / 448.0, min=1e-12)
    return torch.clamp(xf / s, -448.0, 448.0).to(torch.float8_e4m3fn), s


def ref_linear(fmt, x, packed, deq, dtype=torch.float32):
    """y = x W^T in `dtype` (fp32; fp64 for the rounding-level variant), rounded to bf16 once."""
    x2 = x.reshape(-1, x.shape[-1])
    if fmt == "fp8":
        xq, sx = fp8_act(x2)
        q, s = packed
        w = q.to(dtype) * s.to(dtype)[:, None]
        y = (xq.to(dtype) * sx.to(dtype)) @ w.t()
    else:
        y = x2.to(dtype) @ deq.to(dtype).t()
    return y.to(torch.bfloat16).reshape(*x.shape[:-1], -1)


# ---- the model ---------------------------------------------------------------------------

class RandomQwen3:
    """Weights of one format, quantized on the device by the library's pack kernels."""

    def __init__(self, fmt, seed=0, layers=LAYERS, device="cuda"):
        from kernels import qlinear
        self.fmt, self.layers, self.device = fmt, layers, device
        self.ref_dtype = torch.float32
        quant, self.linear_fn, _ = qlinear.FORMATS[fmt]
        g = torch.Generator(device=device).manual_seed(seed)

        def randn(*shape, std=1.0):
            return (torch.randn(*shape, generator=g, device=device) * std).to(torch.bfloat16)

        def norm(n):
            return (1.0 + 0.1 * torch.randn(n, generator=g, device=device)).to(torch.bfloat16)

        self.embed = randn(VOCAB, HIDDEN, std=0.02)
        self.blocks = []
        for _ in range(layers):
            blk = {"in_norm": norm(HIDDEN), "post_norm": norm(HIDDEN), "q_norm": norm(HEAD_DIM),
                   "k_norm": norm(HEAD_DIM)}
            shapes = {"qkv": ((HEADS + 2 * KV_HEADS) * HEAD_DIM, HIDDEN), "o": (HIDDEN, HEADS * HEAD_DIM),
                      "gate_up": (2 * INTER, HIDDEN), "down": (HIDDEN, INTER)}
            for name, (n, k) in shapes.items():
                packed = quant(randn(n, k, std=0.02))
                blk[name] = (packed, qlinear.prepare(packed, fmt), dequantize(fmt, packed) if fmt != "fp8" else None)
            self.blocks.append(blk)
        self.final_norm = norm(HIDDEN)
        lm = quant(self.embed)  # tied: the lm_head is the quantized embedding
        self.lm_head = (lm, qlinear.prepare(lm, fmt), dequantize(fmt, lm) if fmt != "fp8" else None)
        # cos/sin tables (bf16 [positions, 128]) as engine/engine.py:350-358 builds them
        half = HEAD_DIM // 2
        steps = torch.arange(0, half, dtype=torch.int64, device=device).float()
        inv_freq = 1.0 / (THETA ** (steps / half))
        positions = torch.arange(CAPACITY, dtype=torch.int64, device=device).float()
        emb = torch.cat([positions[:, None] * inv_freq[None, :]] * 2, dim=-1)
        self.cos = emb.cos().to(torch.bfloat16).contiguous()
        self.sin = emb.sin().to(torch.bfloat16).contiguous()

    # -- pieces shared by both sides --------------------------------------------------------

    @staticmethod
    def rms_norm(x, w):
        """Qwen3RMSNorm: fp32 statistics, bf16 result times the weight."""
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + EPS)
        return w * xf.to(torch.bfloat16)

    def head_norm_rope(self, x, w, pos):
        """Per-head RMSNorm then RoPE of [B, T, H, D] at positions [T]: the reference's torch
        statement (engine/kernels/reference.py:31-46), three bf16 roundings."""
        f = x.float()
        scale = torch.rsqrt(f.pow(2).mean(-1, keepdim=True) + EPS)
        normed = ((f * scale).to(torch.bfloat16).float() * w.float()).to(torch.bfloat16).float()
        half = HEAD_DIM // 2
        rotated = torch.cat([-normed[..., half:], normed[..., :half]], dim=-1)
        c = self.cos[pos].float()[:, None, :]
        s = self.sin[pos].float()[:, None, :]
        left = (normed * c).to(torch.bfloat16).float()
        right = (rotated * s).to(torch.bfloat16).float()
        return (left + right).to(torch.bfloat16)

    @staticmethod
    def attention(q, k, v, causal_offset):
        """GQA attention in fp32 with contiguous operands: q [B, 32, T, D], k, v [B, 8, S, D];
        query t sees keys 0 .. causal_offset + t."""
        b, _, t, _ = q.shape
        s = k.shape[2]
        rep = HEADS // KV_HEADS
        qf = q.float().reshape(b, KV_HEADS, rep * t, HEAD_DIM)
        kt = k.float().transpose(-1, -2).contiguous()
        scores = torch.matmul(qf, kt).reshape(b, KV_HEADS, rep, t, s) * (HEAD_DIM ** -0.5)
        qpos = torch.arange(t, device=q.device)[:, None] + causal_offset
        mask = torch.arange(s, device=q.device)[None, :] > qpos
        scores = scores.masked_fill(mask, float("-inf"))
        p = torch.softmax(scores, dim=-1).reshape(b, KV_HEADS, rep * t, s)
        out = torch.matmul(p, v.float().contiguous()).reshape(b, HEADS, t, HEAD_DIM)
        return out.to(torch.bfloat16)

    def _linear(self, which, x, w, reference):
        packed, tiled, deq = w
        if reference:
            return ref_linear(self.fmt, x, packed, deq, self.ref_dtype)
        return self.linear_fn(x, tiled, swiglu=which == "gate_up")

    def new_cache(self, batch, device="cuda"):
        """Per-layer bf16 K/V caches [B, 8, CAPACITY, 128] (the layout the library's head-norm +
        RoPE kernel writes and its decode attention reads) and the filled length."""
        shape = (batch, KV_HEADS, CAPACITY, HEAD_DIM)
        return {"len": 0, "k": [torch.zeros(shape, dtype=torch.bfloat16, device=device) for _ in range(self.layers)],
                "v": [torch.zeros(shape, dtype=torch.bfloat16, device=device) for _ in range(self.layers)]}

    def forward(self, ids, cache, reference=True):
        """The torch reference (``reference``: its linears) over [B, T] token ids after the cached
        positions: bf16 logits of every token, K/V written into the cache's slots."""
        b, t = ids.shape
        start = cache["len"]
        pos = torch.arange(start, start + t, device=ids.device)
        h = self.embed[ids]
        for li, blk in enumerate(self.blocks):
            x = self.rms_norm(h, blk["in_norm"])
            qkv = self._linear("qkv", x.reshape(b * t, HIDDEN), blk["qkv"], reference).reshape(b, t, -1)
            q = qkv[..., :HEADS * HEAD_DIM].reshape(b, t, HEADS, HEAD_DIM)
            k = qkv[..., HEADS * HEAD_DIM:(HEADS + KV_HEADS) * HEAD_DIM].reshape(b, t, KV_HEADS, HEAD_DIM)
            v = qkv[..., (HEADS + KV_HEADS) * HEAD_DIM:].reshape(b, t, KV_HEADS, HEAD_DIM)
            q = self.head_norm_rope(q, blk["q_norm"], pos).transpose(1, 2)
            k = self.head_norm_rope(k, blk["k_norm"], pos).transpose(1, 2)
            cache["k"][li][:, :, start:start + t] = k
            cache["v"][li][:, :, start:start + t] = v.transpose(1, 2)
            a = self.attention(q, cache["k"][li][:, :, :start + t], cache["v"][li][:, :, :start + t], start)
            a = a.transpose(1, 2).reshape(b * t, HEADS * HEAD_DIM).contiguous()
            h = h + self._linear("o", a, blk["o"], reference).reshape(b, t, HIDDEN)
            x = self.rms_norm(h, blk["post_norm"]).reshape(b * t, HIDDEN)
            if reference:
                gu = self._linear("gate_up", x, blk["gate_up"], True)
                act = torch.nn.functional.silu(gu[:, :INTER]) * gu[:, INTER:]
            else:
                act = self._linear("gate_up", x, blk["gate_up"], False)
            h = h + self._linear("down", act, blk["down"], reference).reshape(b, t, HIDDEN)
        cache["len"] = start + t
        h = self.rms_norm(h, self.final_norm)
        logits = self._linear("lm_head", h.reshape(-1, HIDDEN), self.lm_head, reference)
        return logits.reshape(b, t, VOCAB)

    def decode_step(self, tok, cache, attention, pos):
        """One decode step of [B] tokens with every op in the library: RMSNorm, the quantized
        projections, head norm + RoPE + cache write, decode attention, residual + RMSNorm.
        ``pos`` (int32 [1], device) is the step's position; returns fp32 logits [B, VOCAB]."""
        from kernels import add_rms_norm, qkv_norm_rope_to_cache, rms_norm
        h = self.embed[tok]
        x = rms_norm(h, self.blocks[0]["in_norm"], EPS)
        for li, blk in enumerate(self.blocks):
            qkv = self.linear_fn(x, blk["qkv"][1], swiglu=False)
            q = qkv_norm_rope_to_cache(qkv, HEADS, KV_HEADS, blk["q_norm"], blk["k_norm"], self.cos, self.sin, pos, 1,
                                       cache["k"][li], cache["v"][li], EPS)
            a = attention(q, cache["k"][li], cache["v"][li], pos)
            h, x = add_rms_norm(h, self.linear_fn(a, blk["o"][1], swiglu=False), blk["post_norm"], EPS)
            act = self.linear_fn(x, blk["gate_up"][1], swiglu=True)
            following = self.blocks[li + 1]["in_norm"] if li + 1 < self.layers else self.final_norm
            h, x = add_rms_norm(h, self.linear_fn(act, blk["down"][1], swiglu=False), following, EPS)
        cache["len"] += 1
        return self.linear_fn(x, self.lm_head[1], swiglu=False).float()

    # -- decode and replay ------------------------------------------------------------------

    def generate(self, prompt, steps):
        """Greedy decode: prefill through the reference (out of scope), then `steps` decode steps
        through the library (``decode_step``). Returns ([B, steps] token ids, [B, steps, VOCAB]
        fp32 logits each emitted token was chosen from): token t is the argmax of logits t,
        which the prefill (t = 0) or decode step t - 1 produced."""
        from kernels import DecodeAttention
        b = prompt.shape[0]
        cache = self.new_cache(b, prompt.device)
        logits = self.forward(prompt, cache, reference=True)[:, -1, :].float()
        attention = DecodeAttention(b, KV_HEADS, HEADS // KV_HEADS, HEAD_DIM, CAPACITY, prompt.device)
        pos = torch.zeros(1, dtype=torch.int32, device=prompt.device)
        out, seen = [], []
        for t in range(steps):
            tok = logits.argmax(dim=-1)
            out.append(tok)
            seen.append(logits)
            if t + 1 < steps:
                pos.fill_(cache["len"])
                logits = self.decode_step(tok, cache, attention, pos)
        return torch.stack(out, dim=1), torch.stack(seen, dim=1)

    def replay_logits(self, prompt, tokens, dtype=torch.float32):
        """Teacher-forced reference logits at every emitted step (bench/harness.py:136-152):
        [B, steps, VOCAB] fp32, entry t conditioned on the prompt and tokens[:, :t]. `dtype` is
        the reference matmuls' precision."""
        full = torch.cat([prompt, tokens], dim=1)
        cache = self.new_cache(prompt.shape[0], prompt.device)
        self.ref_dtype = dtype
        try:
            return self.forward(full, cache, reference=True)[:, prompt.shape[1] - 1:-1, :].float()
        finally:
            self.ref_dtype = torch.float32
