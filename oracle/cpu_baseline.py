"""The reference's CPU-expressible linear path, timed as bench.py's ``cpu_baseline``.

TEST/MEASUREMENT INFRASTRUCTURE ONLY (the reported CPU baseline, never the product).

The reference's torch path is dequantize, then ``F.linear``
(engine/kernels/cuda_fp8.py:1154-1161 followed by ``F.linear`` as in
bench/gpu_checks.py:141-144 and bench/fp8_mma_probe.py:47-50). For FP8 W8A8 both
operands are dequantized: ``(x_q s_x) @ (w_q s_w)^T`` in fp32, then bf16. The activation
quantization is the per-token e4m3 rule (fp8.py:25-27 with group = K, fp32 scale).

Each format has its dequantize (``DEQUANT``) and its matmul on a dequantized weight
(``matmul``), so the baseline can be timed both ways: dequantize + matmul per call, and
the matmul alone on weights dequantized beforehand.
"""

import torch
import torch.nn.functional as F


def fp8_act_quant(x):
    xf = x.float()
    s = (xf.abs().amax(dim=1, keepdim=True) / 448.0).clamp(min=1e-12)
    return (xf / s).clamp(-448.0, 448.0).to(torch.float8_e4m3fn), s


def dequant_fp8(wq, ws):
    """e4m3 [N, K] with bf16 per-channel scales -> fp32 w_q * s_w (exact in fp32)."""
    return wq.float() * ws.float()[:, None]


def dequant_w4(words, scales, group=128):
    """int32 k32 words [N, K/8] + bf16 scales [N, K/group] -> bf16 [N, K]."""
    n = words.shape[0]
    k = words.shape[1] * 8
    shifts = torch.arange(0, 32, 4, dtype=torch.int32)
    codes = (words.unsqueeze(-1) >> shifts) & 0xF
    q = codes.reshape(n, k).float() - 8.0
    return (q.view(n, k // group, group) * scales.float()[:, :, None]).view(n, k).to(torch.bfloat16)


def dequant_w8(q, scales):
    """int8 [N, K] + bf16 per-channel scales [N] -> bf16 [N, K]."""
    return (q.float() * scales.float()[:, None]).to(torch.bfloat16)


DEQUANT = {"fp8": dequant_fp8, "w4a16": dequant_w4, "w8a16": dequant_w8}


def matmul(fmt, x, w):
    """The matmul on a dequantized weight: F.linear in bf16, or for FP8 W8A8 the per-token
    e4m3 activation times the fp32 weight, rounded to bf16."""
    if fmt == "fp8":
        xq, sx = fp8_act_quant(x)
        return ((xq.float() * sx) @ w.T).to(torch.bfloat16)
    return F.linear(x, w)


def linear_fp8_w8a8(x, wq, ws):
    """bf16 [M,K] x e4m3 [N,K] (bf16 scale [N]) -> bf16 [M,N], dequantize-then-matmul."""
    return matmul("fp8", x, dequant_fp8(wq, ws))


def linear_w4a16(x, words, scales, group=128):
    return matmul("w4a16", x, dequant_w4(words, scales, group))


def linear_w8a16(x, q, scales):
    return matmul("w8a16", x, dequant_w8(q, scales))


LINEARS = {"fp8": linear_fp8_w8a8, "w4a16": linear_w4a16, "w8a16": linear_w8a16}
