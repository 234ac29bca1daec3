"""greedy decode of a seeded random-init 36-layer Qwen3-4B-shaped model,
W8A16 / FP8 W8A8 / W4A16 at batch 1 and 32, checked against the torch reference by the
reference harness's teacher-forced replay (bench/harness.py:136-152, TIE_MARGIN at :21).

Every decode-step projection (qkv, o, gate_up with the fused SwiGLU, down, lm_head) runs
through the gfx950 library; attention, norms and RoPE are shared torch code (qwen3_random).

Measured on MI355X (seed 5; batch 1 / batch 32): argmax-exact W4A16 0.906 / 0.888 (the
reference against itself at fp64: 0.922 / 0.902), W8A16 0.922 / 0.888 (0.891 / 0.918),
FP8 W8A8 0.563 / 0.510 (0.547 / 0.517); largest gap 0.19 logits at 16-bit weights, 1.19 at
FP8, against the reference's margin of 2.
"""

import pytest
import torch

from qwen3_random import RandomQwen3, VOCAB

pytestmark = pytest.mark.gpu

PROMPT, STEPS = 512, 64
TIE_MARGIN = 2.0  # the reference harness's gate on best - chosen logit (bench/harness.py:21)


@pytest.fixture(autouse=True)
def _free():
    yield
    torch.cuda.empty_cache()


@pytest.mark.parametrize("fmt", ["w4a16", "w8a16", "fp8"])
def test_greedy_tokens_match_reference(fmt):
    torch.backends.cuda.matmul.allow_tf32 = False
    print(f"greedy {fmt}: building the 36-layer model", flush=True)
    model = RandomQwen3(fmt, seed=5)
    for batch in (1, 32):
        g = torch.Generator(device="cuda").manual_seed(1000 + batch)
        prompt = torch.randint(0, VOCAB, (batch, PROMPT), generator=g, device="cuda")
        with torch.inference_mode():
            tokens = model.generate(prompt, STEPS)
            gap, exact, best, top = model.replay(prompt, tokens)
            # the same reference with fp64 matmuls: how often two roundings of the reference agree
            _, _, _, top64 = model.replay(prompt, tokens, dtype=torch.float64)
        self_agree = (top64 == top).float().mean().item()
        n = exact.numel()
        frac = exact.float().mean().item()
        worst = gap.max().item()
        # the gaps of the steps whose token is not the reference's argmax, in units of one
        # bf16 step of that step's best logit (the logits are bf16 on both sides)
        ulp = torch.ldexp(torch.ones_like(best), torch.frexp(best.abs())[1] - 8)
        miss = (gap[~exact] / ulp[~exact]).tolist()
        print(f"greedy {fmt} batch {batch}: {int(exact.sum())}/{n} argmax exact ({frac:.4f}; reference fp32 vs fp64 "
              f"{self_agree:.4f}), max gap {worst:.4f}, "
              f"misses in bf16 steps {sorted(miss)[-8:]}, best logit range "
              f"{best.min().item():.2f}..{best.max().item():.2f}", flush=True)
        assert worst <= TIE_MARGIN, (fmt, batch, worst)
        # Exact agreement cannot be asked of any path that does not round exactly as the
        # reference: two roundings of the reference itself (fp32 vs fp64 matmuls) disagree on
        # 8-10 % of these random-init steps at 16-bit weights and on ~45 % at FP8 W8A8, whose
        # 3-bit-mantissa activation codes turn one-ulp differences into code flips. The library
        # must agree with the reference as well as the reference agrees with itself, within the
        # sampling noise of the proportion (2 sigma: ~0.12 at 64 steps, ~0.03 at 2048).
        noise = 2.0 * (2 * 0.25 / n) ** 0.5
        assert frac >= self_agree - noise, (fmt, batch, frac, self_agree)
    del model
