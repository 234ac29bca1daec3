"""greedy decode of a seeded random-init 36-layer Qwen3-4B-shaped model,
W8A16 / FP8 W8A8 / W4A16 at batch 1 and 32, checked against the torch reference by the
reference harness's teacher-forced replay (bench/harness.py:136-152, TIE_MARGIN at :21).

Every op of every decode step runs through the gfx950 library (qwen3_random.decode_step):
RMSNorm and residual + RMSNorm, the projections (qkv, o, gate_up with the fused SwiGLU, down,
lm_head), the q/k head norm + RoPE + KV-cache write and decode attention. The reference replays
in torch (its linears, its head norm + RoPE statement, fp32 attention).

The check, per emitted step t of every sequence:

* the library's logits (those token t was chosen from) against the reference's logits on
  the same context (teacher-forced replay): max |delta| and relative L2 are measured. The
  library rounds to bf16 exactly where the reference does (attention: its probabilities enter
  the value product in bf16, as the reference engine's decode kernel has them), so what
  separates them is summation order and that rounding, amplified through 36 layers -- the same
  kind of difference as between the reference's own fp32 and fp64 matmuls. The relative L2 must
  stay within twice that self-spread (the largest over the run's steps);
* the library's max |delta| within DELTA_FACTOR times the reference's own fp32-vs-fp64 max
  |delta| (largest over the run's steps): the library may not be noisier than a stated multiple
  of the reference itself;
* **identity where the reference decides**: wherever the reference's top-1 / top-2 margin
  exceeds twice the reference's own fp32-vs-fp64 max |delta| at that step, the emitted token
  must be the reference's argmax. Which steps count depends on the reference alone, not on the
  library's error (every step is counted; the ones below the bound are printed);
* the harness's own gate: best - chosen reference logit <= TIE_MARGIN on every step.
"""

import pytest
import torch

from qwen3_random import RandomQwen3, VOCAB

pytestmark = pytest.mark.gpu

PROMPT, STEPS = 512, 64
TIE_MARGIN = 2.0  # the reference harness's gate on best - chosen logit (bench/harness.py:21)
#: The library's logits may differ from the fp32 reference's by this multiple of the
#: reference's own fp32-vs-fp64 spread (relative L2 per step, largest over the run).
SELF_SPREAD_FACTOR = 2.0
#: The library's max |delta logit| may be this multiple of the reference's own fp32-vs-fp64
#: max |delta logit| (largest over the run's steps).
DELTA_FACTOR = 2.0


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
            tokens, lib = model.generate(prompt, STEPS)
            ref = model.replay_logits(prompt, tokens)
            ref64 = model.replay_logits(prompt, tokens, dtype=torch.float64)
        delta = (lib - ref).abs().amax(dim=-1)                       # [B, steps]
        rel = (lib - ref).norm(dim=-1) / ref.norm(dim=-1)
        self_delta = (ref64 - ref).abs().amax(dim=-1)                # the reference's own spread
        self_rel = (ref64 - ref).norm(dim=-1) / ref.norm(dim=-1)
        bound = SELF_SPREAD_FACTOR * self_rel.max().item()
        top2 = ref.topk(2, dim=-1).values
        margin = top2[..., 0] - top2[..., 1]
        top = ref.argmax(dim=-1)
        gap = top2[..., 0] - ref.gather(2, tokens[:, :, None])[:, :, 0]
        decided = margin > 2.0 * self_delta
        agree = tokens == top
        n = tokens.numel()
        print(f"greedy {fmt} batch {batch}: max|dlogit| {delta.max().item():.4f} (median "
              f"{delta.median().item():.4f}; reference fp32 vs fp64 {self_delta.max().item():.4f}), rel-L2 max "
              f"{rel.max().item():.2e} (reference fp32 vs fp64 {self_rel.max().item():.2e}, bound {bound:.2e}); "
              f"{int(decided.sum())}/{n} steps decided by the reference "
              f"(margin > 2x its own fp32-vs-fp64 max|dlogit|), all identical: {bool(agree[decided].all())}; "
              f"{n - int(decided.sum())} steps below the bound, of which {int((~agree & ~decided).sum())} "
              f"differ (max gap {gap.max().item():.4f}); argmax-exact overall {int(agree.sum())}/{n}", flush=True)
        assert rel.max().item() <= bound, (fmt, batch, rel.max().item(), bound)
        assert delta.max().item() <= DELTA_FACTOR * self_delta.max().item(), (fmt, batch, delta.max().item())
        assert bool(agree[decided].all()), (fmt, batch, "token differs where the reference decides")
        assert gap.max().item() <= TIE_MARGIN, (fmt, batch, gap.max().item())
        del lib, ref, ref64
    del model
