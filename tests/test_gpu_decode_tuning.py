"""The in-graph races (kernels/decode_tuning.py; the reference's engine/kernels/decode_tuning.py:17-79):
``race_steps`` picks the clearly faster whole step and keeps the incumbent when there is no
clear winner; ``tune_output_projection`` races o's split-K schedules inside a whole captured
decode step of an engine-shaped object (the reference Engine's attributes the race reads and
writes), leaves its position and token as they were, and routes ``matmul["o"]`` to the winner."""

import functools

import pytest
import torch

from kernels import cuda_fp8, decode_tuning, norm

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _weight(n, k, seed, fmt="fp8"):
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = (torch.randn(n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    return cuda_fp8.prepare(cuda_fp8.quantize(w, fmt=fmt))


def test_race_steps_picks_a_clear_winner_and_keeps_a_tie():
    w = _weight(2560, 4096, 1)
    x = torch.randn(1, 4096, device=DEV).to(torch.bfloat16)
    one = lambda: cuda_fp8.matmul(x, w)

    def eight():
        for _ in range(8):
            cuda_fp8.matmul(x, w)
    best, med = decode_tuning.race_steps({"eight": eight, "one": one}, incumbent="eight")
    assert best == "one" and med["one"] < med["eight"], med
    best, med = decode_tuning.race_steps({"a": one, "b": one}, incumbent="a", margin=0.2)
    assert best == "a", med
    with pytest.raises(ValueError):
        decode_tuning.race_steps({"a": one}, incumbent="b")


class EngineShaped:
    """The decode-step surface of the reference Engine that the output-projection race reads and
    writes: ``graph``, ``draft``, ``batch``, ``integer_mlp``, ``families``, ``partial_config``,
    ``matmul``, ``_ordinary_matmul``, ``pos``, ``token`` and ``_decode_step`` (which here runs a
    few layers of o as split-K planes into the residual + RMSNorm, as engine.py:893-906 does)."""

    def __init__(self, batch=1, layers=6):
        self.graph, self.draft, self.batch, self.integer_mlp = object(), False, batch, False
        self.families = {"o": "fp8"}
        self.partial_config = {"o": (8, 4, 1, 1, 0)}
        self.matmul = {"o": functools.partial(cuda_fp8.matmul, config=self.partial_config["o"])}
        self._ordinary_matmul = dict(self.matmul)
        self.pos = torch.tensor([17], dtype=torch.int32, device=DEV)
        self.token = torch.full((batch,), 5, dtype=torch.int64, device=DEV)
        g = torch.Generator(device=DEV).manual_seed(3)
        self.o = [_weight(2560, 4096, 10 + i) for i in range(layers)]
        self.norm_w = [(1 + 0.1 * torch.randn(2560, generator=g, device=DEV)).to(torch.bfloat16)
                       for _ in range(layers)]
        self.attn = torch.randn(batch, 4096, generator=g, device=DEV).to(torch.bfloat16)
        self.h = torch.randn(batch, 2560, generator=g, device=DEV).to(torch.bfloat16)
        self.out = torch.empty(batch, 2560, dtype=torch.bfloat16, device=DEV)

    def _decode_step(self):
        x = self.h
        for o, w in zip(self.o, self.norm_w):
            planes = cuda_fp8.matmul_partials(self.attn, o, self.partial_config["o"])
            x, normed = norm.add_rms_norm_partials(x, planes, w, 1e-6)
        self.out.copy_(normed)
        self.pos += 1
        self.token += 1


@pytest.mark.parametrize("batch", [1, 8])
def test_tune_output_projection_inside_the_captured_step(batch):
    engine = EngineShaped(batch)
    engine._decode_step()
    want = engine.out.clone()
    engine.pos.fill_(17)
    engine.token.fill_(5)
    changed = decode_tuning.tune_output_projection(engine)
    chosen = engine.partial_config["o"]
    assert chosen in [(8, 4, 1, 1, 0)] + [(8, s, 1, 1, 0) for s in decode_tuning.O_SPLITS]
    assert changed == (chosen != (8, 4, 1, 1, 0))
    assert engine.matmul["o"].keywords["config"] == chosen
    assert int(engine.pos.item()) == 17 and bool((engine.token == 5).all())
    engine._decode_step()  # the winner's schedule: the same sums up to fp32 order
    got = engine.out.float()
    assert torch.allclose(got, want.float(), rtol=2 ** -6, atol=2 ** -6 * want.float().abs().max().item())
    # the conditions under which the reference does not race
    for attr, value in (("draft", True), ("batch", 17), ("integer_mlp", True)):
        other = EngineShaped(1, layers=1)
        setattr(other, attr, value)
        assert decode_tuning.tune_output_projection(other) is False
