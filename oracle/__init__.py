"""CPU oracle for the quantized decode linear path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, what the reference computes on the hot path
(quantize, pack, relayout, dequantize-then-matmul, the split-K and SwiGLU
epilogues) and, in ``attention_oracle``, on the path's QKV consumer (head norm,
RoPE, cache writes) and decode attention. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker or
as the reported CPU baseline. The product path (``kernels`` and the HIP
library) never imports, links or calls anything here.

Pinning: every function is checked by ``tests/test_oracle.py`` (``attention_oracle``:
``tests/test_oracle_attention.py``) against the
golden vectors in ``tests/golden/`` (written from the reference's own
functions), the reference's test invariants, torch/transformers library
routines, or brute force on tiny inputs. See the per-function docstrings for
which check pins which function.
"""

from .qlinear_oracle import *  # noqa: F401,F403
