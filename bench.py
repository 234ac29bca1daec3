#!/usr/bin/env python
"""Decode-step linear stack of a Qwen3-4B-shaped model on one MI355X.

One step is the quantized linear stream of one decode step at batch M: 36 layers x
(qkv 2560->6144, o 4096->2560, gate_up 2560->2x9728 with the fused SwiGLU epilogue,
down 9728->2560) plus the lm_head 2560->151936, each layer with its own synthetic
weights (4.03 GB in FP8, so the 256 MB Infinity Cache cannot serve repeats), wired as in a
decode step: rmsnorm(h) -> qkv, o, residual + rmsnorm -> gate_up, down, residual + the next
layer's rmsnorm -> qkv, the final norm -> lm_head. In this linear stack o reads the query
columns of qkv where the attention output would be (same width, same dependency on qkv).
Activations are resident in HBM.

Two product paths run the linear stack: the single-call linears and norm kernels captured
once in a HIP graph, and the decode-step executor (the whole chain, its residual + RMSNorm
stages included, in one launch). ``decode_step`` times the real step with head norm + RoPE +
KV-cache write and decode attention as well: the reference's own call sequence on the
library (what Engine.generate runs), executor launches split where attention sits, and (one
token) the whole step as one executor launch with attention stages inside the chain.

Prints one JSON line (the driver's contract). ``value`` is microseconds per step for
the default workload, FP8 e4m3 W8A8 at M=1.
"""

import argparse
import json
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "dryft-flash-infer_amd"))

import torch  # noqa: E402

PEAK_HBM = 8.0e12
LAYERS = 36
HIDDEN, EPS, THETA = 2560, 1e-6, 5e6
#: Decode-step attention: the token at position CTX (a 512-token prompt) over
#: caches of CAPACITY slots per sequence and KV head.
CTX, CAPACITY = 512, 640
PROJ = [("qkv", 6144, 2560), ("o", 2560, 4096), ("gate_up", 19456, 2560), ("down", 2560, 9728)]
LM_HEAD = ("lm_head", 151936, 2560)
METRIC = "µs per decode-step linear stack + effective weight GB/s (% HBM peak), M=1"
#: Waves per executor workgroup.
EXECUTOR_WAVES = 8
#: Most tokens the decode executor takes (its residual + RMSNorm input stages run in passes
#: of whole token rows).
EXECUTOR_NORM_MAX_M = 16


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def profiled_traffic(fmt, m, kernel="gate_up_swiglu"):
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, calibrated; see its header for the commands), or None."""
    path = os.path.join(ROOT, "profiles", f"{fmt}_{kernel}_m{m}_hbm_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


class Model:
    """A Qwen3-4B-shaped decoder of one weight format: 36 layers of synthetic N(0, 0.02) weights
    (qkv, o, gate_up, down) and the lm_head, each quantized and relaid through the reference's
    own calls (``cuda_fp8.prepare(cuda_fp8.quantize(w, bits=..., fmt=...))``, engine.py:522-532);
    RMSNorm weights 1 + 0.1 N(0, 1) (the reference's tests/test_engine.py:47-51); the hidden state
    entering the step N(0, 1). With ``attention``, also the q/k head norms, bf16 RoPE tables
    (theta 5e6) and per-layer bf16 KV caches holding ``ctx`` random keys and values, the step's
    token at position ``ctx`` (a 512-token prompt)."""

    def __init__(self, fmt, m, seed=0, layers=LAYERS, attention=False, ctx=CTX, capacity=CAPACITY):
        from kernels import cuda_fp8
        self.fmt, self.m, self.layers = fmt, m, layers
        bits = 4 if fmt == "w4a16" else 8
        gen = torch.Generator(device="cuda").manual_seed(seed)

        def weight(n, k):
            w = (torch.randn(n, k, generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
            prepared = cuda_fp8.prepare(cuda_fp8.quantize(w, bits=bits, fmt=fmt))
            del w
            return prepared

        self.w = [{name: weight(n, k) for name, n, k in PROJ} for _ in range(layers)]
        self.lm_head = weight(LM_HEAD[1], LM_HEAD[2])
        #: (name, tiled weight, k, swiglu) of every projection, in step order
        self.calls = [(name, self.w[i][name].tiles, k, name == "gate_up") for i in range(layers) for name, _, k in PROJ]
        self.calls.append((LM_HEAD[0], self.lm_head.tiles, LM_HEAD[2], False))
        ng = torch.Generator(device="cuda").manual_seed(seed + 2)
        norm = lambda: (1.0 + 0.1 * torch.randn(HIDDEN, generator=ng, device="cuda")).to(torch.bfloat16)
        self.norm_in = [norm() for _ in range(layers)]
        self.norm_post = [norm() for _ in range(layers)]
        self.norm_out = norm()
        xg = torch.Generator(device="cuda").manual_seed(seed + 1)
        self.h = torch.randn(m, HIDDEN, generator=xg, device="cuda").to(torch.bfloat16)
        #: N(0, 1) activations of every input width (per-projection timings, the CPU baseline)
        self.x = {k: torch.randn(m, k, generator=xg, device="cuda").to(torch.bfloat16) for k in (2560, 4096, 9728)}
        self.attention = attention
        if attention:
            from kernels import DecodeAttention
            head = lambda: torch.randn(128, generator=ng, device="cuda").to(torch.bfloat16)
            self.q_norm = [head() for _ in range(layers)]
            self.k_norm = [head() for _ in range(layers)]
            inv = 1.0 / (THETA ** (torch.arange(0, 128, 2, dtype=torch.float32, device="cuda") / 128))
            ang = torch.outer(torch.arange(capacity, dtype=torch.float32, device="cuda"), inv)
            ang = torch.cat([ang, ang], dim=1)
            self.cos, self.sin = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
            cg = torch.Generator(device="cuda").manual_seed(seed + 3)
            self.k_cache = [torch.randn(m, 8, capacity, 128, generator=cg, device="cuda").to(torch.bfloat16)
                            for _ in range(layers)]
            self.v_cache = [torch.randn(m, 8, capacity, 128, generator=cg, device="cuda").to(torch.bfloat16)
                            for _ in range(layers)]
            self.positions = torch.tensor([ctx], dtype=torch.int32, device="cuda")
            # planned, then raced over the split counts at both ends of generation before the
            # step is captured, as the engine does (engine.py:840-845)
            self.attend = DecodeAttention(m, 8, 4, 128, capacity, "cuda").tuned(
                self.k_cache, self.v_cache, ctx, capacity - 1)
        torch.cuda.synchronize()

    # ---- the linear stack: every projection of a decode step, attention left out ----------

    def linear_chain(self):
        """The decode step's projections as one executor launch, with its residual adds and
        RMSNorms as input stages (engine.py:866-918: rmsnorm(h) -> qkv, residual + o ->
        rmsnorm -> gate_up, residual + down -> the next layer's rmsnorm -> qkv, the final norm ->
        lm_head). o reads the query columns of qkv in place of the attention output (same width
        and the same dependency on qkv). ``wiring`` records every projection's input."""
        from kernels.decode_stack import DecodeStack
        chain = DecodeStack(self.fmt, self.m, waves=EXECUTOR_WAVES)
        new = lambda n: torch.empty((self.m, n), dtype=torch.bfloat16, device="cuda")
        self.outs, self.wiring = [], []
        resid, delta, q = self.h, None, None
        for i, (name, tiled, k, sw) in enumerate(self.calls):
            layer = i // 4
            y = new(tiled.rows // 2 if sw else tiled.rows)
            if name in ("qkv", "lm_head", "gate_up"):
                w = {"qkv": self.norm_in[min(layer, self.layers - 1)], "lm_head": self.norm_out,
                     "gate_up": self.norm_post[min(layer, self.layers - 1)]}[name]
                r_out = new(HIDDEN)
                chain.add_normed(tiled, resid, y, w, EPS, delta=delta, resid_out=r_out, swiglu=sw)
                self.wiring.append({"resid": resid, "delta": delta, "w": w, "resid_out": r_out})
                resid = r_out
            else:
                x = q[:, :4096] if name == "o" else q
                chain.add(tiled, x, y)
                self.wiring.append({"x": x})
            if name in ("o", "down"):
                delta = y
            self.outs.append(y)
            q = y
        return chain.build()

    def linear_step(self):
        """The same chain as single calls (the library's linears and norm kernels), for a
        graph: FP8 W8A8 takes the fused residual + RMSNorm + per-token quantize
        (``qlinear.add_norm_quant_fp8``) in front of qkv, gate_up and the lm_head."""
        from kernels import norm, qlinear
        from kernels.cuda_small import rms_norm
        linear = qlinear.FORMATS[self.fmt][1]
        fp8 = self.fmt == "fp8"

        def normed_linear(resid, delta, w, tiled, swiglu=False):
            if fp8:
                r, xq, sx = qlinear.add_norm_quant_fp8(resid, delta, w, EPS)
                return (resid if r is None else r), qlinear.linear_fp8_w8a8_quantized(xq, sx, tiled, swiglu=swiglu)
            if delta is None:
                return resid, linear(rms_norm(resid, w, EPS), tiled, swiglu=swiglu)
            r, x = norm.add_rms_norm(resid, delta, w, EPS)
            return r, linear(x, tiled, swiglu=swiglu)

        def step():
            resid, delta = self.h, None
            for i in range(self.layers):
                w = self.w[i]
                resid, qkv = normed_linear(resid, delta, self.norm_in[i], w["qkv"].tiles)
                o = linear(qkv[:, :4096].contiguous(), w["o"].tiles)
                resid, act = normed_linear(resid, o, self.norm_post[i], w["gate_up"].tiles, swiglu=True)
                delta = linear(act, w["down"].tiles)
            return normed_linear(resid, delta, self.norm_out, self.lm_head.tiles)[1]
        return step

    # ---- the real decode step: attention included -----------------------------------------

    def engine_step(self):
        """One decode step as the reference engine runs it (engine.py:866-918, 972-986), every
        call through the reference's own signatures on this model's weights: rms_norm, then per
        layer ``cuda_fp8.matmul`` (qkv), ``qkv_norm_rope_to_cache``, ``DecodeAttention``,
        ``cuda_fp8.matmul_add_norm`` or ``matmul`` + ``add_rms_norm`` for o (whichever a race of
        whole captured steps picks, as the engine races them; only the latter past 16 rows),
        ``cuda_fp8.gate_up_swiglu``, the same for down (into the next norm), and
        ``cuda_fp8.matmul`` for the lm_head."""
        from kernels import cuda_fp8, decode_tuning, norm, qkv_norm_rope_to_cache
        from kernels.cuda_small import rms_norm
        scratch = {n: cuda_fp8.add_norm_scratch(self.m, HIDDEN, "cuda") for n in ("o", "down")}
        fused = [False]

        def add_project_norm(name, src, prepared, resid, w):
            if fused[0]:
                return cuda_fp8.matmul_add_norm(src, prepared, resid, w, EPS, scratch[name])
            return norm.add_rms_norm(resid, cuda_fp8.matmul(src, prepared), w, EPS)

        def variant(use_fused):
            def run():
                fused[0] = use_fused  # read while the step is captured
                step()
            return run

        def step():
            x = self.h
            normed = rms_norm(x, self.norm_in[0], EPS)
            for i in range(self.layers):
                w = self.w[i]
                qkv = cuda_fp8.matmul(normed, w["qkv"])
                q = qkv_norm_rope_to_cache(qkv, 32, 8, self.q_norm[i], self.k_norm[i], self.cos, self.sin,
                                           self.positions, 1, self.k_cache[i], self.v_cache[i], EPS)
                att = self.attend(q, self.k_cache[i], self.v_cache[i], self.positions)
                x, normed = add_project_norm("o", att, w["o"], x, self.norm_post[i])
                inner = cuda_fp8.gate_up_swiglu(normed, w["gate_up"])
                following = self.norm_in[i + 1] if i + 1 < self.layers else self.norm_out
                x, normed = add_project_norm("down", inner, w["down"], x, following)
            return cuda_fp8.matmul(normed, self.lm_head)

        # The engine's choice for o and down (engine.py:881-918, its fused_out race): the fused
        # GEMM + residual add + RMSNorm (up to 16 rows) or the GEMM and a separate add-norm,
        # raced as whole captured steps.
        if self.m > 16:
            return variant(False)
        choice, _ = decode_tuning.race_steps({"separate": variant(False), "fused": variant(True)}, "separate",
                                             rounds=3, replays=2)
        self.engine_choice = choice
        return variant(choice == "fused")

    def executor_step(self):
        """The same decode step with its projections on the executor, split where attention
        sits: one launch for rmsnorm -> qkv of layer 0, then per layer the head norm + RoPE +
        cache write and attention, then one launch for o, rmsnorm -> gate_up, down and the next
        layer's rmsnorm -> qkv (the last: the final norm -> lm_head). 37 executor launches and
        36 x (rope, attention) in one graph."""
        from kernels import qkv_norm_rope_to_cache
        from kernels.decode_stack import DecodeStack
        new = lambda n: torch.empty((self.m, n), dtype=torch.bfloat16, device="cuda")
        self.seg_keep = []
        qkv_out = [new(6144) for _ in range(self.layers)]
        segments = []
        chain = DecodeStack(self.fmt, self.m, waves=EXECUTOR_WAVES)
        r0 = new(HIDDEN)
        chain.add_normed(self.w[0]["qkv"].tiles, self.h, qkv_out[0], self.norm_in[0], EPS, resid_out=r0)
        segments.append(chain.build())
        resid = r0
        for i in range(self.layers):
            w = self.w[i]
            chain = DecodeStack(self.fmt, self.m, waves=EXECUTOR_WAVES)
            o, act, down, r1 = new(HIDDEN), new(9728), new(HIDDEN), new(HIDDEN)
            chain.add(w["o"].tiles, self.attend.out, o)
            chain.add_normed(w["gate_up"].tiles, resid, act, self.norm_post[i], EPS, delta=o, resid_out=r1,
                             swiglu=True)
            chain.add(w["down"].tiles, act, down)
            r2 = new(HIDDEN)
            if i + 1 < self.layers:
                chain.add_normed(self.w[i + 1]["qkv"].tiles, r1, qkv_out[i + 1], self.norm_in[i + 1], EPS,
                                 delta=down, resid_out=r2)
            else:
                self.logits = new(LM_HEAD[1])
                chain.add_normed(self.lm_head.tiles, r1, self.logits, self.norm_out, EPS, delta=down, resid_out=r2)
            segments.append(chain.build())
            self.seg_keep += [o, act, down, r1, r2]
            resid = r2
        self.segments = segments

        def step():
            segments[0].run()
            for i in range(self.layers):
                q = qkv_norm_rope_to_cache(qkv_out[i], 32, 8, self.q_norm[i], self.k_norm[i], self.cos, self.sin,
                                           self.positions, 1, self.k_cache[i], self.v_cache[i], EPS)
                self.attend(q, self.k_cache[i], self.v_cache[i], self.positions)
                segments[i + 1].run()
        return step

    def executor_one_launch(self, splits=4):
        """The same decode step as ONE executor launch (m = 1): each layer's attention is a stage
        of the chain (DecodeStack.add_attention: head norm + RoPE + cache write, split attention
        and its merge) between qkv and o, so no launch boundary remains inside the step."""
        from kernels.decode_stack import DecodeStack
        new = lambda n: torch.empty((self.m, n), dtype=torch.bfloat16, device="cuda")
        chain = DecodeStack(self.fmt, self.m, waves=EXECUTOR_WAVES)
        qkv, r0 = new(6144), new(HIDDEN)
        chain.add_normed(self.w[0]["qkv"].tiles, self.h, qkv, self.norm_in[0], EPS, resid_out=r0)
        self.one_keep, resid = [qkv, r0], r0
        for i in range(self.layers):
            w = self.w[i]
            att, o, act, down, r1, r2 = new(4096), new(HIDDEN), new(9728), new(HIDDEN), new(HIDDEN), new(HIDDEN)
            chain.add_attention(qkv, 32, 8, self.q_norm[i], self.k_norm[i], self.cos, self.sin, self.positions,
                                self.k_cache[i], self.v_cache[i], att, EPS, splits=splits)
            chain.add(w["o"].tiles, att, o)
            chain.add_normed(w["gate_up"].tiles, resid, act, self.norm_post[i], EPS, delta=o, resid_out=r1,
                             swiglu=True)
            chain.add(w["down"].tiles, act, down)
            if i + 1 < self.layers:
                qkv = new(6144)
                chain.add_normed(self.w[i + 1]["qkv"].tiles, r1, qkv, self.norm_in[i + 1], EPS, delta=down,
                                 resid_out=r2)
            else:
                self.logits1 = new(LM_HEAD[1])
                chain.add_normed(self.lm_head.tiles, r1, self.logits1, self.norm_out, EPS, delta=down, resid_out=r2)
            self.one_keep += [att, o, act, down, r1, r2, qkv]
            resid = r2
        return chain.build()

    def attention_only(self):
        """The step's rope + attention calls alone (the same calls as in the steps above)."""
        from kernels import qkv_norm_rope_to_cache
        qkv = torch.randn(self.m, 6144, device="cuda").to(torch.bfloat16)

        def step():
            for i in range(self.layers):
                q = qkv_norm_rope_to_cache(qkv, 32, 8, self.q_norm[i], self.k_norm[i], self.cos, self.sin,
                                           self.positions, 1, self.k_cache[i], self.v_cache[i], EPS)
                self.attend(q, self.k_cache[i], self.v_cache[i], self.positions)
        return step

    # ---- per projection --------------------------------------------------------------------

    def run(self, which):
        """Every instance of one projection, single calls on resident N(0, 1) inputs."""
        from kernels import qlinear
        linear = qlinear.FORMATS[self.fmt][1]
        for name, tiled, k, sw in self.calls:
            if name == which:
                linear(self.x[k], tiled, swiglu=sw)

    def bytes_alg(self, which=None):
        """Algorithmic bytes: weight codes + scales + M*K*2 (x in) + M*N_out*2 (y out)."""
        total = 0
        for name, t, k, sw in self.calls:
            if which is None or name == which:
                total += t.bytes_moved() + self.m * k * 2 + self.m * (t.rows // 2 if sw else t.rows) * 2
        return total

    def weight_bytes(self, which=None):
        return sum(t.bytes_moved() for name, t, _, _ in self.calls if which is None or name == which)

    def count(self, which):
        return sum(1 for c in self.calls if c[0] == which)


def graph_of(fn):
    fn()  # eager warmup: allocates the ticket counters outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def time_graph(g, reps, warmup):
    """ms per replay over `reps` replays, events on the replaying stream, synced both sides."""
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps


def median_graph_ms(g, reps, warmup, trials=5):
    return statistics.median(time_graph(g, reps, warmup if i == 0 else 1) for i in range(trials))


def stream_floor(nbytes=4 << 30):
    """Best pure-read rate over `nbytes` resident bytes (GB/s), via qlx_stream_read."""
    from kernels import _lib
    buf = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    buf.fill_(1)
    best = 0.0
    for blocks in (2048, 4096, 8192):
        sink = torch.empty(blocks, dtype=torch.int32, device="cuda")

        def run():
            _lib.call("qlx_stream_read", _lib.ptr(buf), nbytes, _lib.ptr(sink), blocks,
                      _lib.stream(buf.device))
        g = graph_of(run)
        ms = median_graph_ms(g, 5, 2, trials=3)
        best = max(best, nbytes / (ms * 1e-3) / 1e9)
    del buf
    torch.cuda.empty_cache()
    return best


def untile(tiled):
    """Row-major bytes of a tile-layout weight (inverse of qlx_tile_rows), on the host."""
    rows, cols = tiled.shape
    b = tiled.contiguous().view(torch.uint8).view(rows, -1)
    width = b.shape[1]
    v = b.reshape(rows // 16, width // 128, 2, 4, 16, 16).permute(0, 4, 1, 2, 3, 5)
    return v.reshape(rows, width).contiguous().view(tiled.dtype).view(rows, cols)


def cpu_model_name():
    """The host CPU's model name with its family / model / stepping numbers (/proc/cpuinfo;
    a virtual machine may report only a short name such as "AMD EPYC"), else lscpu's."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if not ln.strip():
                    break  # first processor only
                key, _, val = ln.partition(":")
                fields[key.strip()] = val.strip()
    except OSError:
        pass
    name = fields.get("model name", "")
    if not name:
        import subprocess
        try:
            out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
            name = next((ln.split(":", 1)[1].strip() for ln in out.splitlines() if ln.startswith("Model name:")), "")
        except (OSError, subprocess.SubprocessError):
            name = platform.processor()
    ids = [f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields]
    return f"{name} ({', '.join(ids)})" if ids else name


def cpu_baseline(stack, reps=5, warmup=2):
    """The reference's torch CPU path -- dequantize (engine/kernels/cuda_fp8.py:1154-1161), then
    F.linear -- timed on the host cores of the GPU box in the same run.

    Every projection of the stack (36 distinct layers + the lm_head: the same synthetic
    weights and activations, copied to host memory in their row-major packed form) runs
    once per step, each on its own resident input; the step is timed `warmup` + `reps`
    times and the median of the last `reps` is reported. Two variants: dequantize + matmul
    per call (the baseline) and the matmul alone on weights dequantized beforehand."""
    sys.path.insert(0, ROOT)
    from oracle import cpu_baseline as cb
    fmt = stack.fmt
    deq, mm = cb.DEQUANT[fmt], cb.matmul
    # the CPU path reads the row-major packed weight: undo the tile relayout on the host
    host = [(untile(t.weight.cpu()), t.scale.cpu(), k) for _, t, k, _ in stack.calls]
    xs = {k: v.cpu() for k, v in stack.x.items()}

    def timed(step):
        runs = []
        for _ in range(warmup + reps):
            t0 = time.perf_counter()
            step()
            runs.append(time.perf_counter() - t0)
        return statistics.median(runs[warmup:])

    def dequant_matmul():
        for q, s, k in host:
            mm(fmt, xs[k], deq(q, s))

    step_s = timed(dequant_matmul)
    weights = [(deq(q, s), k) for q, s, k in host]
    del host

    def matmul_only():
        for w, k in weights:
            mm(fmt, xs[k], w)

    mm_s = timed(matmul_only)
    del weights
    return {
        "value": round(step_s * 1e6, 1), "unit": "us per step", "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"one whole step: torch CPU dequantize + matmul ({fmt}, M={stack.m}) of every projection of "
                   f"the 36 distinct layers and the lm_head, median of {reps} steps after {warmup}"),
        "matmul_only_us": round(mm_s * 1e6, 1),
        "cpu_model": cpu_model_name(), "os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads(),
        "effective_weight_GBps": round(stack.weight_bytes() / step_s / 1e9, 2),
    }


def time_fn(fn, reps, warmup, trials=5):
    """Median over trials of ms per call, `reps` calls between events on the current stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    res = []
    for _ in range(trials):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            fn()
        end.record()
        torch.cuda.synchronize()
        res.append(start.elapsed_time(end) / reps)
    return statistics.median(res)


def timed_step(fn, steps, warmup):
    """us per step of ``fn`` captured once in a HIP graph and replayed (median of 5 trials)."""
    g = graph_of(fn)
    us = median_graph_ms(g, steps, warmup) * 1e3
    del g
    return us


def measure_stack(fmt, m, steps, warmup, breakdown=True, decode_step=True):
    """The decode-step linear stack of one format at batch m, by two product paths: the
    executor (one launch, m <= 16) and a graph of single calls; ``us`` is the path the
    library's whole-step race picks. With ``decode_step``, also the real decode
    step, attention included: through the reference's signatures (the path Engine.generate
    runs) and, where the executor applies, executor launches split at attention."""
    from kernels import decode_tuning
    model = Model(fmt, m, attention=decode_step)
    single = model.linear_step()
    out = {"graph_us": timed_step(single, steps, warmup)}
    out["path"] = "graph"
    if m <= EXECUTOR_NORM_MAX_M:
        chain = model.linear_chain()
        out["executor_us"] = timed_step(chain.run, steps, warmup)
        if chain.failed():
            raise RuntimeError("decode executor: a wait gave up")
        out["executor_launch"] = {"kind": "stack", "grid": chain.grid, "lds": chain.lds, "waves": chain.waves,
                                  "desc_lds": chain.launch.desc_lds >= 0, "pieces": chain.launch.pieces != 0}
        # the library's whole-step race picks the path (graph of single calls is the incumbent)
        out["path"], race = decode_tuning.race_steps({"graph": single, "executor": chain.run}, "graph",
                                                     rounds=5, replays=4)
        out["race_ms"] = {k: round(v, 4) for k, v in race.items()}
        del chain
    us = out["executor_us"] if out["path"] == "executor" else out["graph_us"]
    out.update({"us": us, "weight_GB": model.weight_bytes() / 1e9, "alg_GB": model.bytes_alg() / 1e9})
    out["effective_weight_GBps"] = model.weight_bytes() / (us * 1e-6) / 1e9
    out["alg_GBps"] = model.bytes_alg() / (us * 1e-6) / 1e9
    out["hbm_frac"] = out["alg_GBps"] * 1e9 / PEAK_HBM
    if decode_step:
        ds = {"engine_path_us": round(timed_step(model.engine_step(), steps, warmup), 2)}
        ds["engine_path_add_norm"] = getattr(model, "engine_choice", "separate")
        ds["attention_splits"] = model.attend.splits
        if m <= EXECUTOR_NORM_MAX_M:
            step = model.executor_step()
            ds["executor_path_us"] = round(timed_step(step, steps, warmup), 2)
            if any(seg.failed() for seg in model.segments):
                raise RuntimeError("decode step executor: a wait gave up")
            del step
            model.segments = None
        if m == 1:
            # the whole step in one executor launch, attention stages inside (the split count
            # per KV head raced like the engine races its attention configs)
            best = None
            for splits in (4, 8):
                chain = model.executor_one_launch(splits)
                us = timed_step(chain.run, steps, warmup)
                if chain.failed():
                    raise RuntimeError("one-launch decode step: a wait gave up")
                if best is None or us < best[0]:
                    best = (us, splits)
                del chain
            ds["executor_one_launch_us"] = round(best[0], 2)
            ds["executor_one_launch_splits"] = best[1]
        ds["rope_and_attention_alone_us"] = round(timed_step(model.attention_only(), steps, warmup), 2)
        ds["context_keys"] = CTX + 1
        out["decode_step"] = ds
    if breakdown:
        # single calls of each projection over >= 1 GiB of distinct weights (the Infinity Cache
        # serves none of them)
        per = {}
        for name, _, _ in PROJ + [LM_HEAD]:
            r = measure_projection(fmt, name, m, max(3, steps // 2))
            per[name] = {"us": r["us"], "alg_MB": r["alg_MB"], "GBps": r["GBps"]}
            torch.cuda.empty_cache()
        out["per_projection"] = per
    return model, out


def measure_one_launch(fmt, steps, warmup):
    """The real decode step (m = 1, 513 keys) as one executor launch with its attention stages,
    for a kernel-trace profile of that launch: the split count raced over 4 and 8 as in
    measure_stack, then the winner timed again. No other path runs, so the profile's
    attention-instance launches are this step's."""
    model = Model(fmt, 1, attention=True)
    best = None
    for splits in (4, 8):
        chain = model.executor_one_launch(splits)
        us = timed_step(chain.run, steps, warmup)
        if chain.failed():
            raise RuntimeError("one-launch decode step: a wait gave up")
        if best is None or us < best[0]:
            best = (us, splits)
        del chain
    chain = model.executor_one_launch(best[1])
    us = timed_step(chain.run, steps, warmup)
    out = {"workload": fmt, "us": round(us, 2), "splits": best[1], "raced_us": round(best[0], 2),
           "context_keys": CTX + 1,
           "launch": {"grid": chain.grid, "lds": chain.lds, "waves": chain.waves, "desc_lds": chain.launch.desc_lds >= 0,
                      "attention": bool(chain.launch.attention)}}
    del chain, model
    torch.cuda.empty_cache()
    return out


def measure_projection(fmt, name, m, reps):
    """Single calls of one Qwen3-4B projection in one format at batch m, over enough distinct
    weights to cover >= 1 GiB (so the Infinity Cache serves none of them), replayed as one HIP
    graph: us per call and algorithmic GB/s. For counter profiles of the decode kernel."""
    import math
    from kernels import qlinear
    n, k = {nm: (nn, kk) for nm, nn, kk in PROJ + [LM_HEAD]}[name]
    quant, linear, _ = qlinear.FORMATS[fmt]
    gen = torch.Generator(device="cuda").manual_seed(21)
    w = (torch.randn(n, k, generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
    first = qlinear.prepare(quant(w), fmt)
    del w
    per = first.bytes_moved()
    ws = [first] + [qlinear.Tiled(first.weight.clone(), first.scale.clone(), n, k, fmt)
                    for _ in range(math.ceil((1 << 30) / per) - 1)]
    x = torch.randn(m, k, generator=gen, device="cuda").to(torch.bfloat16)
    sw = name == "gate_up"

    def run():
        for t in ws:
            linear(x, t, swiglu=sw)
    us = timed_step(run, reps, 5) / len(ws)  # steady state: the first replays of a process run slower
    alg = per + m * k * 2 + m * (n // 2 if sw else n) * 2
    log(f"{fmt} {name} M={m}: {us:.2f} us per call, {alg / us / 1e3:.0f} GB/s ({len(ws)} weights)")
    return {"fmt": fmt, "projection": name, "m": m, "us": round(us, 2), "alg_MB": round(alg / 1e6, 3),
            "GBps": round(alg / us / 1e3, 1), "weights": len(ws)}


def measure_config1(reps=20, cpu=True):
    """the W8A16 GEMV of the down shape at M = 1 (K = 9728, N = 2560), its
    inputs drawn exactly as specified -- one CPU generator seeded 0: W int8 randint(-127, 128),
    then bf16 scales U(0.001, 0.02), then x bf16 N(0, 1) -- and copied to the GPU; timed as
    single calls over 41 copies of the weight (1.02 GB, past the Infinity Cache) replayed as one
    HIP graph; with the reference's torch CPU dequantize + matmul on the same inputs."""
    import math
    from kernels import qlinear
    g = torch.Generator().manual_seed(0)
    q = torch.randint(-127, 128, (2560, 9728), generator=g).to(torch.int8)
    s = (torch.rand(2560, generator=g) * (0.02 - 0.001) + 0.001).to(torch.bfloat16)
    x = torch.randn(1, 9728, generator=g).to(torch.bfloat16)
    tiled = qlinear.prepare((q.cuda(), s.cuda()), "w8a16")
    per = tiled.bytes_moved()
    copies = math.ceil((1 << 30) / per)
    ws = [tiled] + [qlinear.Tiled(tiled.weight.clone(), tiled.scale.clone(), tiled.rows, tiled.k, "w8a16")
                    for _ in range(copies - 1)]
    xd = x.cuda()

    def run():
        for w in ws:
            qlinear.linear_w8a16(xd, w)
    us = timed_step(run, reps, 2) / len(ws)
    alg = per + 9728 * 2 + 2560 * 2
    out = {"us": round(us, 2), "alg_bytes": alg, "GBps": round(alg / us / 1e3, 1),
           "hbm_frac": round(alg / us / 1e3 / (PEAK_HBM / 1e9), 4),
           "effective_weight_GBps": round(per / us / 1e3, 1), "weight_copies": len(ws)}
    del ws
    if cpu:
        sys.path.insert(0, ROOT)
        from oracle import cpu_baseline as cb
        runs = []
        for _ in range(7):
            t0 = time.perf_counter()
            cb.matmul("w8a16", x, cb.DEQUANT["w8a16"](q, s))
            runs.append(time.perf_counter() - t0)
        cpu_us = statistics.median(runs[2:]) * 1e6
        out["cpu_baseline"] = {"us": round(cpu_us, 1), "unit": "us per call", "cores": torch.get_num_threads(),
                               "kind": "port", "sample": "torch CPU dequantize + matmul on the same inputs, median "
                                                         "of 5 after 2"}
    log(f"config 1 W8A16 GEMV down M=1: {us:.2f} us, {alg / us / 1e3:.0f} GB/s "
        f"({100 * alg / us / 1e3 / (PEAK_HBM / 1e9):.1f} % of 8 TB/s)")
    torch.cuda.empty_cache()
    return out


PEAK_BF16_MFMA = 2.5e15  # dense bf16 MFMA, MI355X


def measure_config4(reps, layers=LAYERS):
    """W4A16 g128 gate_up (2 x 9728 rows, fused SwiGLU) then down, at
    M = 16, 32, 64 (the skinny GEMM), over `layers` distinct weight pairs (1.4 GB, past the
    Infinity Cache) replayed as one HIP graph. Per pair: algorithmic bytes (weights + scales,
    x in, activation out and back in, y out), bf16-equivalent MFMA flops, and both roofline
    fractions (HBM 8 TB/s; dense bf16 MFMA 2.5 PFLOP/s)."""
    from kernels import qlinear
    gen = torch.Generator(device="cuda").manual_seed(4)

    def make(n, k):
        w = (torch.randn(n, k, generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
        return qlinear.prepare(qlinear.quantize_w4(w))
    pairs = [(make(2 * 9728, 2560), make(2560, 9728)) for _ in range(layers)]
    out = {}
    for m in (16, 32, 64):
        x = torch.randn(m, 2560, generator=gen, device="cuda").to(torch.bfloat16)

        def run():
            for gu, dn in pairs:
                qlinear.linear_w4a16(qlinear.linear_w4a16(x, gu, swiglu=True), dn)
        g = graph_of(run)
        us = median_graph_ms(g, reps, 2, trials=3) / layers * 1e3
        del g
        gu, dn = pairs[0]
        alg = gu.bytes_moved() + dn.bytes_moved() + m * 2 * (2560 + 9728 + 9728 + 2560)
        flop = 2 * m * (2 * 9728 * 2560 + 2560 * 9728)
        out[f"M{m}"] = {"us_per_pair": round(us, 2), "alg_MB": round(alg / 1e6, 2),
                        "TBps": round(alg / us / 1e6, 3), "hbm_frac": round(alg / us / 1e6 / 8.0, 4),
                        "TFLOPs": round(flop / us / 1e6, 1), "mfma_frac_bf16": round(flop / us * 1e6 / PEAK_BF16_MFMA, 4)}
        log(f"config 4 M={m}: {us:.1f} us per gate_up+down pair, {alg / us / 1e6:.2f} TB/s, {flop / us / 1e6:.0f} TFLOP/s")
    del pairs
    torch.cuda.empty_cache()
    return out


#: The reference's published H100 times (us) for its own INT8 g64 W8A16 kernel at M=1 on these
#: shapes (NOTES.md:354-360 of the reference): context for the same call on MI355X, not a target.
REF_H100_INT8_US = {"qkv": 9.5, "o": 8.1, "gate_up": 21.0, "down": 12.4, "lm_head": 150.8}


def measure_reference_formats(reps=10):
    """The reference engine's own weight formats through its own calls (cuda_fp8.quantize /
    prepare / matmul and gate_up_swiglu, engine/engine.py:522-532, 881-884, 950-951): INT8 and
    INT4 with an fp16 scale per 64 values in the tiled Prepared layout, at M=1, per projection
    over enough distinct weights to cover >= 1 GiB (up to 36), replayed as one HIP graph. Bytes:
    weight + scales + x in + y out. With the derived M=1 stack, 36 x (qkv + o + gate_up + down) +
    lm_head, and the reference's published H100 INT8 figures beside them."""
    import math
    from kernels import cuda_fp8
    gen = torch.Generator(device="cuda").manual_seed(9)
    out = {}
    for bits in (8, 4):
        res = {}
        for name, n, k in PROJ + [LM_HEAD]:
            per = n * k * (bits / 8) + n * (k // 64) * 2
            count = min(LAYERS, max(1, math.ceil((1 << 30) / per)))
            ws = []
            for _ in range(count):
                w = (torch.randn(n, k, generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
                ws.append(cuda_fp8.prepare(cuda_fp8.quantize(w, bits=bits)))
                del w
            x = torch.randn(1, k, generator=gen, device="cuda").to(torch.bfloat16)
            fn = cuda_fp8.gate_up_swiglu if name == "gate_up" else cuda_fp8.matmul

            def run():
                for p in ws:
                    fn(x, p)
            g = graph_of(run)
            us = median_graph_ms(g, reps, 2, trials=3) / count * 1e3
            del g
            n_out = n // 2 if name == "gate_up" else n
            alg = ws[0].bytes_moved() + 2 * k + 2 * n_out
            res[name] = {"us": round(us, 2), "alg_MB": round(alg / 1e6, 3), "GBps": round(alg / us / 1e3, 1)}
            del ws
            torch.cuda.empty_cache()
        stack_us = LAYERS * sum(res[nm]["us"] for nm, _, _ in PROJ) + res["lm_head"]["us"]
        stack_b = LAYERS * sum(res[nm]["alg_MB"] for nm, _, _ in PROJ) + res["lm_head"]["alg_MB"]
        res["stack_M1_us"] = round(stack_us, 1)
        res["stack_M1_GBps"] = round(stack_b / stack_us * 1e3, 1)
        if bits == 8:
            res["reference_h100_us"] = dict(REF_H100_INT8_US, stack_M1=round(
                LAYERS * sum(REF_H100_INT8_US[nm] for nm, _, _ in PROJ) + REF_H100_INT8_US["lm_head"], 1))
        out[f"int{bits}_g64"] = res
        log(f"reference formats int{bits} g64 M=1 (cuda_fp8.matmul): " +
            ", ".join(f"{nm} {res[nm]['us']:.1f} us" for nm in ("qkv", "o", "gate_up", "down", "lm_head")) +
            f"; stack {stack_us:.0f} us")
    return out


#: Decode attention cases (Qwen3-4B: 8 KV heads x 4 query heads, head_dim 128): batch, cache
#: capacity, live keys. Batch 32 at 576 keys is config 5's last step (prompt 512 + 64 tokens).
ATTENTION_CASES = ((1, 4096, 4096), (1, 32768, 32768), (32, 640, 576))


def measure_attention(reps=10):
    """The QKV consumer and decode attention of a Qwen3-4B decode step (the path after qkv):
    ``qkv_norm_rope_to_cache`` at 1 and 32 rows, and ``DecodeAttention`` at ATTENTION_CASES.
    Each is replayed over enough distinct caches (up to one per layer) to cover >= 1 GiB, so
    the Infinity Cache serves nothing hot. Algorithmic bytes of attention: the live K and V
    (live x 8 heads x 128 x 2 bytes each, per sequence) plus q in and the output."""
    import math
    from kernels import DecodeAttention, qkv_norm_rope_to_cache
    gen = torch.Generator(device="cuda").manual_seed(11)
    out = {}
    for batch, cap, live in ATTENTION_CASES:
        per_layer = batch * 8 * cap * 128 * 2 * 2
        n = min(LAYERS, max(1, math.ceil((1 << 30) / per_layer)))
        caches = [(torch.randn(batch, 8, cap, 128, generator=gen, device="cuda").bfloat16(),
                   torch.randn(batch, 8, cap, 128, generator=gen, device="cuda").bfloat16()) for _ in range(n)]
        q = torch.randn(batch, 32 * 128, generator=gen, device="cuda").bfloat16()
        pos = torch.tensor([live - 1], dtype=torch.int32, device="cuda")
        att = DecodeAttention(batch, 8, 4, 128, cap, "cuda")

        def run():
            for k, v in caches:
                att(q, k, v, pos)
        g = graph_of(run)
        us = median_graph_ms(g, reps, 2, trials=3) / n * 1e3
        del g
        alg = batch * 8 * live * 128 * 2 * 2 + 2 * q.numel() * 2
        key = f"B{batch}_ctx{live}"
        out[key] = {"us": round(us, 2), "alg_MB": round(alg / 1e6, 3), "GBps": round(alg / us / 1e3, 1),
                    "hbm_frac": round(alg / us / 1e3 / (PEAK_HBM / 1e9), 4), "splits": att.splits,
                    "kernel": f"attn_kernel<1, false> (grid {batch * 8} x {att.splits})"}
        log(f"decode attention batch {batch}, {live} live keys: {us:.2f} us, {alg / us / 1e3:.0f} GB/s "
            f"({att.splits} splits)")
        del caches
        torch.cuda.empty_cache()
    # The reference's CPU path for the same call (engine/engine.py:988-1005, its fallback: the
    # group's query heads as query positions against the whole cache with a live-key mask),
    # torch on the host cores, batch 1 at 4096 keys, median of 5 after 2.
    import torch.nn.functional as F
    kc = torch.randn(1, 8, 4096, 128).bfloat16()
    vc = torch.randn(1, 8, 4096, 128).bfloat16()
    qc = torch.randn(1, 8, 4, 128).bfloat16()
    mask = torch.ones(4096, dtype=torch.bool)
    times = []
    for i in range(7):
        t0 = time.perf_counter()
        F.scaled_dot_product_attention(qc, kc, vc, attn_mask=mask.view(1, 1, 1, -1))
        if i >= 2:
            times.append(time.perf_counter() - t0)
    out["cpu_baseline_B1_ctx4096"] = {"us": round(statistics.median(times) * 1e6, 1), "kind": "port",
                                      "cores": torch.get_num_threads(),
                                      "sample": "torch CPU scaled_dot_product_attention as the reference's fallback "
                                                "calls it, batch 1, 4096 keys, median of 5 after 2"}
    for rows in (1, 32):
        cap = 1024
        n = LAYERS
        qkv = torch.randn(rows, 6144, generator=gen, device="cuda").bfloat16()
        qn = torch.randn(128, generator=gen, device="cuda").bfloat16()
        kn = torch.randn(128, generator=gen, device="cuda").bfloat16()
        ang = torch.randn(cap, 128, generator=gen, device="cuda")
        cos, sin = ang.cos().bfloat16(), ang.sin().bfloat16()
        positions = torch.tensor([700], dtype=torch.int32, device="cuda")
        caches = [(torch.zeros(rows, 8, cap, 128, device="cuda", dtype=torch.bfloat16),
                   torch.zeros(rows, 8, cap, 128, device="cuda", dtype=torch.bfloat16)) for _ in range(n)]

        def run():
            for k, v in caches:
                qkv_norm_rope_to_cache(qkv, 32, 8, qn, kn, cos, sin, positions, 1, k, v, 1e-6)
        g = graph_of(run)
        us = median_graph_ms(g, reps, 2, trials=3) / n * 1e3
        del g, caches
        alg = rows * (6144 + 4096 + 2048) * 2 + 2 * 256 * 2
        out[f"norm_rope_rows{rows}"] = {"us": round(us, 2), "alg_KB": round(alg / 1e3, 1)}
        log(f"qkv head norm + RoPE + cache write, {rows} rows: {us:.2f} us")
    torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="fp8", choices=["fp8", "w4a16", "w8a16"])
    ap.add_argument("--m", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--quick", action="store_true", help="headline stack only")
    ap.add_argument("--only-config4", action="store_true",
                    help="only BASELINE config 4 (W4 gate_up+SwiGLU then down, M = 16, 32, 64): one JSON line "
                         "of its figures, for profiling the skinny GEMM (not the driver's line)")
    ap.add_argument("--only-attention", action="store_true",
                    help="only the QKV consumer and decode attention figures: one JSON line, for profiling "
                         "(not the driver's line)")
    ap.add_argument("--only-projection", choices=[n for n, _, _ in PROJ] + [LM_HEAD[0]],
                    help="only single calls of one projection (--workload, --m) over >= 1 GiB of distinct "
                         "weights: one JSON line, for counter profiles (not the driver's line)")
    ap.add_argument("--only-decode-step", action="store_true",
                    help="only the one-launch decode step (--workload, m = 1, attention stages inside): one "
                         "JSON line, for kernel-trace profiles of that launch (not the driver's line)")
    ap.add_argument("--only-reference-formats", action="store_true",
                    help="only the reference formats' cuda_fp8.matmul figures: one JSON line (not the driver's line)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py runs on exactly one GPU: this build has no multi-GPU path "
              "(the projections would shard column- and row-parallel, one process per GPU).", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X GPU", file=sys.stderr)
        sys.exit(2)
    from kernels import _lib
    _lib.lib()
    torch.backends.cuda.matmul.allow_tf32 = False
    if args.only_config4:
        print(json.dumps({"config4_w4_gate_up_swiglu_down": measure_config4(max(3, args.steps // 4))}), flush=True)
        return
    if args.only_projection:
        print(json.dumps({"single_calls": measure_projection(args.workload, args.only_projection, args.m,
                                                             max(3, args.steps))}), flush=True)
        return
    if args.only_decode_step:
        print(json.dumps({"decode_step_one_launch": measure_one_launch(args.workload, args.steps, args.warmup)}),
              flush=True)
        return
    if args.only_reference_formats:
        print(json.dumps({"reference_formats_cuda_fp8_matmul": measure_reference_formats(max(3, args.steps // 2))}),
              flush=True)
        return
    if args.only_attention:
        print(json.dumps({"qkv_consumer_and_decode_attention": measure_attention(max(3, args.steps // 2))}),
              flush=True)
        return

    model, head = measure_stack(args.workload, args.m, args.steps, args.warmup, breakdown=not args.quick,
                                decode_step=not args.quick)
    log(f"{args.workload} M={args.m}: {head['us']:.1f} us/step ({head['path']}; graph {head['graph_us']:.1f}, "
        f"executor {head.get('executor_us', float('nan')):.1f}), "
        f"{head['effective_weight_GBps']:.0f} GB/s weights, {100 * head['hbm_frac']:.1f}% of 8 TB/s")
    if "decode_step" in head:
        log(f"{args.workload} M={args.m} decode step with attention: {head['decode_step']}")

    fmt_name = {'fp8': 'FmtFP8', 'w4a16': 'FmtW4', 'w8a16': 'FmtW8'}[args.workload]
    if head["path"] == "executor":
        # The whole linear stack is one launch of the executor: its algorithmic bytes over its time.
        el = head["executor_launch"]
        kname = f"stack_kernel<{fmt_name}, {el['waves']}, {str(el['desc_lds']).lower()}, {str(el['pieces']).lower()}>"
        roofline = {
            "bound": "hbm", "achieved": round(head["alg_GBps"], 1), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
            "frac": round(head["hbm_frac"], 4),
            "traffic": profiled_traffic(args.workload, args.m, el["kind"]),
            "kernel": f"{kname} (the whole linear stack with its norm stages, M={args.m})",
            "us_per_launch": round(head["us"], 2), "alg_MB_per_launch": round(head["alg_GB"] * 1e3, 3),
        }
    else:
        # The fused gate_up+SwiGLU projection (the largest share of the step's bytes),
        # averaged over its 36 launches in one graph.
        dom = head.get("per_projection", {}).get("gate_up")
        if dom is None:
            gp = graph_of(lambda: model.run("gate_up"))
            t = median_graph_ms(gp, max(3, args.steps // 2), 2, trials=3) / model.count("gate_up")
            b = model.bytes_alg("gate_up") / model.count("gate_up")
            dom = {"us": t * 1e3, "alg_MB": b / 1e6, "GBps": b / (t * 1e-3) / 1e9}
        roofline = {
            "bound": "hbm", "achieved": round(dom["GBps"], 1), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
            "frac": round(dom["GBps"] * 1e9 / PEAK_HBM, 4), "traffic": profiled_traffic(args.workload, args.m),
            "kernel": f"gemm_kernel<{fmt_name}, ..., SwiGLU> (gate_up 2560->2x9728, M={args.m})",
            "us_per_launch": round(dom["us"], 2), "alg_MB_per_launch": round(dom["alg_MB"], 3),
        }

    extra = {}
    # the stream read also calibrates rocprofv3's FETCH_SIZE (a known byte count)
    extra["stream_floor_GBps"] = round(stream_floor(1 << 30 if args.quick else 4 << 30), 1)
    extra["stack_frac_of_stream_floor"] = round(head["alg_GBps"] / extra["stream_floor_GBps"], 4)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(model)
        log(f"cpu baseline {args.workload} M={args.m}: {cpu['value'] / 1e3:.1f} ms per step, matmul only "
            f"{cpu['matmul_only_us'] / 1e3:.1f} ms ({cpu['cores']} threads, {cpu['cpu_model']})")
    del model
    torch.cuda.empty_cache()
    if not args.quick:
        extra["config1_w8a16_gemv_down_m1"] = measure_config1(max(5, args.steps), cpu=not args.no_cpu)
        # BASELINE configs 2, 3 and 5: the other formats and batches. Per projection (single
        # calls, 36 distinct weights per projection in one graph): FP8 W8A8 at M = 1, 8; W4A16 at
        # M = 1, 4, 8 with the lm_head. Stacks and decode steps: each format at batch 1 and 32.
        per_cfg = {"config2_fp8_w8a8": {}, "config3_w4a16": {}}
        if args.workload == "fp8" and args.m == 1 and "per_projection" in head:
            per_cfg["config2_fp8_w8a8"]["M1"] = head["per_projection"]
        runs = [("w4a16", 1), ("w8a16", 1), ("w4a16", 4), ("fp8", 8), ("w4a16", 8),
                ("fp8", 32), ("w4a16", 32), ("w8a16", 32)]
        for fmt, m in runs:
            if (fmt, m) == (args.workload, args.m):
                continue
            per_proj = fmt != "w8a16" and m <= 8
            st, res = measure_stack(fmt, m, max(5, args.steps // 2), 2, breakdown=per_proj,
                                    decode_step=m in (1, 32))
            if per_proj:
                per = res.pop("per_projection")
                per_cfg["config2_fp8_w8a8" if fmt == "fp8" else "config3_w4a16"][f"M{m}"] = per
            if (fmt, m) == ("w4a16", 1) and not args.no_cpu:
                res["cpu_baseline"] = cpu_baseline(st)
                log(f"cpu baseline w4a16 M=1: {res['cpu_baseline']['value'] / 1e3:.1f} ms per step "
                    f"({res['cpu_baseline']['cores']} threads)")
            if m != 4:
                extra[f"{fmt}_M{m}_stack"] = {k: (round(v, 4 if k == "hbm_frac" else 2) if isinstance(v, float) else v)
                                              for k, v in res.items()}
            log(f"{fmt} M={m}: {res['us']:.1f} us/step ({res['path']}), {100 * res['hbm_frac']:.1f}% of 8 TB/s"
                + (f"; decode step {res['decode_step']}" if "decode_step" in res else ""))
            del st
            torch.cuda.empty_cache()
        extra["per_projection_single_calls"] = per_cfg
        extra["config4_w4_gate_up_swiglu_down"] = measure_config4(max(3, args.steps // 4))
        extra["qkv_consumer_and_decode_attention"] = measure_attention(max(3, args.steps // 2))
        extra["reference_formats_cuda_fp8_matmul"] = measure_reference_formats(max(3, args.steps // 2))

    line = {
        "metric": METRIC,
        "value": round(head["us"], 2),
        "unit": "us",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us"] / 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"fp8": "fp8e4m3", "w4a16": "int4xbf16", "w8a16": "int8xbf16"}[args.workload],
        "data": "synthetic (seeded N(0,0.02) weights quantized on device, N(0,1) hidden state, RMSNorm weights "
                "1+0.1N(0,1))",
        "config": {
            "workload": f"Qwen3-4B decode-step linear stack, {args.workload}: 36 layers x (rmsnorm -> qkv, o, "
                        f"residual + rmsnorm -> gate_up+SwiGLU, down) + final norm -> lm_head, one dependent "
                        f"chain; o reads the query columns of qkv where attention sits (the step with "
                        f"attention: extra.decode_step)",
            "m": args.m, "hidden": 2560, "intermediate": 9728, "vocab": 151936, "layers": LAYERS,
            "weight_GB": round(head["weight_GB"], 4), "alg_GB": round(head["alg_GB"], 4),
            "path": head["path"],
        },
        "paths_us": {"graph_of_single_calls": round(head["graph_us"], 2),
                     "executor": round(head["executor_us"], 2) if "executor_us" in head else None},
        "decode_step": head.get("decode_step"),
        "effective_weight_GBps": round(head["effective_weight_GBps"], 1),
        "hbm_frac": round(head["hbm_frac"], 4),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "per_projection": head.get("per_projection"),
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
