"""CPU tests of the boundary: the C-ABI library loads, exports every declared symbol, and
the host-side logic (planner, contract checks, no-CPU-fallback) behaves -- no GPU calls."""

import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qlinear.h")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w[\w\s\*]*?\b(qlx_\w+)\s*\(", text, re.M)))


def test_library_exports_every_header_symbol():
    from kernels import _lib
    lib = _lib.lib()
    names = declared()
    assert len(names) >= 25
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures cover exactly the header"
    assert lib.qlx_abi_version() == 1


def test_library_is_gfx950_only_and_has_no_torch_dependency():
    from kernels import _lib
    import subprocess
    out = subprocess.run(["readelf", "-d", _lib.LIB_PATH], capture_output=True, text=True).stdout
    assert "libtorch" not in out and "libc10" not in out
    assert "libamdhip64" in out


def test_planner_defaults_are_valid_and_fit():
    from kernels import _lib, _linear
    lib = _lib.lib()
    for fmt in range(7):
        for n, k in ((6144, 2560), (2560, 4096), (19456, 2560), (2560, 9728), (151936, 2560)):
            for m in (1, 8, 16, 32, 64):
                p = _lib.Plan()
                assert lib.qlx_plan_linear(fmt, 0, m, n, k, p) == 0, (fmt, n, k, m)
                assert p.waves in (4, 8) and p.waves % p.kw == 0 and p.rw in (1, 2) and p.splits >= 1
                again = _linear.make_plan(fmt, 0, m, n, k, (p.waves, p.kw, p.rw, p.splits))
                assert again.splits == p.splits, "the default plan is already normalised"
                assert lib.qlx_plan_tickets(p, fmt, m, n, k) >= 1


def test_plan_fit_normalises_splits_like_the_reference():
    """cuda_fp8._plan (engine/kernels/cuda_fp8.py:1255-1276): gps = ceil(groups/splitk),
    splitk = ceil(groups/gps)."""
    from kernels import _lib, _linear
    for groups, splitk in ((20, 3), (20, 7), (76, 16), (32, 5), (10, 10), (10, 40)):
        k = 128 * groups
        plan = _linear.make_plan(_lib.FMT_REF8, _lib.MODE_PLANES, 1, 2560, k, (8, 8, 1, splitk))
        s = max(1, min(splitk, groups))
        gps = -(-groups // s)
        assert plan.splits == -(-groups // gps), (groups, splitk, plan.splits)


def test_contract_violations_fail_before_any_launch():
    """Bad shapes and plans return QLX_EINVAL with a message (no GPU needed to reject them)."""
    from kernels import _lib
    import ctypes
    lib = _lib.lib()
    bad = _lib.Plan()
    bad.mode, bad.waves, bad.kw, bad.rw, bad.splits = 0, 4, 3, 1, 1
    rc = lib.qlx_linear_w4a16(None, None, None, None, 1, 256, 512, 0, ctypes.byref(bad), None)
    assert rc == _lib.QLX_EINVAL and "kw" in _lib.last_error()
    good = _lib.Plan()
    assert lib.qlx_plan_linear(_lib.FMT_W4A16, 0, 1, 256, 512, good) == 0
    assert lib.qlx_linear_w4a16(None, None, None, None, 1, 256, 500, 0, ctypes.byref(good), None) == _lib.QLX_EINVAL
    assert lib.qlx_linear_w4a16(None, None, None, None, 65, 256, 512, 0, ctypes.byref(good), None) == _lib.QLX_EINVAL
    assert lib.qlx_quantize_weight(None, None, None, 4, 100, 64, 8, 0, 1, 0, None) == _lib.QLX_EINVAL
    assert lib.qlx_tile_rows(None, None, 17, 128, None) == _lib.QLX_EINVAL
    # skinny GEMM: W4A16/W8A16 only, m <= 64, whole 16-row tiles; NULL pointers; K slices
    # without a workspace
    sk = _lib.Plan()
    assert lib.qlx_plan_skinny(_lib.FMT_INT8, 0, 16, 256, 512, sk) == _lib.QLX_EINVAL
    assert lib.qlx_plan_skinny(_lib.FMT_W4A16, 0, 65, 256, 512, sk) == _lib.QLX_EINVAL
    assert lib.qlx_plan_skinny(_lib.FMT_W4A16, 0, 16, 250, 512, sk) == _lib.QLX_EINVAL
    assert lib.qlx_plan_skinny(_lib.FMT_W8A16, 0, 16, 2560, 9728, sk) == 0 and sk.waves == 4 and sk.splits > 1
    assert lib.qlx_linear_skinny(_lib.FMT_W8A16, None, None, None, None, 16, 2560, 9728, ctypes.byref(sk),
                                 None) == _lib.QLX_EINVAL
    p = 1 << 20
    assert lib.qlx_linear_skinny(_lib.FMT_W8A16, p, p, p, p, 16, 2560, 9728, ctypes.byref(sk), None) == _lib.QLX_EINVAL
    assert "workspace" in _lib.last_error()


def test_python_ops_refuse_cpu_tensors():
    """No CPU fallback: the product path raises instead of computing on the host."""
    from kernels import cuda_fp8, fp8, qlinear
    w = torch.randn(64, 256).to(torch.bfloat16)
    for fn in (lambda: cuda_fp8.quantize(w), lambda: fp8.quantize(w), lambda: qlinear.quantize_w4(w),
               lambda: qlinear.quantize_fp8(w), lambda: qlinear.quantize_w8(w)):
        with pytest.raises(ValueError, match="GPU"):
            fn()


def test_package_mirrors_reference_names():
    import kernels
    from kernels import cuda_fp8, cuda_int8, fp8
    for name in ("quantize", "dequantize", "prepare", "Prepared", "matmul", "matmul_partials", "splits",
                 "gate_up_swiglu", "matmul_add_norm", "add_norm_scratch", "ready", "applicable",
                 "CONFIGS", "SWIGLU_CONFIGS", "ADD_NORM_CONFIGS", "GROUP", "TILED", "_FUSED_ROWS", "_module_for"):
        assert hasattr(cuda_fp8, name), name
    for name in ("quantize", "fp8_matmul", "CONFIGS", "bytes_moved"):
        assert hasattr(fp8, name), name
    for name in ("quantize_activation", "Prepared", "matmul", "matmul_quantized", "add_norm_quant"):
        assert hasattr(cuda_int8, name), name
    for name in ("rms_norm", "add_rms_norm", "add_rms_norm_partials", "swiglu", "swiglu_partials"):
        assert hasattr(kernels, name), name
    assert callable(kernels.swiglu)


def test_oracle_is_not_imported_by_the_product():
    pkg = os.path.join(ROOT, "dryft-flash-infer_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert "import oracle" not in text and "from oracle" not in text, f


def test_decode_stack_contract_on_host():
    """The executor rejects unsupported formats, batch sizes, shapes, overlapping outputs and
    empty chains before any device work."""
    from kernels import _lib
    from kernels.decode_stack import DecodeStack
    import ctypes
    lib = _lib.lib()
    assert lib.qlx_stack_desc_size() >= 128
    out = [ctypes.c_longlong(0), ctypes.byref(_lib.StackLaunch())]

    def build(fmt, m, calls, gpc=1, waves=8):
        arr = (_lib.StackCall * max(len(calls), 1))(*calls)
        return lib.qlx_stack_build(fmt, m, arr, len(calls), waves, gpc, None, None, None, *out)

    ok = _lib.StackCall(1 << 20, 1 << 21, 1 << 22, 1 << 23, 256, 512, _lib.MODE_BF16, 0)
    assert build(_lib.FMT_REF8, 1, [ok]) == _lib.QLX_EINVAL
    assert build(_lib.FMT_W4A16, 17, [ok]) == _lib.QLX_EINVAL
    assert build(_lib.FMT_W4A16, 1, []) == _lib.QLX_EINVAL
    assert build(_lib.FMT_FP8, 1, [ok], gpc=5) == _lib.QLX_EINVAL
    assert build(_lib.FMT_FP8, 1, [ok], waves=6) == _lib.QLX_EINVAL
    assert build(_lib.FMT_FP8, 1, [ok], waves=12) == _lib.QLX_EINVAL
    bad_k = _lib.StackCall(1 << 20, 1 << 21, 1 << 22, 1 << 23, 256, 500, _lib.MODE_BF16, 0)
    assert build(_lib.FMT_W8A16, 1, [bad_k]) == _lib.QLX_EINVAL
    bad_kw = _lib.StackCall(1 << 20, 1 << 21, 1 << 22, 1 << 23, 256, 512, _lib.MODE_BF16, 3)
    assert build(_lib.FMT_W8A16, 1, [bad_kw]) == _lib.QLX_EINVAL
    # two outputs in the same bytes; an input overlapping a later output
    a = _lib.StackCall(1 << 20, 1 << 21, 1 << 22, 1 << 23, 256, 512, _lib.MODE_BF16, 0)
    b = _lib.StackCall(1 << 20, 1 << 21, 1 << 22, (1 << 23) + 64, 256, 512, _lib.MODE_BF16, 0)
    assert build(_lib.FMT_W8A16, 1, [a, b]) == _lib.QLX_EINVAL and "overlap" in _lib.last_error()
    c = _lib.StackCall(1 << 20, 1 << 21, (1 << 23) + 16, 1 << 24, 256, 512, _lib.MODE_BF16, 0)
    assert build(_lib.FMT_W8A16, 1, [a, c]) == _lib.QLX_EINVAL and "writes" in _lib.last_error()
    for fmt, m in (("int8", 1), ("w4a16", 0), ("fp8", 17)):
        with pytest.raises(ValueError):
            DecodeStack(fmt, m)
    with pytest.raises(ValueError):
        DecodeStack("w8a16", 1).build()
    launch = _lib.StackLaunch(256, 1024, 8, -1, 1, 0)
    A, E = 1 << 21, 1 << 22  # arena (256-byte aligned) and error word
    assert lib.qlx_stack_run(_lib.FMT_W4A16, None, 1, launch, A, E, 10, None) == _lib.QLX_EINVAL
    assert lib.qlx_stack_run(_lib.FMT_W4A16, 1 << 20, 1, launch, None, E, 10, None) == _lib.QLX_EINVAL
    assert lib.qlx_stack_run(_lib.FMT_W4A16, 1 << 20, 1, launch, A, None, 10, None) == _lib.QLX_EINVAL
    assert lib.qlx_stack_run(_lib.FMT_W4A16, 1 << 20, 1, None, A, E, 10, None) == _lib.QLX_EINVAL
    assert lib.qlx_stack_run(_lib.FMT_W4A16, 1 << 20, 1, launch, A + 16, E, 10, None) == _lib.QLX_EINVAL
    assert "aligned" in _lib.last_error()
    bad = _lib.StackLaunch(256, 1024, 8, 1000, 1, 0)  # descriptor copy past the LDS
    assert lib.qlx_stack_run(_lib.FMT_W4A16, 1 << 20, 4, bad, A, E, 10, None) == _lib.QLX_EINVAL
    # 6 waves per workgroup; FP8 row maxima past the LDS or misaligned
    for waves, amax_off in ((6, 0), (4, 1020), (4, 8)):
        bad = _lib.StackLaunch(256, 1024, waves, -1, 1, amax_off)
        assert lib.qlx_stack_run(_lib.FMT_FP8, 1 << 20, 1, bad, A, E, 10, None) == _lib.QLX_EINVAL
    # a budget past its limit
    good = _lib.StackLaunch(256, 1024, 4, -1, 1, 0)
    assert lib.qlx_stack_run(_lib.FMT_FP8, 1 << 20, 1, good, A, E, 700000000, None) == _lib.QLX_EINVAL
    # the pieces flag selects the kernel with or without the K-piece reduction: 0 or 1 only
    bad = _lib.StackLaunch(256, 1024, 8, -1, 1, 0, 2)
    assert lib.qlx_stack_run(_lib.FMT_FP8, 1 << 20, 1, bad, A, E, 10, None) == _lib.QLX_EINVAL
    assert "pieces" in _lib.last_error()


def test_selection_api_mirrors_the_reference():
    """gemm.pick_matmul and timing.time_calls keep the reference's signatures
    (engine/kernels/gemm.py:134-135, timing.py:9) and contract checks."""
    import inspect
    from kernels import gemm, timing
    params = list(inspect.signature(gemm.pick_matmul).parameters)
    assert params == ["batch", "every", "reps", "trials", "packed", "use_graph", "family", "quick"]
    sig = inspect.signature(timing.time_calls)
    assert list(sig.parameters) == ["fn", "operands", "reps", "trials", "use_graph"]
    assert sig.parameters["reps"].default == 3 and sig.parameters["trials"].default == 5
    for bad in (dict(operands=[]), dict(operands=[1], reps=0), dict(operands=[1], trials=0)):
        ops = bad.pop("operands")
        with pytest.raises(ValueError):
            timing.time_calls(lambda w: None, ops, **bad)


def test_norm_stage_contract_on_host():
    """The executor's residual + RMSNorm stages are checked before any device work: x must be
    NULL exactly for a norm stage, the delta must be the whole output of an earlier projection,
    the residual may not be memory the chain writes, and m * k must fit one staging pass."""
    from kernels import _lib
    import ctypes
    lib = _lib.lib()
    out = (ctypes.c_longlong(0), _lib.StackLaunch())

    def build(m, calls, norms, waves=8):
        arr = (_lib.StackCall * len(calls))(*calls)
        nrm = (_lib.NormInput * len(norms))(*norms)
        return lib.qlx_stack_build_normed(_lib.FMT_FP8, m, arr, len(calls), nrm, waves, 1, None, None, None,
                                          ctypes.byref(out[0]), ctypes.byref(out[1]))

    W, S, R, NW = 1 << 30, 1 << 31, 1 << 32, 1 << 33
    first = _lib.StackCall(W, S, 1 << 34, 1 << 35, 2560, 2560, _lib.MODE_BF16, 0)  # y = 1 << 35, 2560 wide
    normed = _lib.StackCall(W, S, None, 1 << 36, 256, 2560, _lib.MODE_BF16, 0)
    plain = _lib.NormInput()
    good = _lib.NormInput(R, 1 << 35, NW, None, None, 1e-6, 0)
    # x given for a norm stage
    with_x = _lib.StackCall(W, S, 1 << 34, 1 << 36, 256, 2560, _lib.MODE_BF16, 0)
    assert build(1, [first, with_x], [plain, good]) == _lib.QLX_EINVAL and "x must be NULL" in _lib.last_error()
    # a delta that is not an earlier projection's output
    bad_delta = _lib.NormInput(R, 1 << 37, NW, None, None, 1e-6, 0)
    assert build(1, [first, normed], [plain, bad_delta]) == _lib.QLX_EINVAL and "delta" in _lib.last_error()
    # a residual the chain writes
    bad_resid = _lib.NormInput(1 << 35, None, NW, None, None, 1e-6, 0)
    assert build(1, [first, normed], [plain, bad_resid]) == _lib.QLX_EINVAL and "residual" in _lib.last_error()
    # a token row beyond one staging pass (3 chunks of 8 per thread: k <= 12288 at 8 waves, 6144 at 4)
    wide = _lib.StackCall(W, S, 1 << 34, 1 << 35, 6400, 6400, _lib.MODE_BF16, 0)   # y = 1 << 35, 6400 wide
    wide_normed = _lib.StackCall(W, S, None, 1 << 36, 256, 6400, _lib.MODE_BF16, 0)
    assert build(1, [wide, wide_normed], [plain, good], waves=4) == _lib.QLX_EINVAL
    assert "norm stage" in _lib.last_error()
    # many token rows are fine (several passes), so these pass every host check
    for m, waves in ((5, 8), (16, 8), (3, 4)):
        assert build(m, [first, normed], [plain, good], waves=waves) != _lib.QLX_EINVAL, _lib.last_error()
    # Two layers that reuse one resid_out buffer (separate outputs y): two stages would write the
    # same residual and a later stage could not tell which one it reads.
    H0, H1 = 1 << 38, 1 << 39
    third = _lib.StackCall(W, S, None, 1 << 41, 256, 2560, _lib.MODE_BF16, 0)
    layer1 = _lib.NormInput(R, None, NW, H0, None, 1e-6, 0)
    layer2 = _lib.NormInput(H0, 1 << 35, NW, H0, None, 1e-6, 0)             # writes H0 again
    assert build(1, [first, normed, third], [plain, layer1, layer2]) == _lib.QLX_EINVAL
    assert "resid_out" in _lib.last_error() and "overlap" in _lib.last_error()
    # a stage's resid_out inside another projection's output, and a normed_out overlapping a resid_out
    into_y = _lib.NormInput(R, None, NW, (1 << 35) + 64, None, 1e-6, 0)
    assert build(1, [first, normed], [plain, into_y]) == _lib.QLX_EINVAL and "overlap" in _lib.last_error()
    both = _lib.NormInput(R, None, NW, H0, H0 + 1024, 1e-6, 0)
    assert build(1, [first, normed], [plain, both]) == _lib.QLX_EINVAL and "normed_out" in _lib.last_error()
    # disjoint per-layer buffers pass every host check (and reach the device query)
    layer2_ok = _lib.NormInput(H0, 1 << 35, NW, H1, None, 1e-6, 0)
    status = build(1, [first, normed, third], [plain, layer1, layer2_ok])
    assert status != _lib.QLX_EINVAL, _lib.last_error()


def test_qkv_consumer_and_attention_contract_on_host():
    """The rope and attention entry points reject bad arguments before any launch; the Python
    ops keep the reference's names and refuse CPU tensors; plan_splits follows its rule."""
    import ctypes
    from kernels import _lib, attention, rope
    import kernels
    lib = _lib.lib()
    a = _lib.RopeArgs()
    a.rows, a.n_q, a.n_kv, a.seq_len, a.stride = 2, 32, 8, 3, 6144   # rows not a multiple of seq_len
    assert lib.qlx_qkv_norm_rope(ctypes.byref(a), None) == _lib.QLX_EINVAL and "seq_len" in _lib.last_error()
    a.seq_len, a.qkv, a.planes = 1, 1 << 20, 1 << 20                   # both inputs given
    assert lib.qlx_qkv_norm_rope(ctypes.byref(a), None) == _lib.QLX_EINVAL
    a.planes, a.cos, a.sin, a.positions, a.table_rows = None, 1 << 20, 1 << 20, 1 << 20, 8
    a.q_out, a.q_norm_w, a.k_norm_w, a.k_cache, a.v_cache, a.capacity = (1 << 20,) * 5 + (8,)
    a.q_col, a.k_col, a.v_col = 0, 4096, 5120
    a.stride = 6000                                                     # V heads past the row
    assert lib.qlx_qkv_norm_rope(ctypes.byref(a), None) == _lib.QLX_EINVAL and "columns" in _lib.last_error()
    a.stride, a.k_scale = 6144, 1 << 20                                 # one cache scale only
    assert lib.qlx_qkv_norm_rope(ctypes.byref(a), None) == _lib.QLX_EINVAL
    size = ctypes.c_size_t()
    assert lib.qlx_attention_workspace(1, 8, 4, 1, 1, ctypes.byref(size)) == 0 and size.value == 0
    assert lib.qlx_attention_workspace(2, 8, 4, 3, 16, ctypes.byref(size)) == 0
    assert size.value == 2 * 8 * 16 * 12 * 130 * 4
    p = 1 << 20
    args = [p, p, p, None, None, p, p, None, 0, 1, 8, 4, 128, 1, 4096, 16, 0.088, None]
    assert lib.qlx_decode_attention(*args) == _lib.QLX_EINVAL and "workspace" in _lib.last_error()
    args[12] = 64                                                        # head_dim
    assert lib.qlx_decode_attention(*args) == _lib.QLX_EINVAL and "head_dim" in _lib.last_error()
    args[12], args[13] = 128, 17                                         # 17 tokens x 4 > 64 rows
    assert lib.qlx_decode_attention(*args) == _lib.QLX_EINVAL
    args[13], args[3] = 1, p                                             # k_scale without v_scale
    assert lib.qlx_decode_attention(*args) == _lib.QLX_EINVAL

    for name in ("DecodeAttention", "qkv_norm_rope_to_cache", "qkv_planes_norm_rope_to_cache", "q_norm_rope",
                 "kv_norm_rope_to_cache"):
        assert hasattr(kernels, name), name
    assert hasattr(attention, "plan_splits") and hasattr(attention.DecodeAttention, "tuned")
    # plan_splits: double while the grid is under one workgroup per CU and a split keeps >= 128 keys
    assert attention.plan_splits(4096, 1, 8) == (32, 128) and attention.plan_splits(32768, 1, 8) == (32, 1024)
    assert attention.plan_splits(640, 32, 8) == (1, 640) and attention.plan_splits(640, 1, 8) == (4, 160)
    assert attention.plan_splits(100000, 1, 1)[0] == 64
    qkv = torch.randn(1, 6144).to(torch.bfloat16)
    cos = torch.randn(8, 128).to(torch.bfloat16)
    pos = torch.zeros(1, dtype=torch.int32)
    with pytest.raises(ValueError, match="GPU"):
        rope.q_norm_rope(qkv, 32, torch.ones(128, dtype=torch.bfloat16), cos, cos, pos, 1, 1e-6)


def test_decode_tuning_mirrors_the_reference():
    """kernels.decode_tuning keeps the reference's entry point (engine/kernels/decode_tuning.py:17)
    and its conditions for not racing (checked on the host: no device work happens)."""
    import inspect
    import types
    from kernels import decode_tuning
    assert list(inspect.signature(decode_tuning.tune_output_projection).parameters)[0] == "engine"
    base = dict(graph=object(), draft=False, batch=1, integer_mlp=False, families={"o": "fp8"},
                partial_config={"o": (8, 4, 1, 1, 0)})
    for change in (dict(graph=None), dict(draft=True), dict(batch=17), dict(integer_mlp=True),
                   dict(families={"o": "bf16"}), dict(partial_config={})):
        assert decode_tuning.tune_output_projection(types.SimpleNamespace(**{**base, **change})) is False
    with pytest.raises(ValueError):
        decode_tuning.race_steps({"a": lambda: None}, incumbent="b")
