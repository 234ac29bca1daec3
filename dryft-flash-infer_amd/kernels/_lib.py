"""ctypes binding of ``libqlinear.so`` (declared in ``include/qlinear.h``).

The reference reaches its kernels the same way -- ctypes into a native loader
(engine/kernels/cuda_jit.py:141-289) -- so this module is the MI355X counterpart
of ``cuda_jit``: it loads one prebuilt gfx950 library instead of compiling CUDA at
run time. There is no fallback: without the library every op raises.
"""

import ctypes
import os

import torch  # noqa: F401  (loads the HIP runtime the library then shares)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqlinear.so")

QLX_OK, QLX_EINVAL, QLX_EHIP = 0, -1, -2
MODE_BF16, MODE_PLANES, MODE_SWIGLU = 0, 1, 2
SCALE_F16, SCALE_BF16 = 0, 1
STORE_OFFSET, STORE_SIGNED, STORE_K32 = 0, 1, 2
FMT_W8A16, FMT_W4A16, FMT_FP8, FMT_REF8, FMT_REF4, FMT_FP8WO, FMT_INT8 = range(7)


class Plan(ctypes.Structure):
    """``qlx_plan``: mode, splits, waves, kw, rw, workspace, tickets."""

    _fields_ = [
        ("mode", ctypes.c_int), ("splits", ctypes.c_int), ("waves", ctypes.c_int),
        ("kw", ctypes.c_int), ("rw", ctypes.c_int),
        ("workspace", ctypes.c_void_p), ("tickets", ctypes.c_void_p),
    ]


class StackCall(ctypes.Structure):
    """``qlx_stack_call``: one projection of a decode-step chain."""

    _fields_ = [
        ("w", ctypes.c_void_p), ("w_scale", ctypes.c_void_p), ("x", ctypes.c_void_p), ("y", ctypes.c_void_p),
        ("n", ctypes.c_int), ("k", ctypes.c_int), ("mode", ctypes.c_int), ("kw", ctypes.c_int),
    ]


class StackLaunch(ctypes.Structure):
    """``qlx_stack_launch``: grid, LDS bytes, waves, descriptor LDS offset, lanes, the LDS offset
    of the FP8 row maxima, whether row blocks are cut into K pieces, and whether the chain has
    attention stages."""

    _fields_ = [(f, ctypes.c_int) for f in ("grid", "lds_bytes", "waves", "desc_lds", "lanes", "amax_off", "pieces",
                                            "attention")]


class NormInput(ctypes.Structure):
    _fields_ = [("resid", ctypes.c_void_p), ("delta", ctypes.c_void_p), ("norm_w", ctypes.c_void_p),
                ("resid_out", ctypes.c_void_p), ("normed_out", ctypes.c_void_p), ("eps", ctypes.c_float),
                ("pad", ctypes.c_int)]


class StackAttention(ctypes.Structure):
    """``qlx_stack_attention``: what entry c of an executor chain is -- kind 0 a projection, 1
    an attention stage's splits, 2 their merge -- and the attention stage's parameters."""

    _fields_ = [("kind", ctypes.c_int), ("n_q", ctypes.c_int), ("n_kv", ctypes.c_int), ("splits", ctypes.c_int),
                ("capacity", ctypes.c_int), ("table_rows", ctypes.c_int), ("q_norm_w", ctypes.c_void_p),
                ("k_norm_w", ctypes.c_void_p), ("cos", ctypes.c_void_p), ("sin", ctypes.c_void_p),
                ("positions", ctypes.c_void_p), ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p),
                ("eps", ctypes.c_float), ("scale", ctypes.c_float)]


class RopeArgs(ctypes.Structure):
    """``qlx_rope_args``: the fused QKV head-norm + RoPE + cache write."""

    _fields_ = [("qkv", ctypes.c_void_p), ("planes", ctypes.c_void_p), ("stride", ctypes.c_longlong),
                ("splits", ctypes.c_int), ("rows", ctypes.c_int), ("n_q", ctypes.c_int), ("n_kv", ctypes.c_int),
                ("q_col", ctypes.c_int), ("k_col", ctypes.c_int), ("v_col", ctypes.c_int),
                ("seq_len", ctypes.c_int), ("capacity", ctypes.c_int), ("table_rows", ctypes.c_int),
                ("pos_int64", ctypes.c_int), ("eps", ctypes.c_float),
                ("q_norm_w", ctypes.c_void_p), ("k_norm_w", ctypes.c_void_p), ("cos", ctypes.c_void_p),
                ("sin", ctypes.c_void_p), ("positions", ctypes.c_void_p), ("q_out", ctypes.c_void_p),
                ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p), ("k_scale", ctypes.c_void_p),
                ("v_scale", ctypes.c_void_p), ("k_copy", ctypes.c_void_p), ("v_copy", ctypes.c_void_p)]


_P, _I, _F, _LL = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_longlong
_PLAN = ctypes.POINTER(Plan)
_PI, _PLL = ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_longlong)

#: Every exported entry point and its argument types (the header's declarations).
SIGNATURES = {
    "qlx_last_error": ([], ctypes.c_char_p),
    "qlx_abi_version": ([], _I),
    "qlx_quantize_weight": ([_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P], _I),
    "qlx_dequantize": ([_P, _P, _P, _I, _I, _I, _I, _I, _I, _P], _I),
    "qlx_prepare_ref": ([_P, _P, _I, _I, _I, _I, _P], _I),
    "qlx_row_major_ref": ([_P, _P, _I, _I, _P], _I),
    "qlx_quantize_fp8_weight": ([_P, _P, _P, _I, _I, _I, _P], _I),
    "qlx_quantize_fp8_act": ([_P, _P, _P, _I, _I, _P], _I),
    "qlx_fp8_selfcheck": ([_P, _P], _I),
    "qlx_int8_prepare": ([_P, _P, _I, _I, _P], _I),
    "qlx_quantize_act_int8": ([_P, _P, _P, _P, _P, _I, _I, _P], _I),
    "qlx_plan_linear": ([_I, _I, _I, _I, _I, _PLAN], _I),
    "qlx_plan_tickets": ([_PLAN, _I, _I, _I, _I], _I),
    "qlx_plan_fit": ([_PLAN, _I, _I, _I, _I, _I, _I], _I),
    "qlx_tile_rows": ([_P, _P, _I, _I, _P], _I),
    "qlx_linear_w8a16": ([_P, _P, _P, _P, _I, _I, _I, _I, _PLAN, _P], _I),
    "qlx_linear_w4a16": ([_P, _P, _P, _P, _I, _I, _I, _I, _PLAN, _P], _I),
    "qlx_plan_skinny": ([_I, _I, _I, _I, _I, _PLAN], _I),
    "qlx_linear_skinny": ([_I, _P, _P, _P, _P, _I, _I, _I, _PLAN, _P], _I),
    "qlx_linear_skinny_noalloc": ([_I, _P, _P, _P, _P, _I, _I, _I, _I, _P], _I),
    "qlx_linear_skinny_fp8": ([_P, _P, _P, _P, _P, _I, _I, _I, _PLAN, _P], _I),
    "qlx_linear_fp8_w8a8_q": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _PLAN, _P], _I),
    "qlx_linear_fp8_w8a8": ([_P, _P, _P, _P, _I, _I, _I, _I, _PLAN, _P], _I),
    "qlx_linear_ref": ([_P, _P, _P, _P, _I, _I, _I, _I, _I, _PLAN, _P], _I),
    "qlx_linear_fp8wo": ([_P, _P, _P, _P, _I, _I, _I, _I, _PLAN, _P], _I),
    "qlx_linear_int8": ([_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _PLAN, _P], _I),
    "qlx_linear_add_norm": ([_I, _P, _P, _P, _I, _I, _I, _I, _P, _P, _F, _P, _P, _P, _P, _PLAN, _P], _I),
    "qlx_reduce_planes": ([_P, _P, _LL, _I, _P], _I),
    "qlx_residual_planes": ([_P, _P, _P, _LL, _I, _P], _I),
    "qlx_add_rms_norm": ([_P, _P, _P, _I, _P, _P, _P, _I, _I, _F, _P], _I),
    "qlx_add_norm_quant_int8": ([_P, _P, _P, _I, _P, _P, _P, _P, _I, _I, _F, _P], _I),
    "qlx_add_norm_quant_fp8": ([_P, _P, _P, _I, _P, _P, _P, _P, _P, _I, _I, _F, _P], _I),
    "qlx_swiglu": ([_P, _P, _I, _P, _I, _I, _P], _I),
    "qlx_stack_desc_size": ([], _I),
    "qlx_stack_build": ([_I, _I, ctypes.POINTER(StackCall), _I, _I, _I, _P, _PLAN, _P, _PLL,
                         ctypes.POINTER(StackLaunch)], _I),
    "qlx_stack_build_normed": ([_I, _I, ctypes.POINTER(StackCall), _I, ctypes.POINTER(NormInput), _I, _I, _P,
                                _PLAN, _P, _PLL, ctypes.POINTER(StackLaunch)], _I),
    "qlx_stack_build_step": ([_I, _I, ctypes.POINTER(StackCall), _I, ctypes.POINTER(NormInput),
                              ctypes.POINTER(StackAttention), _I, _I, _P, _PLAN, _P, _PLL, ctypes.POINTER(StackLaunch)],
                             _I),
    "qlx_stack_run": ([_I, _P, _I, ctypes.POINTER(StackLaunch), _P, _P, _LL, _P], _I),
    "qlx_stream_read": ([_P, _LL, _P, _I, _P], _I),
    "qlx_qkv_norm_rope": ([ctypes.POINTER(RopeArgs), _P], _I),
    "qlx_attention_workspace": ([_I, _I, _I, _I, _I, ctypes.POINTER(ctypes.c_size_t)], _I),
    "qlx_decode_attention": ([_P, _P, _P, _P, _P, _P, _P, _P, ctypes.c_size_t, _I, _I, _I, _I, _I, _I, _I, _F, _P],
                             _I),
}

_lib = None


def lib():
    """The loaded library; raises RuntimeError if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                "(there is no CPU or Python fallback for these ops)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        _lib = handle
    return _lib


def last_error():
    return lib().qlx_last_error().decode(errors="replace")


def check(rc, what):
    """Map a status to the reference's conventions: ValueError for contract violations,
    RuntimeError for runtime failures (engine/kernels/cuda_jit.py:43-45)."""
    if rc == QLX_OK:
        return
    msg = f"{what}: {last_error()}"
    if rc == QLX_EINVAL:
        raise ValueError(msg)
    raise RuntimeError(msg)


def call(name, *args):
    check(getattr(lib(), name)(*args), name)


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_device(*tensors):
    """The ops run only on a ROCm device; CPU tensors are a contract violation."""
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError("quantized linear ops need tensors on a ROCm GPU (no CPU path)")
        if t is not None and not t.is_contiguous():
            raise ValueError("tensors must be contiguous")


_tickets = {}


def tickets(device, count):
    """Per-device ticket counters for split-K, zero between calls (kernels reset them)."""
    index = torch.device(device).index or 0
    buf = _tickets.get(index)
    if buf is None or buf.numel() < count:
        size = max(count, 1 << 16)
        buf = torch.zeros(size, dtype=torch.int32, device=device)
        _tickets[index] = buf
    return buf
