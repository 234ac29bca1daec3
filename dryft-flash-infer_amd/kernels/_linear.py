"""Shared host logic of every quantized linear: plan, workspace, tickets, launch.

A config is ``(waves, kw, rw, splits)``: waves per workgroup (4 or 8), waves splitting
one 16-row tile's K range, 16-row tiles per wave, and K slices across workgroups.
``None`` takes the library's default for the shape (``qlx_plan_linear``).
"""

import ctypes

import torch

from . import _lib


def make_plan(fmt, mode, m, n, k, config=None, fit=False, comp=1):
    """A plan from ``config`` (or the library default) with its splits normalised by the
    library (every K slice non-empty); ``fit`` first grows the splits until the LDS fits.
    The library default always fits."""
    plan = _lib.Plan()
    if config is None:  # the library's plan fits as it is (a second activation component may not)
        _lib.check(_lib.lib().qlx_plan_linear(fmt, mode, m, n, k, plan), "plan_linear")
        fit = comp > 1
    else:
        waves, kw, rw, splits = config
        plan.mode, plan.waves, plan.kw, plan.rw, plan.splits = mode, waves, kw, rw, splits
    _lib.check(_lib.lib().qlx_plan_fit(plan, fmt, m, n, k, comp, int(fit)), "plan_fit")
    return plan


def run(fmt, entry, x, n, k, args_before_y, args_after_dims=(), mode=_lib.MODE_BF16, config=None,
        m=None, fit=False, comp=1):
    """Launch ``entry(*args_before_y, y, m, n, k, *args_after_dims, plan, stream)``.

    Returns bf16 ``[m, n]`` (``[m, n/2]`` for SwiGLU) or fp32 planes ``[splits, m, n]``.
    """
    m = x.shape[0] if m is None else m
    device = x.device
    plan = make_plan(fmt, mode, m, n, k, config, fit, comp)
    splits = plan.splits
    if mode == _lib.MODE_PLANES:
        plan.splits = splits
        out = torch.empty((splits, m, n), dtype=torch.float32, device=device)
        plan.workspace = out.data_ptr()
    else:
        width = n // 2 if mode == _lib.MODE_SWIGLU else n
        out = torch.empty((m, width), dtype=torch.bfloat16, device=device)
        if splits > 1:
            work = torch.empty((splits, m, n), dtype=torch.float32, device=device)
            plan.workspace = work.data_ptr()
            count = _lib.lib().qlx_plan_tickets(plan, fmt, m, n, k)
            plan.tickets = _lib.tickets(device, count).data_ptr()
    _lib.call(entry, *args_before_y, _lib.ptr(out), m, n, k, *args_after_dims,
              ctypes.byref(plan), _lib.stream(device))
    return out


def splits_for(fmt, mode, m, n, k, config=None, fit=False, comp=1):
    return make_plan(fmt, mode, m, n, k, config, fit, comp).splits


def run_add_norm(fmt, weight_args, x, n, k, tiled, residual, norm_weight, eps, delta, counter, config=None):
    """``qlx_linear_add_norm``: delta = bf16(x W^T) into ``delta``, then (new residual, normed)
    in the same launch. Split-K workspace and tickets are handled as in ``run``."""
    m = x.shape[0]
    device = x.device
    plan = make_plan(fmt, _lib.MODE_BF16, m, n, k, config, fit=True)
    work = None
    if plan.splits > 1:
        work = torch.empty((plan.splits, m, n), dtype=torch.float32, device=device)
        plan.workspace = work.data_ptr()
        count = _lib.lib().qlx_plan_tickets(plan, fmt, m, n, k)
        plan.tickets = _lib.tickets(device, count).data_ptr()
    res = torch.empty_like(residual)
    normed = torch.empty_like(residual)
    w, ws = weight_args
    _lib.call("qlx_linear_add_norm", fmt, _lib.ptr(w), _lib.ptr(ws), _lib.ptr(x), m, n, k, int(tiled),
              _lib.ptr(residual), _lib.ptr(norm_weight), float(eps), _lib.ptr(delta), _lib.ptr(counter),
              _lib.ptr(res), _lib.ptr(normed), ctypes.byref(plan), _lib.stream(device))
    return res, normed
