"""Ops of the reference's head path (nanospec/ops.py), on HIP.

* ``ce_kl_loss`` / ``ce_kl_backward``: re-exported as in ops.py:12.
* ``linear(x, weight)``: the LM-head projection (ops.py:34-35 as called at
  train.py:272, 279 and 284) on the bf16 MFMA tiles; bf16 in and out.
* ``lm_head_backward(dl, weight)``: ``dl @ lm_head.w`` (train.py:302).
* ``fp8_linear(x, weight, scale)``: block-FP8 projection with ops.py:183-200
  numerics; a non-fp8 weight takes the bf16 ``linear`` path as in the reference.
* ``rms_norm(x, weight, eps)`` / ``rms_norm_backward(dy, saved, weight, weight_grad)``:
  ops.py:48-66 for final_norm (train.py:271, 308-310), with the same
  ``RMSActivations(input, inverse_rms, normalized)`` saved state.

No CPU fallback: unsupported dtypes or shapes raise ``ValueError``.
"""

from __future__ import annotations

import ctypes
from typing import NamedTuple

import torch

from nanospec_amd import _lib
from nanospec_amd.head import lm_head_linear, lm_head_linear_backward
from nanospec_amd.objective import ce_kl_backward as ce_kl_backward  # noqa: F401
from nanospec_amd.objective import ce_kl_loss as ce_kl_loss  # noqa: F401


def linear(x, weight, bias=None):
    if bias is not None:
        raise ValueError("the LM-head projection has no bias")
    return lm_head_linear(x, weight)


def lm_head_backward(dl, weight):
    return lm_head_linear_backward(dl, weight)


@torch.no_grad()
def fp8_linear(x, weight, scale):
    """Reference quantisation, expanded scales, fp32 accumulation, bf16 output."""
    if weight.dtype != torch.float8_e4m3fn:
        return linear(x, weight)
    return _fp8_linear(x, weight, scale, with_lse=False)[0]


@torch.no_grad()
def fp8_teacher_logits(x, weight, scale):
    """Teacher logits from a block-FP8 head (ops.fp8_linear numerics) together with the
    log-sum-exp of each bf16 output row, formed in the GEMM epilogue: a
    ``head.TeacherLogits`` whose first pass reads no teacher logits."""
    from nanospec_amd.head import TeacherLogits

    if weight.dtype != torch.float8_e4m3fn:
        raise ValueError(f"fp8_teacher_logits needs float8_e4m3fn weights (got {weight.dtype})")
    out, lse = _fp8_linear(x, weight, scale, with_lse=True)
    return TeacherLogits(out.reshape(-1, out.shape[-1]), None, lse)


def _fp8_linear(x, weight, scale, with_lse):
    v, d = weight.shape
    if v % 128 or d % 128:
        raise ValueError("Expected checkpoint's 128x128 FP8 weight blocks")
    if x.dtype != torch.bfloat16:
        raise ValueError(f"fp8_linear activations must be bfloat16 (got {x.dtype})")
    device = _lib.require_device(x, weight, scale)
    xr, ldx = _lib.rows_2d(x, d)
    wq = weight.view(torch.uint8)
    wr, ldw = _lib.rows_2d(wq, d)
    sc = scale.to(torch.float32).contiguous()
    if tuple(sc.shape) != (v // 128, d // 128):
        raise ValueError(f"scale must be [{v // 128}, {d // 128}] (got {tuple(sc.shape)})")
    n = xr.shape[0]
    out = torch.empty((n, v), dtype=torch.bfloat16, device=device)
    lse = torch.empty(n, dtype=torch.float32, device=device) if with_lse else None
    ws = _lib.workspace(_lib.NS_WS_FP8, n, v, d, device)
    status = _lib.load().ns_fp8_teacher_logits(
        _lib.ptr(xr), ldx, _lib.ptr(wr), ldw, _lib.ptr(sc), _lib.ptr(out), v, _lib.ptr(lse), n, v, d,
        _lib.ptr(ws), ws.numel(), _lib.stream(device),
    )
    _lib.check(status, "ns_fp8_teacher_logits")
    return out.view(tuple(x.shape[:-1]) + (v,)), lse


@torch.no_grad()
def fp8_quantize_rows(x):
    """(codes uint8 [N, d], scales fp32 [N, d/128]) of the 1x128 activation
    quantisation of ops.py:189-196."""
    n_rows = x.numel() // x.shape[-1]
    d = x.shape[-1]
    device = _lib.require_device(x)
    xr, ldx = _lib.rows_2d(x, d)
    q = torch.empty((n_rows, d), dtype=torch.uint8, device=device)
    xs = torch.empty((n_rows, d // 128), dtype=torch.float32, device=device)
    status = _lib.load().ns_fp8_quantize_rows(_lib.ptr(xr), ldx, n_rows, d, _lib.ptr(q), _lib.ptr(xs),
                                              _lib.stream(device))
    _lib.check(status, "ns_fp8_quantize_rows")
    return q, xs


class RMSActivations(NamedTuple):
    """Saved state of rms_norm, the reference's fields (ops.py:16-19): input [..., d],
    inverse_rms [..., 1] fp32 and normalized = bf16(input * inverse_rms)."""

    input: torch.Tensor
    inverse_rms: torch.Tensor
    normalized: torch.Tensor


def _norm_width(weight, d):
    if weight.dtype != torch.bfloat16 or weight.dim() != 1 or weight.shape[0] != d:
        raise ValueError(f"rms-norm weight must be bfloat16 [{d}] (got {weight.dtype} {tuple(weight.shape)})")
    return weight.contiguous()


@torch.no_grad()
def rms_norm(x, weight, eps):
    """weight * bf16(x * rsqrt(mean(x^2) + eps)) in bf16 (ops.py:48-52)."""
    if x.dtype != torch.bfloat16:
        raise ValueError(f"rms_norm input must be bfloat16 (got {x.dtype})")
    d = x.shape[-1]
    device = _lib.require_device(x, weight)
    w = _norm_width(weight, d)
    xr, ldx = _lib.rows_2d(x, d)
    n = xr.shape[0]
    out = torch.empty((n, d), dtype=torch.bfloat16, device=device)
    normalized = torch.empty_like(out)
    inv = torch.empty((n, 1), dtype=torch.float32, device=device)
    status = _lib.load().ns_rms_norm_fwd(_lib.ptr(xr), ldx, _lib.ptr(w), n, d, float(eps), _lib.ptr(out), d,
                                         _lib.ptr(normalized), d, _lib.ptr(inv), _lib.stream(device))
    _lib.check(status, "ns_rms_norm_fwd")
    lead = tuple(x.shape[:-1])
    return out.view(lead + (d,)), RMSActivations(x, inv.view(lead + (1,)), normalized.view(lead + (d,)))


def norm_args(saved: RMSActivations, weight, weight_grad, dx):
    """The C struct ns_rms_norm_args for a saved rms_norm; returns (struct, keep-alive).
    Every tensor whose pointer goes into the struct must be on dx's device."""
    if _lib.require_device(saved.input, saved.inverse_rms, weight, weight_grad, dx) != dx.device:
        raise ValueError(f"rms-norm operands live on {saved.input.device}, dx on {dx.device}")
    d = saved.input.shape[-1]
    x, ldx = _lib.rows_2d(saved.input, d)
    if x.dtype != torch.bfloat16:
        raise ValueError(f"rms_norm input must be bfloat16 (got {x.dtype})")
    inv = saved.inverse_rms.reshape(-1).to(torch.float32).contiguous()
    if inv.numel() != x.shape[0]:
        raise ValueError(f"inverse_rms has {inv.numel()} rows, the input {x.shape[0]}")
    w = _norm_width(weight, d)
    if weight_grad.dtype != torch.bfloat16 or tuple(weight_grad.shape) != (d,) or not weight_grad.is_contiguous():
        raise ValueError(f"weight_grad must be a contiguous bfloat16 [{d}] buffer")
    args = _lib.RmsNormBwd(x.data_ptr(), ldx, inv.data_ptr(), w.data_ptr(), dx.data_ptr(), d, weight_grad.data_ptr())
    return args, (x, inv, w)


@torch.no_grad()
def rms_norm_backward(dy, saved, weight, weight_grad):
    """dx (bf16) of rms_norm, and weight_grad overwritten with sum(dy * normalized)
    (ops.py:55-66)."""
    d = dy.shape[-1]
    device = _lib.require_device(dy, saved.input, weight, weight_grad)
    g, ldg = _lib.rows_2d(dy, d)
    if g.dtype != torch.bfloat16:
        raise ValueError(f"dy must be bfloat16 (got {g.dtype})")
    n = g.shape[0]
    dx = torch.empty((n, d), dtype=torch.bfloat16, device=device)
    args, keep = norm_args(saved, weight, weight_grad, dx)
    ws = _lib.workspace(_lib.NS_WS_RMS_NORM_BWD, n, 0, d, device)
    status = _lib.load().ns_rms_norm_bwd(_lib.ptr(g), ldg, ctypes.byref(args), n, d, _lib.ptr(ws), ws.numel(),
                                         _lib.stream(device))
    _lib.check(status, "ns_rms_norm_bwd")
    del keep
    return dx.view(saved.input.shape)
