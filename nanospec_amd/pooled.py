"""Pooled-normalisation tail on HIP: the metric pooling of the training loop
(nanospec/train.py:525-535) and the gradient factor of the optimizer step
(nanospec/shard.py:318-330).

The objective's derivative is that of the *numerator* (not divided by the
denominator), so the reference scales every gradient once per optimizer step by
world_size * accumulation_steps / pooled denominator (0 when nothing was
supervised).  ``pooled_tail`` sums LossMetrics buffers in a fixed order and
returns loss, accept_len, that factor and the pooled denominator as 0-d device
tensors; ``scale_gradients_`` applies the factor in place without a host sync.
Across ranks the reference all-reduces the four sums first; on one GPU the
buffers of the micro-batches (or of gathered ranks) are passed together.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from nanospec_amd import _lib


@dataclass
class PooledTail:
    loss: torch.Tensor          # numerator / max(denominator, 1e-6)
    accept_len: torch.Tensor    # accept_len_sum / max(accept_len_total, 1)
    factor: torch.Tensor        # world * accumulation_steps / max(den, 1e-6) if den > 0 else 0
    denominator: torch.Tensor


def _metric_buffer(m) -> torch.Tensor:
    """[6] fp32 view of a LossMetrics (its fields view one buffer) or a [6] tensor."""
    if isinstance(m, torch.Tensor):
        t = m
    else:
        t = torch.stack((m.ce, m.kl, m.numerator, m.denominator, m.accept_len_sum, m.accept_len_total))
    if t.numel() != 6:
        raise ValueError(f"a metrics buffer has 6 entries (got {t.numel()})")
    return t.reshape(6).to(torch.float32)


@torch.no_grad()
def pooled_tail(metrics, world_size: int = 1, accumulation_steps: int = 1) -> PooledTail:
    """``metrics``: one LossMetrics, a sequence of them, or a [count, 6] fp32 tensor."""
    if isinstance(metrics, torch.Tensor) and metrics.dim() == 2:
        buf = metrics.to(torch.float32).contiguous()
    else:
        items = [metrics] if not isinstance(metrics, (list, tuple)) else list(metrics)
        if not items:
            raise ValueError("no metrics to pool")
        buf = torch.stack([_metric_buffer(m) for m in items]).contiguous()
    if buf.shape[-1] != 6:
        raise ValueError(f"metrics buffers are [count, 6] (got {tuple(buf.shape)})")
    device = _lib.require_device(buf)
    out = torch.empty(4, dtype=torch.float32, device=device)
    status = _lib.load().ns_pooled_tail(_lib.ptr(buf), buf.shape[0], int(world_size), int(accumulation_steps),
                                        _lib.ptr(out), _lib.stream(device))
    _lib.check(status, "ns_pooled_tail")
    return PooledTail(*out.unbind(0))


@torch.no_grad()
def scale_gradients_(grads, factor: torch.Tensor):
    """grad.mul_(factor) for each gradient buffer (shard.py:330), factor a 0-d fp32
    device tensor; bf16 buffers are rounded once."""
    lib = _lib.load()
    f = factor.reshape(1).to(torch.float32)
    for g in grads:
        device = _lib.require_device(g, f)
        if not g.is_contiguous():
            raise ValueError("gradient buffers must be contiguous to be scaled in place")
        status = lib.ns_scale_gradient(_lib.ptr(g), _lib.dtype_code(g), g.numel(), _lib.ptr(f), _lib.stream(device))
        _lib.check(status, "ns_scale_gradient")
    return grads
