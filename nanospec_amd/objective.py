"""CE + KL objective, acceptance length and the handwritten derivative, on HIP.

Drop-in for nanospec/objective.py (reference lines 11-80): the same names
(``LossMetrics``, ``LossActivations``, ``ce_kl_loss``, ``ce_kl_backward``),
the same call signatures, metric fields and derivative contract:

* ``ce_kl_loss(logits, target_logits, prepared, objective)`` returns
  ``(LossMetrics, LossActivations)``; metrics are 0-d fp32 device tensors
  (views of one [6] buffer), nothing synchronises the device.
* ``ce_kl_backward(saved, accumulation_steps=1)`` returns
  dl = (w / acc) [c_ce (p - e_y) + c_kl (p - t)] in the logits dtype -- the
  derivative of the *numerator*, not divided by the denominator.

The arithmetic runs in ``libnanospec_hip.so`` (HIP kernels for gfx950): a
statistics pass over V, a per-row merge, and an emit pass that forms the
acceptance rate and dl together, so no [N, V] probability tensor is ever
stored.  Because accept_len needs both log-normalisers, dl is produced during
the forward at the cost of one extra write, and ``ce_kl_backward`` hands it
over; the saved state holds per-row statistics and that dl buffer instead of
the reference's two fp32 [N, V] probability tensors.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from nanospec_amd import _lib
from nanospec_amd.config import Objective


@dataclass
class LossMetrics:
    """Same fields and properties as the reference (objective.py:11-26)."""

    ce: torch.Tensor
    kl: torch.Tensor
    numerator: torch.Tensor
    denominator: torch.Tensor
    accept_len_sum: torch.Tensor
    accept_len_total: torch.Tensor

    @property
    def loss(self):
        return self.numerator / self.denominator.clamp_min(1e-6)

    @property
    def accept_len(self):
        return self.accept_len_sum / self.accept_len_total.clamp_min(1.0)

    @classmethod
    def from_buffer(cls, buf: torch.Tensor) -> "LossMetrics":
        return cls(*buf.unbind(0))


@dataclass
class LossActivations:
    """What ``ce_kl_backward`` needs (replaces objective.py:29-36's fields
    ``probabilities`` / ``target_probabilities`` by per-row statistics).

    row_stats [N, 8] fp32 = (lse_z, lse_u, ce, kl, accept_rate, z_label, 0, 0).
    dlogits is the derivative emitted during the forward for
    ``accumulation_steps == emitted_steps`` (handed over once, then dropped).
    """

    objective: Objective
    logits: torch.Tensor
    target_logits: torch.Tensor
    weights: torch.Tensor
    target_ids: torch.Tensor
    row_stats: torch.Tensor
    dlogits: torch.Tensor | None = None
    emitted_steps: int = 1


def _slot_inputs(prepared, n: int, device: torch.device):
    """Flatten prepared.{weights, target_ids, valid} ([.., K]) into [N] device tensors."""
    weights, labels, valid = prepared.weights, prepared.target_ids, prepared.valid
    if weights.numel() != n or labels.numel() != n or valid.numel() != n:
        raise ValueError(
            f"prepared tensors must have one entry per logits row ({n}); got weights "
            f"{tuple(weights.shape)}, target_ids {tuple(labels.shape)}, valid {tuple(valid.shape)}"
        )
    k = weights.shape[-1] if weights.dim() > 0 else 1
    w = weights.reshape(-1).to(device=device, dtype=torch.float32).contiguous()
    y = labels.reshape(-1).to(device=device, dtype=torch.int64).contiguous()
    v = valid.reshape(-1).to(device=device, dtype=torch.bool).contiguous()
    return w, y, v.view(torch.uint8), k


@torch.no_grad()
def ce_kl_loss(logits, target_logits, prepared, objective, *, accumulation_steps=1, emit_dlogits=True):
    """Forward objective on HIP (objective.py:49-67).

    ``logits`` / ``target_logits``: [..., K, V] bf16 or fp32 on one device.
    ``prepared``: any object with ``weights`` (fp32), ``target_ids`` (int64) and
    ``valid`` (bool), each [..., K] -- e.g. the reference's PreparedBatch.
    A target id of -100 is F.cross_entropy's ignore_index: that row has no CE term.  Any
    other id outside [0, V) makes the loss NaN (the reference raises; the device cannot).
    Keyword extensions: ``accumulation_steps`` pre-scales the dl emitted with the
    forward (default 1: the reference passes the count to ce_kl_backward only, and a
    power-of-two count there rescales this dl in place); ``emit_dlogits=False`` skips it
    (metrics only).
    """
    o = objective
    if logits.shape != target_logits.shape:
        raise ValueError(f"logits {tuple(logits.shape)} and target {tuple(target_logits.shape)} differ")
    if accumulation_steps < 1:
        raise ValueError("accumulation_steps must be >= 1")
    device = _lib.require_device(logits, target_logits)
    lib = _lib.load()
    vocab = logits.shape[-1]
    z, ldz = _lib.rows_2d(logits, vocab)
    u, ldu = _lib.rows_2d(target_logits, vocab)
    n = z.shape[0]
    w, y, valid, k = _slot_inputs(prepared, n, device)
    metrics = torch.empty(6, dtype=torch.float32, device=device)
    row_stats = torch.empty((n, 8), dtype=torch.float32, device=device)
    dl = torch.empty((n, vocab), dtype=logits.dtype, device=device) if emit_dlogits else None
    ws = _lib.workspace(_lib.NS_WS_LOGITS, n, vocab, 0, device)
    status = lib.ns_ce_kl_logits_fwd(
        _lib.ptr(z), _lib.dtype_code(z), ldz, _lib.ptr(u), _lib.dtype_code(u), ldu,
        _lib.ptr(y), _lib.ptr(w), _lib.ptr(valid), n, vocab, k,
        float(o.ce), float(o.kl), 1.0 / accumulation_steps,
        _lib.ptr(dl), vocab, _lib.ptr(row_stats), _lib.ptr(metrics),
        _lib.ptr(ws), ws.numel(), _lib.stream(device),
    )
    _lib.check(status, "ns_ce_kl_logits_fwd")
    saved = LossActivations(
        o, logits, target_logits, w, y, row_stats,
        dl.view(logits.shape) if dl is not None else None, accumulation_steps,
    )
    return LossMetrics.from_buffer(metrics), saved


@torch.no_grad()
def ce_kl_backward(saved, accumulation_steps=1):
    """dl in the logits dtype (objective.py:70-80).

    The dl the forward emitted (for its ``accumulation_steps``, 1 by default, as
    train.py:291 calls ce_kl_loss) is handed over when the counts match.  When they differ
    by a power of two (the reference passes the count only here, train.py:301), that dl is
    scaled in place, which gives the bits the forward would have emitted for this count.
    Any other count, or a second backward, runs the emit pass again."""
    if saved.dlogits is not None:
        dl, saved.dlogits = saved.dlogits, None
        if accumulation_steps == saved.emitted_steps:
            return dl
        ratio = _lib.pow2_ratio(saved.emitted_steps, accumulation_steps)
        if ratio is not None:
            _lib.scale_inplace(dl, ratio)
            return dl
        del dl
    o = saved.objective
    logits, target = saved.logits, saved.target_logits
    device = _lib.require_device(logits, target)
    vocab = logits.shape[-1]
    z, ldz = _lib.rows_2d(logits, vocab)
    u, ldu = _lib.rows_2d(target, vocab)
    n = z.shape[0]
    dl = torch.empty((n, vocab), dtype=logits.dtype, device=device)
    status = _lib.load().ns_ce_kl_logits_bwd(
        _lib.ptr(z), _lib.dtype_code(z), ldz, _lib.ptr(u), _lib.dtype_code(u), ldu,
        _lib.ptr(saved.target_ids), _lib.ptr(saved.weights), n, vocab,
        float(o.ce), float(o.kl), 1.0 / accumulation_steps,
        _lib.ptr(saved.row_stats), _lib.ptr(dl), vocab, _lib.stream(device),
    )
    _lib.check(status, "ns_ce_kl_logits_bwd")
    return dl.view(logits.shape)
