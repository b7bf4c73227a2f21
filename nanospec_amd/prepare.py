"""Objective inputs of every draft slot, on HIP (nanospec/dspark.py:109-144).

``prepare_slots`` is the objective-facing part of the reference's ``prepare``
(dspark.py:116-127, 143): given sampled anchors and their keep flags it builds
labels (``target_ids``), the teacher-forced ``previous`` ids, the prefix-valid
supervision mask, the position weights valid * exp(-slot / gamma) and the
teacher-logit row indices.  Anchor sampling (dspark.py:71-92), positions and the
attention mask are outside the objective path.  The result duck-types the
reference's PreparedBatch for ``ce_kl_loss`` (weights, target_ids, valid).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from nanospec_amd import _lib


@dataclass
class SlotBatch:
    anchors: torch.Tensor
    keep: torch.Tensor
    target_ids: torch.Tensor
    previous: torch.Tensor
    weights: torch.Tensor
    valid: torch.Tensor
    teacher_indices: torch.Tensor


@torch.no_grad()
def prepare_slots(ids, loss_mask, objective, anchors, keep) -> SlotBatch:
    """ids [b, s] int64, loss_mask [b, s] (float, > 0.5 supervised), anchors [b, nb]
    int64 in [0, s), keep [b, nb] bool.  Raises ValueError on an empty sequence
    (dspark.py:112-113)."""
    device = _lib.require_device(ids, loss_mask, anchors, keep)
    b, s = ids.shape
    nb = anchors.shape[1]
    k = objective.block_size
    ids_c = ids.to(torch.int64).contiguous()
    mask_c = loss_mask.to(torch.float32).contiguous()
    anc = anchors.to(torch.int64).contiguous()
    kp = keep.to(torch.bool).contiguous()
    target_ids = torch.empty((b, nb, k), dtype=torch.int64, device=device)
    previous = torch.empty_like(target_ids)
    weights = torch.empty((b, nb, k), dtype=torch.float32, device=device)
    valid = torch.empty((b, nb, k), dtype=torch.bool, device=device)
    teacher_indices = torch.empty((b, nb * k), dtype=torch.int64, device=device)
    status = _lib.load().ns_prepare_slots(
        _lib.ptr(ids_c), _lib.ptr(mask_c), _lib.ptr(anc), _lib.ptr(kp), b, s, nb, k, float(objective.gamma),
        _lib.ptr(target_ids), _lib.ptr(previous), _lib.ptr(weights), _lib.ptr(valid),
        _lib.ptr(teacher_indices), _lib.stream(device),
    )
    _lib.check(status, "ns_prepare_slots")
    return SlotBatch(anc, kp, target_ids, previous, weights, valid, teacher_indices)
