"""Fused LM head + objective on HIP: the head region of the reference's train().

Reference region (nanospec/train.py:268-312)::

    logits = ops.linear(hidden, lm_head.w)            # train.py:272 (ops.py:34-35)
    logits = logits + markov                          # train.py:276-279
    metrics, saved = ops.ce_kl_loss(logits, target, prepared, o)   # train.py:291
    dl = ops.ce_kl_backward(saved, accumulation_steps)             # train.py:301
    dh = dl @ lm_head.w                               # train.py:302

Here the forward never materialises the [N, V] draft logits: bf16 MFMA tiles of
hidden . W^T feed an online log-softmax over V for both distributions (pass 1),
then a second pass recomputes each tile to form the acceptance rate and dl,
which feeds the dh = dl . W GEMM in the backward.  The metrics keep the
``LossMetrics`` names; dl is available for the Markov-head backward
(train.py:303-307).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from nanospec_amd import _lib
from nanospec_amd.config import Objective
from nanospec_amd.objective import LossMetrics, _slot_inputs


@dataclass
class MarkovFactors:
    """The Markov head in factored form (MarkovHead, layers.py:74-78; train.py:276-279):
    logits += markov_w1[previous] . markov_w2^T.  previous int64 [..., K] (the
    prepared batch's previous ids), w1 / w2 bf16 [V, r] with r % 64 == 0."""

    previous: torch.Tensor
    w1: torch.Tensor
    w2: torch.Tensor


@dataclass
class HeadActivations:
    """State the fused backward needs: per-row statistics, the emitted dl and the
    frozen head weight.  row_stats [N, 8] = (lse_z, lse_u, ce, kl, accept_rate, z_label, 0, 0)."""

    objective: Objective
    weight: torch.Tensor
    row_stats: torch.Tensor
    dlogits: torch.Tensor | None
    accumulation_steps: int
    shape: tuple
    markov: MarkovFactors | None = None


def _bf16_rows(t: torch.Tensor, cols: int, name: str):
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16 (got {t.dtype})")
    return _lib.rows_2d(t, cols)


@torch.no_grad()
def lm_head_ce_kl_loss(hidden, lm_head_weight, target_logits, prepared, objective, *, markov_logits=None,
                       markov=None, accumulation_steps=1, emit_dlogits=True):
    """Fused forward: LM-head projection (+ Markov addend) and the CE + KL + accept objective.

    hidden [..., K, d] bf16; lm_head_weight [V, d] bf16; target_logits [..., K, V]
    bf16 or fp32; markov_logits [..., K, V] bf16 or None; prepared has weights,
    target_ids, valid [..., K].  dl is emitted for ``accumulation_steps`` (pass the
    same value to the backward).  ``markov`` (a ``MarkovFactors``) adds the Markov
    head in factored form instead of a dense ``markov_logits`` tensor: it is fused
    into the GEMM as a second K segment, and the backward can form its gradients.
    """
    o = objective
    if accumulation_steps < 1:
        raise ValueError("accumulation_steps must be >= 1")
    vocab, d = lm_head_weight.shape
    device = _lib.require_device(hidden, lm_head_weight, target_logits, markov_logits)
    lib = _lib.load()
    h, ldh = _bf16_rows(hidden, d, "hidden")
    w, ldw = _bf16_rows(lm_head_weight, d, "lm_head_weight")
    n = h.shape[0]
    u, ldu = _lib.rows_2d(target_logits, vocab)
    if u.shape[0] != n:
        raise ValueError(f"target_logits has {u.shape[0]} rows, hidden has {n}")
    if markov_logits is not None:
        m, ldm = _bf16_rows(markov_logits, vocab, "markov_logits")
        if m.shape[0] != n:
            raise ValueError(f"markov_logits has {m.shape[0]} rows, hidden has {n}")
    else:
        m, ldm = None, vocab
    if markov is not None and markov_logits is not None:
        raise ValueError("pass either markov_logits or markov factors, not both")
    wts, y, valid, k = _slot_inputs(prepared, n, device)
    metrics = torch.empty(6, dtype=torch.float32, device=device)
    row_stats = torch.empty((n, 8), dtype=torch.float32, device=device)
    dl = torch.empty((n, vocab), dtype=torch.bfloat16, device=device) if emit_dlogits else None
    ws = _lib.workspace(_lib.NS_WS_LMHEAD, n, vocab, d, device)
    tail = (_lib.ptr(u), _lib.dtype_code(u), ldu, _lib.ptr(y), _lib.ptr(wts), _lib.ptr(valid), n, d, vocab, k,
            float(o.ce), float(o.kl), 1.0 / accumulation_steps, _lib.ptr(dl), vocab, _lib.ptr(row_stats),
            _lib.ptr(metrics), _lib.ptr(ws), ws.numel(), _lib.stream(device))
    if markov is None:
        status = lib.ns_lmhead_ce_kl_fwd(_lib.ptr(h), ldh, _lib.ptr(w), ldw, _lib.ptr(m), ldm, *tail)
        _lib.check(status, "ns_lmhead_ce_kl_fwd")
    else:
        prev, w1, ldw1, w2, ldw2, r = _markov_inputs(markov, vocab, n, device)
        status = lib.ns_lmhead_markov_ce_kl_fwd(_lib.ptr(h), ldh, _lib.ptr(w), ldw, _lib.ptr(prev), _lib.ptr(w1),
                                                ldw1, _lib.ptr(w2), ldw2, r, *tail)
        _lib.check(status, "ns_lmhead_markov_ce_kl_fwd")
    shape = tuple(hidden.shape[:-1]) + (vocab,)
    saved = HeadActivations(o, lm_head_weight, row_stats, dl, accumulation_steps, shape, markov)
    return LossMetrics.from_buffer(metrics), saved


def _markov_inputs(markov: MarkovFactors, vocab: int, n: int, device):
    """Flatten and check the factored Markov head's inputs."""
    prev = markov.previous.reshape(-1).to(device=device, dtype=torch.int64).contiguous()
    if prev.numel() != n:
        raise ValueError(f"markov.previous has {prev.numel()} entries, hidden has {n} rows")
    if markov.w1.dim() != 2 or markov.w2.dim() != 2 or markov.w1.shape != markov.w2.shape:
        raise ValueError(f"markov w1 {tuple(markov.w1.shape)} and w2 {tuple(markov.w2.shape)} must both be [V, r]")
    if markov.w1.shape[0] != vocab:
        raise ValueError(f"markov weights have {markov.w1.shape[0]} rows, the vocabulary is {vocab}")
    r = markov.w1.shape[1]
    w1, ldw1 = _bf16_rows(markov.w1, r, "markov.w1")
    w2, ldw2 = _bf16_rows(markov.w2, r, "markov.w2")
    return prev, w1, ldw1, w2, ldw2, r


@torch.no_grad()
def lm_head_linear_backward(dl, lm_head_weight):
    """dh = dl . W_lm (train.py:302) on the split-K MFMA GEMM; bf16 in and out."""
    vocab, d = lm_head_weight.shape
    device = _lib.require_device(dl, lm_head_weight)
    g, ldg = _bf16_rows(dl, vocab, "dl")
    w, ldw = _bf16_rows(lm_head_weight, d, "lm_head_weight")
    n = g.shape[0]
    dh = torch.empty((n, d), dtype=torch.bfloat16, device=device)
    ws = _lib.workspace(_lib.NS_WS_LMHEAD_BWD, n, vocab, d, device)
    status = _lib.load().ns_lmhead_bwd(
        _lib.ptr(g), ldg, _lib.ptr(w), ldw, _lib.ptr(dh), d, n, vocab, d,
        _lib.ptr(ws), ws.numel(), _lib.stream(device),
    )
    _lib.check(status, "ns_lmhead_bwd")
    return dh.view(tuple(dl.shape[:-1]) + (d,))


@torch.no_grad()
def lm_head_ce_kl_backward(saved: HeadActivations, accumulation_steps=1, *, return_dlogits=False):
    """dh = dl . W_lm with the dl emitted by the forward.  Returns dh [..., d] bf16
    (and dl [..., V] bf16 when ``return_dlogits``, for the Markov backward)."""
    if saved.dlogits is None:
        raise ValueError("no dl to propagate: the forward ran with emit_dlogits=False, or the backward already ran")
    if accumulation_steps != saved.accumulation_steps:
        raise ValueError(
            f"dl was emitted for accumulation_steps={saved.accumulation_steps}; pass the same value "
            "to lm_head_ce_kl_loss and lm_head_ce_kl_backward"
        )
    dl, saved.dlogits = saved.dlogits, None   # handed over once, so it is freed after dh unless returned
    dh = lm_head_linear_backward(dl, saved.weight)
    dl = dl.view(saved.shape)
    dh = dh.view(saved.shape[:-1] + (saved.weight.shape[1],))
    return (dh, dl) if return_dlogits else dh


@torch.no_grad()
def lm_head_linear(x, lm_head_weight, addend=None):
    """logits = x . W^T (+ addend) in bf16: ops.linear for the LM head (ops.py:34-35;
    train.py:272, 279, 284) on the same MFMA tiles, for callers that need logits."""
    vocab, d = lm_head_weight.shape
    device = _lib.require_device(x, lm_head_weight, addend)
    a, lda_ = _bf16_rows(x, d, "x")
    w, ldw = _bf16_rows(lm_head_weight, d, "lm_head_weight")
    n = a.shape[0]
    if addend is not None:
        b, ldb = _bf16_rows(addend, vocab, "addend")
    else:
        b, ldb = None, vocab
    out = torch.empty((n, vocab), dtype=torch.bfloat16, device=device)
    status = _lib.load().ns_lmhead_linear(
        _lib.ptr(a), lda_, _lib.ptr(w), ldw, _lib.ptr(b), ldb, _lib.ptr(out), vocab, n, vocab, d,
        _lib.stream(device),
    )
    _lib.check(status, "ns_lmhead_linear")
    return out.view(tuple(x.shape[:-1]) + (vocab,))


@torch.no_grad()
def head_step(hidden, lm_head_weight, target_logits, prepared, objective, *, markov_logits=None,
              accumulation_steps=1):
    """The head region of train() (train.py:268-312) on the fused path: returns
    (LossMetrics, dh, dl); dl feeds the Markov-head backward (train.py:303-307)."""
    metrics, saved = lm_head_ce_kl_loss(hidden, lm_head_weight, target_logits, prepared, objective,
                                        markov_logits=markov_logits, accumulation_steps=accumulation_steps)
    dh, dl = lm_head_ce_kl_backward(saved, accumulation_steps, return_dlogits=True)
    return metrics, dh, dl
