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

import ctypes
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
class TeacherLogits:
    """Teacher logits as their producer left them (train.py:280-290).

    logits [R, V] bf16 or fp32 (R teacher rows, e.g. the verifier's B*S positions);
    rows [N] int64: the teacher row of each objective row -- the gather by
    prepared.teacher_indices (``teacher_rows``), done inside the loads, with no gathered
    copy; None: row t (R == N).  lse [R] fp32: the log-sum-exp of every teacher row when
    its producer formed it (``teacher_logits``): the first pass then reads no teacher."""

    logits: torch.Tensor
    rows: torch.Tensor | None = None
    lse: torch.Tensor | None = None


def teacher_rows(teacher_indices, sequence_length):
    """Flat teacher row of every objective row: b * S + teacher_indices[b, j], the rows
    ``logits.gather(1, teacher_indices)`` selects from [B, S, V] (train.py:285-290)."""
    ti = teacher_indices.to(torch.int64)
    b = ti.shape[0]
    base = torch.arange(b, device=ti.device, dtype=torch.int64).unsqueeze(-1) * int(sequence_length)
    return (ti.reshape(b, -1) + base).reshape(-1).contiguous()


@torch.no_grad()
def teacher_logits(x, lm_head_weight, rows=None):
    """Teacher logits from hidden states through the LM head (train.py:172-173, and
    281-284 with the teacher's last hidden state gathered at teacher_indices): bf16
    x[rows] . W^T, plus their log-sum-exp per row from the GEMM epilogue.  x [R, d] bf16
    (any leading shape), rows [N] int64 or None.  Returns TeacherLogits(logits [N, V],
    None, lse [N])."""
    vocab, d = lm_head_weight.shape
    device = _lib.require_device(x, lm_head_weight, rows)
    a, lda = _bf16_rows(x, d, "x")
    w, ldw = _bf16_rows(lm_head_weight, d, "lm_head_weight")
    if rows is not None:
        r = rows.reshape(-1).to(device=device, dtype=torch.int64).contiguous()
        n, n_rows = r.numel(), a.shape[0]
    else:
        r, n, n_rows = None, a.shape[0], 0
    out = torch.empty((n, vocab), dtype=torch.bfloat16, device=device)
    lse = torch.empty(n, dtype=torch.float32, device=device)
    ws = _lib.workspace(_lib.NS_WS_TEACHER_LOGITS, n, vocab, d, device)
    status = _lib.load().ns_lmhead_teacher_logits(
        _lib.ptr(a), lda, _lib.ptr(r), n_rows, _lib.ptr(w), ldw, _lib.ptr(out), vocab, _lib.ptr(lse), n, vocab, d,
        _lib.ptr(ws), ws.numel(), _lib.stream(device))
    _lib.check(status, "ns_lmhead_teacher_logits")
    return TeacherLogits(out, None, lse)


@dataclass
class _HeadInputs:
    """The fused forward's operands as [rows, cols] views of the caller's tensors (no
    copies), kept so the backward can run pass 2 again for another accumulation_steps."""

    h: torch.Tensor
    ldh: int
    w: torch.Tensor
    ldw: int
    m: torch.Tensor | None
    ldm: int
    factors: tuple | None      # (prev, w1, ldw1, w2, ldw2, r)
    u: torch.Tensor
    ldu: int
    rows: torch.Tensor | None
    lse: torch.Tensor | None
    labels: torch.Tensor
    weights: torch.Tensor


@dataclass
class _Compact:
    """Pass 2 ran on a subset of the rows (``skip_masked_rows``): their dl rows, in order,
    and for each of the N rows its index among them or -1."""

    dl: torch.Tensor       # [m, V] bf16
    index: torch.Tensor    # [N] int64

    def expand(self) -> torch.Tensor:
        """The [N, V] dl: the kept rows in place, zero rows between (ns_copy_rows)."""
        n = self.index.shape[0]
        return _lib.copy_rows(self.dl, self.index, n,
                              torch.empty((n, self.dl.shape[1]), dtype=self.dl.dtype, device=self.dl.device))


@dataclass
class HeadActivations:
    """State the fused backward needs: per-row statistics, the emitted dl, the frozen head
    weight and references to the forward's inputs.  row_stats [N, 8] = (lse_z, lse_u, ce,
    kl, accept_rate, z_label, 0, 0)."""

    objective: Objective
    weight: torch.Tensor
    row_stats: torch.Tensor
    dlogits: torch.Tensor | None
    accumulation_steps: int
    shape: tuple
    markov: MarkovFactors | None = None
    inputs: _HeadInputs | None = None
    compact: _Compact | None = None


def _bf16_rows(t: torch.Tensor, cols: int, name: str):
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16 (got {t.dtype})")
    return _lib.rows_2d(t, cols)


@torch.no_grad()
def lm_head_ce_kl_loss(hidden, lm_head_weight, target_logits, prepared, objective, *, markov_logits=None,
                       markov=None, accumulation_steps=1, emit_dlogits=True, skip_masked_rows=False):
    """Fused forward: LM-head projection (+ Markov addend) and the CE + KL + accept objective.

    hidden [..., K, d] bf16; lm_head_weight [V, d] bf16; target_logits [..., K, V]
    bf16 or fp32, or a ``TeacherLogits`` (teacher rows gathered in the loads, and the
    producer's log-normalisers); markov_logits [..., K, V] bf16 or None; prepared has weights,
    target_ids, valid [..., K].  dl is emitted for ``accumulation_steps`` (a backward
    with another value, or after ``emit_dlogits=False``, runs pass 2 again).  ``saved``
    keeps references to these inputs for that.  ``markov`` (a ``MarkovFactors``) adds the Markov
    head in factored form instead of a dense ``markov_logits`` tensor: it is fused
    into the GEMM as a second K segment, and the backward can form its gradients.

    ``skip_masked_rows=True`` (dense or no Markov addend, plain teacher logits): pass 1 runs on
    every row, then pass 2 and the backward's dh GEMM only on the rows whose dl is not all
    zero -- the supervised ones, and unsupervised ones whose log-normalisers are not finite
    (their dl is the reference's 0 * NaN).  An unsupervised row with finite statistics has
    dl = +0 and contributes (accept_rate * 0) to accept_len, exactly as in the reference, so the
    outputs are those of the full pass (dl, CE/KL sums bit for bit; accept rates may differ in
    their last bit, from a different split of the vocabulary).  Choosing the rows reads their
    count on the host (one synchronisation), so this path cannot be captured into a graph; row
    statistics of the skipped rows carry accept_rate 0.
    """
    o = objective
    if accumulation_steps < 1:
        raise ValueError("accumulation_steps must be >= 1")
    vocab, d = lm_head_weight.shape
    spec = target_logits if isinstance(target_logits, TeacherLogits) else TeacherLogits(target_logits)
    device = _lib.require_device(hidden, lm_head_weight, spec.logits, spec.rows, spec.lse, markov_logits)
    lib = _lib.load()
    h, ldh = _bf16_rows(hidden, d, "hidden")
    w, ldw = _bf16_rows(lm_head_weight, d, "lm_head_weight")
    n = h.shape[0]
    u, ldu = _lib.rows_2d(spec.logits, vocab)
    keep = []
    targs = None
    if spec.rows is not None or spec.lse is not None:
        rows = spec.rows.reshape(-1).to(device=device, dtype=torch.int64).contiguous() if spec.rows is not None \
            else None
        if rows is not None and rows.numel() != n:
            raise ValueError(f"teacher rows has {rows.numel()} entries, hidden has {n} rows")
        lse = spec.lse.reshape(-1).to(torch.float32).contiguous() if spec.lse is not None else None
        if lse is not None and lse.numel() != u.shape[0]:
            raise ValueError(f"teacher lse has {lse.numel()} entries, the teacher logits {u.shape[0]} rows")
        keep = [rows, lse]
        targs = _lib.TeacherArgs(_lib.ptr(rows), u.shape[0] if rows is not None else 0, _lib.ptr(lse))
    if spec.rows is None and u.shape[0] != n:
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
    if skip_masked_rows and markov is None and targs is None and emit_dlogits:
        return _forward_skipping_masked(o, lm_head_weight, hidden.shape, h, ldh, w, ldw, m, ldm, u, ldu, y, wts,
                                        valid, k, accumulation_steps, device)
    metrics = torch.empty(6, dtype=torch.float32, device=device)
    row_stats = torch.empty((n, 8), dtype=torch.float32, device=device)
    dl = torch.empty((n, vocab), dtype=torch.bfloat16, device=device) if emit_dlogits else None
    ws = _lib.workspace(_lib.NS_WS_LMHEAD, n, vocab, d, device)
    tail = (_lib.ptr(u), _lib.dtype_code(u), ldu, ctypes.byref(targs) if targs is not None else None, _lib.ptr(y),
            _lib.ptr(wts), _lib.ptr(valid), n, d, vocab, k, float(o.ce), float(o.kl), 1.0 / accumulation_steps,
            _lib.ptr(dl), vocab, _lib.ptr(row_stats), _lib.ptr(metrics), _lib.ptr(ws), ws.numel(),
            _lib.stream(device))
    factors = None
    if markov is None:
        status = lib.ns_lmhead_ce_kl_fwd(_lib.ptr(h), ldh, _lib.ptr(w), ldw, _lib.ptr(m), ldm, *tail)
        _lib.check(status, "ns_lmhead_ce_kl_fwd")
    else:
        factors = _markov_inputs(markov, vocab, n, device)
        prev, w1, ldw1, w2, ldw2, r = factors
        status = lib.ns_lmhead_markov_ce_kl_fwd(_lib.ptr(h), ldh, _lib.ptr(w), ldw, _lib.ptr(prev), _lib.ptr(w1),
                                                ldw1, _lib.ptr(w2), ldw2, r, *tail)
        _lib.check(status, "ns_lmhead_markov_ce_kl_fwd")
    inputs = _HeadInputs(h, ldh, w, ldw, m, ldm, factors, u, ldu, keep[0] if keep else None,
                         keep[1] if keep else None, y, wts)
    del keep
    shape = tuple(hidden.shape[:-1]) + (vocab,)
    saved = HeadActivations(o, lm_head_weight, row_stats, dl, accumulation_steps, shape, markov, inputs)
    return LossMetrics.from_buffer(metrics), saved


def _forward_skipping_masked(o, lm_head_weight, hidden_shape, h, ldh, w, ldw, m, ldm, u, ldu, y, wts, valid, k,
                             accumulation_steps, device):
    """lm_head_ce_kl_loss(skip_masked_rows=True): pass 1 on every row, pass 2 on the rows whose
    dl is not all zero -- their hidden and Markov rows gathered into compact copies
    (ns_copy_rows), their teacher rows read in place through the teacher-row gather of the
    kernels' loads -- the metrics from every row's statistics.  The compact dl is kept with
    each row's index among the kept ones; the backward runs the dh GEMM on it and scatters dh
    among zero rows, and forms the [N, V] dl (zero rows between) only for a caller that asks
    for it (return_dlogits, final_norm).  At C3 (18,326 of 32,768 rows kept) reading the teacher rows in place instead of
    copying them saved 3.9 of 12.7 ms of copies per step and left pass 2's time unchanged."""
    lib = _lib.load()
    st = _lib.stream(device)
    n = h.shape[0]
    vocab, d = lm_head_weight.shape
    inv_acc = 1.0 / accumulation_steps

    def part(which, hh, ldhh, mm, ldmm, uu, lduu, yy, ww, rows, dl, row_stats, targs=None):
        ws = _lib.workspace(_lib.NS_WS_LMHEAD, rows, vocab, d, device)
        status = lib.ns_lmhead_ce_kl_fwd_part(
            which, _lib.ptr(hh), ldhh, _lib.ptr(w), ldw, _lib.ptr(mm), ldmm, _lib.ptr(uu), _lib.dtype_code(uu), lduu,
            ctypes.byref(targs) if targs is not None else None, _lib.ptr(yy), _lib.ptr(ww), rows, d, vocab,
            float(o.ce), float(o.kl), inv_acc, _lib.ptr(dl), vocab, _lib.ptr(row_stats), _lib.ptr(ws), ws.numel(), st)
        _lib.check(status, "ns_lmhead_ce_kl_fwd_part")

    row_stats = torch.empty((n, 8), dtype=torch.float32, device=device)
    part(_lib.NS_PART_STATS, h, ldh, m, ldm, u, ldu, y, wts, n, None, row_stats)
    # rows whose pass-2 outputs are not all zero: supervised ones, and unsupervised ones whose
    # log-normalisers are not finite (the reference's dl there is 0 * NaN, its accept 0 * NaN)
    need = (valid != 0) | (wts != 0) | ~torch.isfinite(row_stats[:, 0]) | ~torch.isfinite(row_stats[:, 1])
    act = torch.nonzero(need).reshape(-1)   # reads the count on the host: it sizes the compacted pass
    rows = act.numel()
    dl = compact = None
    if rows == n:
        dl = torch.empty((n, vocab), dtype=torch.bfloat16, device=device)
        part(_lib.NS_PART_EMIT, h, ldh, m, ldm, u, ldu, y, wts, n, dl, row_stats)
    else:
        hc = _lib.copy_rows(h, act, rows, torch.empty((rows, d), dtype=h.dtype, device=device))
        mc = _lib.copy_rows(m, act, rows, torch.empty((rows, vocab), dtype=m.dtype, device=device)) \
            if m is not None else None
        # the teacher rows are read in place, gathered in the kernels' loads
        targs = _lib.TeacherArgs(_lib.ptr(act), u.shape[0], None)
        rs = row_stats.index_select(0, act)
        dlc = torch.empty((rows, vocab), dtype=torch.bfloat16, device=device)
        part(_lib.NS_PART_EMIT, hc, d, mc, vocab, u, ldu, y.index_select(0, act), wts.index_select(0, act), rows,
             dlc, rs, targs)
        del hc, mc
        row_stats.index_copy_(0, act, rs)
        row_stats[:, 4].masked_fill_(~need, 0.0)   # (accept_rate * valid) is 0 there either way
        index = torch.full((n,), -1, dtype=torch.int64, device=device)
        index.index_copy_(0, act, torch.arange(rows, dtype=torch.int64, device=device))
        compact = _Compact(dlc, index)   # the [N, V] dl is formed only if a caller asks for it
    metrics = torch.empty(6, dtype=torch.float32, device=device)
    status = lib.ns_objective_metrics(_lib.ptr(row_stats), _lib.ptr(wts), _lib.ptr(valid), n, k, float(o.ce),
                                      float(o.kl), _lib.ptr(metrics), st)
    _lib.check(status, "ns_objective_metrics")
    inputs = _HeadInputs(h, ldh, w, ldw, m, ldm, None, u, ldu, None, None, y, wts)
    shape = tuple(hidden_shape[:-1]) + (vocab,)
    saved = HeadActivations(o, lm_head_weight, row_stats, dl, accumulation_steps, shape, None, inputs, compact)
    return LossMetrics.from_buffer(metrics), saved


def _reemit_dlogits(saved: HeadActivations, accumulation_steps: int) -> torch.Tensor:
    """dl [N, V] bf16 for ``accumulation_steps``: pass 2 of the fused forward again, over the
    kept inputs and row statistics (ns_lmhead_ce_kl_bwd), the bits a forward with that
    accumulation_steps emits (objective.py:70-80 as train.py:301 calls it)."""
    x, o = saved.inputs, saved.objective
    n = x.h.shape[0]
    vocab, d = saved.weight.shape
    device = x.h.device
    dl = torch.empty((n, vocab), dtype=torch.bfloat16, device=device)
    ws = _lib.workspace(_lib.NS_WS_LMHEAD, n, vocab, d, device)
    targs = None
    if x.rows is not None or x.lse is not None:
        targs = _lib.TeacherArgs(_lib.ptr(x.rows), x.u.shape[0] if x.rows is not None else 0, _lib.ptr(x.lse))
    prev, w1, ldw1, w2, ldw2, r = x.factors if x.factors is not None else (None, None, 0, None, 0, 0)
    status = _lib.load().ns_lmhead_ce_kl_bwd(
        _lib.ptr(x.h), x.ldh, _lib.ptr(x.w), x.ldw, _lib.ptr(x.m), x.ldm, _lib.ptr(prev), _lib.ptr(w1), ldw1,
        _lib.ptr(w2), ldw2, r, _lib.ptr(x.u), _lib.dtype_code(x.u), x.ldu,
        ctypes.byref(targs) if targs is not None else None, _lib.ptr(x.labels), _lib.ptr(x.weights), n, d, vocab,
        float(o.ce), float(o.kl), 1.0 / accumulation_steps, _lib.ptr(saved.row_stats), _lib.ptr(dl), vocab,
        _lib.ptr(ws), ws.numel(), _lib.stream(device))
    _lib.check(status, "ns_lmhead_ce_kl_bwd")
    return dl


def _markov_inputs(markov: MarkovFactors, vocab: int, n: int, device):
    """Flatten and check the factored Markov head's inputs: all three on ``device`` (the
    kernels take their raw pointers, so a host tensor is refused here, not copied)."""
    if _lib.require_device(markov.previous, markov.w1, markov.w2) != device:
        raise ValueError(f"markov factors live on {markov.w1.device}, the head's operands on {device}")
    prev = markov.previous.reshape(-1).to(dtype=torch.int64).contiguous()
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


def _grad_rows(t: torch.Tensor, vocab: int, r: int, name: str):
    """A [V, r] bf16 gradient buffer written in place: rows must be unit-stride."""
    if t.dtype != torch.bfloat16 or t.dim() != 2 or tuple(t.shape) != (vocab, r):
        raise ValueError(f"{name} must be bfloat16 [{vocab}, {r}] (got {t.dtype} {tuple(t.shape)})")
    if t.stride(1) != 1 or t.stride(0) < r:
        raise ValueError(f"{name} must have unit-stride rows to be written in place")
    return t, t.stride(0)


def _final_norm_args(final_norm, n, d, device):
    """(struct pointer, dx, keep-alive) for final_norm = (RMSActivations, weight, weight_grad)."""
    from nanospec_amd import ops

    saved, weight, weight_grad = final_norm
    if saved.input.shape[-1] != d or saved.input.numel() // d != n:
        raise ValueError(f"final_norm input {tuple(saved.input.shape)} does not match dh [{n}, {d}]")
    _lib.require_device(saved.input, weight, weight_grad)
    dx = torch.empty((n, d), dtype=torch.bfloat16, device=device)
    args, keep = ops.norm_args(saved, weight, weight_grad, dx)
    return ctypes.byref(args), dx, (args, keep)


@torch.no_grad()
def lm_head_norm_backward(dl, lm_head_weight, final_norm):
    """dh = dl . W_lm (train.py:302) followed by final_norm's backward (train.py:308-310,
    ops.py:55-66) as the dh GEMM's split-K reduction: returns dx [..., d] bf16 and
    overwrites the norm weight's gradient; dh is never stored.  final_norm =
    (RMSActivations from ops.rms_norm, norm weight, norm weight gradient buffer)."""
    vocab, d = lm_head_weight.shape
    device = _lib.require_device(dl, lm_head_weight)
    g, ldg = _bf16_rows(dl, vocab, "dl")
    w, ldw = _bf16_rows(lm_head_weight, d, "lm_head_weight")
    n = g.shape[0]
    args, dx, keep = _final_norm_args(final_norm, n, d, device)
    ws = _lib.workspace(_lib.NS_WS_LMHEAD_NORM_BWD, n, vocab, d, device)
    status = _lib.load().ns_lmhead_norm_bwd(_lib.ptr(g), ldg, _lib.ptr(w), ldw, args, None, d, n, vocab, d,
                                            _lib.ptr(ws), ws.numel(), _lib.stream(device))
    _lib.check(status, "ns_lmhead_norm_bwd")
    del keep
    return dx.view(final_norm[0].input.shape)


@torch.no_grad()
def lm_head_markov_backward(dl, lm_head_weight, markov: MarkovFactors, w1_grad, w2_grad, final_norm=None):
    """The head backward with the factored Markov head (train.py:302-307):
    dh = dl . W_lm; markov_w2.grad = dl^T . w1[previous] (overwritten, as
    ops.linear_backward's copy_, ops.py:38-45); markov_w1.grad.index_add_(previous,
    dl . w2) (accumulated, ops.embedding_backward, ops.py:73-74).  d(previous) stays
    fp32 inside the library and each w1.grad row gets its tokens' sum in token order.
    Returns dh [..., d] bf16, or with ``final_norm`` (as in ``lm_head_norm_backward``)
    dx [..., d] bf16."""
    vocab, d = lm_head_weight.shape
    device = _lib.require_device(dl, lm_head_weight, markov.w1, markov.w2, w1_grad, w2_grad)
    g, ldg = _bf16_rows(dl, vocab, "dl")
    w, ldw = _bf16_rows(lm_head_weight, d, "lm_head_weight")
    n = g.shape[0]
    prev, w1, ldw1, w2, ldw2, r = _markov_inputs(markov, vocab, n, device)
    g1, ldg1 = _grad_rows(w1_grad, vocab, r, "w1_grad")
    g2, ldg2 = _grad_rows(w2_grad, vocab, r, "w2_grad")
    lib = _lib.load()
    if final_norm is not None:
        args, out, keep = _final_norm_args(final_norm, n, d, device)
        dh = None
    else:
        args, keep = None, None
        out = dh = torch.empty((n, d), dtype=torch.bfloat16, device=device)
    nbytes = int(lib.ns_lmhead_markov_bwd_workspace_bytes(n, vocab, d, r))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
    status = lib.ns_lmhead_markov_bwd(
        _lib.ptr(g), ldg, _lib.ptr(w), ldw, _lib.ptr(prev), _lib.ptr(w1), ldw1, _lib.ptr(w2), ldw2, r,
        _lib.ptr(dh), d, args, _lib.ptr(g1), ldg1, _lib.ptr(g2), ldg2, n, vocab, d, _lib.ptr(ws), ws.numel(),
        _lib.stream(device),
    )
    _lib.check(status, "ns_lmhead_markov_bwd")
    del keep
    return out.view(tuple(dl.shape[:-1]) + (d,))


@torch.no_grad()
def lm_head_ce_kl_backward(saved: HeadActivations, accumulation_steps=1, *, return_dlogits=False,
                           markov_grads=None, final_norm=None):
    """dh = dl . W_lm (train.py:301-302).  Returns dh [..., d] bf16 (and dl [..., V] bf16
    when ``return_dlogits``, for the Markov backward).  dl is the one the forward emitted
    when it was emitted for this ``accumulation_steps``, or that dl scaled in place when the
    two counts differ by a power of two (bit-identical to an emission for this count, for
    normal values); otherwise (another count, ``emit_dlogits=False``, or a second backward)
    pass 2 runs again from the saved row statistics, giving the bits a forward with this
    count emits.
    ``markov_grads=(w1_grad, w2_grad)`` with a factored Markov forward also runs the
    Markov-head backward in the same GEMM (``lm_head_markov_backward``).
    ``final_norm=(RMSActivations, norm weight, norm weight grad)`` fuses final_norm's
    backward into the dh reduction and returns dx in place of dh (train.py:308-310)."""
    if accumulation_steps < 1:
        raise ValueError("accumulation_steps must be >= 1")
    dl, saved.dlogits = saved.dlogits, None   # handed over once, so it is freed after dh unless returned
    compact, saved.compact = saved.compact, None
    if accumulation_steps != saved.accumulation_steps and (dl is not None or compact is not None):
        ratio = _lib.pow2_ratio(saved.accumulation_steps, accumulation_steps)
        if ratio is not None:
            # the bits an emission for this count has
            _lib.scale_inplace(compact.dl if compact is not None else dl, ratio)
        else:
            dl = compact = None
    if compact is not None:
        if markov_grads is None and final_norm is None:
            # dh of the rows pass 2 ran on, scattered among the zero rows of the others
            dhc = lm_head_linear_backward(compact.dl, saved.weight)
            n, d = compact.index.shape[0], saved.weight.shape[1]
            dh = _lib.copy_rows(dhc, compact.index, n, torch.empty((n, d), dtype=torch.bfloat16, device=dhc.device))
            dh = dh.view(saved.shape[:-1] + (d,))
            return (dh, compact.expand().view(saved.shape)) if return_dlogits else dh
        dl = compact.expand()
    elif dl is None:
        dl = _reemit_dlogits(saved, accumulation_steps)
    del compact
    if markov_grads is not None:
        if saved.markov is None:
            raise ValueError("markov_grads given, but the forward ran without Markov factors")
        dh = lm_head_markov_backward(dl, saved.weight, saved.markov, *markov_grads, final_norm=final_norm)
    elif final_norm is not None:
        dh = lm_head_norm_backward(dl, saved.weight, final_norm)
    else:
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
              markov=None, markov_grads=None, final_norm=None, accumulation_steps=1, skip_masked_rows=False):
    """The head region of train() (train.py:268-312) on the fused path: returns
    (LossMetrics, dh, dl); dl feeds the Markov-head backward (train.py:303-307).
    With ``markov`` factors and ``markov_grads=(w1_grad, w2_grad)`` that backward runs
    here too, and the gradient buffers are updated in place.  With ``final_norm``
    (RMSActivations, norm weight, norm weight grad) the second value is dx, not dh.
    ``skip_masked_rows``: as in lm_head_ce_kl_loss."""
    metrics, saved = lm_head_ce_kl_loss(hidden, lm_head_weight, target_logits, prepared, objective,
                                        markov_logits=markov_logits, markov=markov,
                                        accumulation_steps=accumulation_steps, skip_masked_rows=skip_masked_rows)
    dh, dl = lm_head_ce_kl_backward(saved, accumulation_steps, return_dlogits=True, markov_grads=markov_grads,
                                    final_norm=final_norm)
    return metrics, dh, dl
