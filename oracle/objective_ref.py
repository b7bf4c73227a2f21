"""CPU restatement (numpy) of nanospec's draft-objective hot path.

TEST INFRASTRUCTURE ONLY.  This module is the parity checker for the HIP
library and the timed CPU baseline of ``bench.py``; the product never calls it.

Every function is a restatement, written from the formulas, of the reference
file:line named in its docstring (paths relative to the reference checkout).
Each function is pinned by an independent check in ``tests/test_oracle.py``:

=========================  ==================================================
function                   pinned by
=========================  ==================================================
row_objective (CE)         torch ``F.cross_entropy`` (fp64); z const -> log V
row_objective (KL)         torch ``F.kl_div`` (experiments/reference.py:67
                           formulation); z == u -> 0
row_objective (accept a)   total-variation identity 1 - |p - t|_1 / 2;
                           z == u -> 1; pure-Python brute force at V <= 64
acceptance_length_counts   hand-computed known answers (all-invalid block,
                           truncation at a gap, a = 1, a = 0); brute force
ce_kl_loss                 torch library loss (cross_entropy + kl_div);
                           den = 0 clamp; empty batch -> accept_len 0;
                           NaN / inf logits against torch's evaluation of
                           objective.py:42-46, 53-60
metrics_from_rows          the tail of ce_kl_loss (same pins); chunked rows
                           equal the whole batch's metrics
ce_kl_backward             torch.autograd on the library loss; rows sum to 0;
                           w = 0 rows are 0; linear in 1/accumulation_steps
lm_head_logits / dhidden   torch fp64 matmul; linearity
markov_logits / backward   torch F.embedding + F.linear forward, torch.autograd
                           for d(previous), d(w2) and the index_add d(w1);
                           hand-worked index_add with repeated ids
slot_preparation           hand-computed known answers; brute-force loops
rms_norm                   fp64 closed form x / sqrt(mean(x^2) + eps)
rms_norm_backward          torch.autograd (fp64) of sum(dy * weight * rms_norm(x))
                           for dx and the weight gradient, with dy correlated with
                           x so the projection (dvar) term carries weight
pooled_tail                hand-computed known answers (den = 0 -> factor 0 and
                           the 1e-6 clamp; accept total 0 -> clamp 1); torch's
                           own evaluation of shard.py:321-327 on fp32 tensors;
                           factor * den == world * acc
scale_gradient             torch products (bit-exact, CPU): fp32 x fp32 factor;
                           bf16 x bf16-cast factor; the device semantics of
                           bf16.mul_(0-d fp32) against torch's device mul_ (GPU)
e4m3 round / fp8_linear    torch ``float8_e4m3fn`` cast; exact products for
                           e4m3-grid inputs with power-of-two scales
bf16_round                 torch ``bfloat16`` cast
=========================  ==================================================

No reference golden vectors exist for this path (the reference has no test
suite), so these library and closed-form checks are the pins.
"""

from __future__ import annotations

import math

import numpy as np

F32_TINY = np.finfo(np.float32).tiny


# ---------------------------------------------------------------------------
# Number formats
# ---------------------------------------------------------------------------


def bf16_round(x) -> np.ndarray:
    """Round float32 values to bfloat16 (round-to-nearest-even); returns float32.

    Same rounding as ``tensor.to(torch.bfloat16)`` used by the reference's bf16
    boundaries (ops.py:200, train.py:287).
    """
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    bits = a.view(np.uint32).astype(np.uint64)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000
    out = rounded.astype(np.uint32).view(np.float32).copy()
    nan = np.isnan(a)
    out[nan] = np.nan
    return out


def bf16_bits(x) -> np.ndarray:
    """bfloat16 bit patterns (uint16) of float32 values, rounded to nearest even."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def _e4m3_table() -> np.ndarray:
    """Values of all 256 OCP e4m3fn codes (bias 7, no infinities, S.1111.111 is NaN)."""
    vals = np.zeros(256, dtype=np.float64)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        exp = (code >> 3) & 0xF
        man = code & 0x7
        if exp == 0xF and man == 0x7:
            vals[code] = np.nan
        elif exp == 0:
            vals[code] = sign * man * 2.0 ** -9
        else:
            vals[code] = sign * (1.0 + man / 8.0) * 2.0 ** (exp - 7)
    return vals


E4M3_VALUES = _e4m3_table()
_POS_CODES = np.arange(0, 127)  # 0x00 .. 0x7E, increasing values 0 .. 448
_POS_VALUES = E4M3_VALUES[_POS_CODES]


def e4m3_encode(x) -> np.ndarray:
    """float -> e4m3fn code (uint8), round-to-nearest-even, inputs already in [-448, 448].

    Same conversion as ``tensor.to(torch.float8_e4m3fn)`` (ops.py:192-196).
    """
    a = np.asarray(x, dtype=np.float64)
    mag = np.abs(a)
    idx = np.clip(np.searchsorted(_POS_VALUES, mag, side="left"), 1, len(_POS_VALUES) - 1)
    lo, hi = _POS_VALUES[idx - 1], _POS_VALUES[idx]
    take_hi = (hi - mag) < (mag - lo)
    tie = (hi - mag) == (mag - lo)
    # ties go to the even code (mantissa lsb 0)
    take_hi = take_hi | (tie & ((_POS_CODES[idx] & 1) == 0))
    code = np.where(take_hi, _POS_CODES[idx], _POS_CODES[idx - 1])
    code = np.where(mag == 0, 0, code)
    # the sign survives rounding to zero (-0 is code 0x80), as in the e4m3fn cast
    code = code.astype(np.uint8) | np.where(np.signbit(a), 0x80, 0).astype(np.uint8)
    return np.where(np.isnan(a), np.uint8(0x7F), code).astype(np.uint8)


def e4m3_decode(codes) -> np.ndarray:
    return E4M3_VALUES[np.asarray(codes, dtype=np.uint8)].astype(np.float32)


# ---------------------------------------------------------------------------
# A1: slot preparation (labels, validity, weights)  dspark.py:116-127, 143
# ---------------------------------------------------------------------------


def slot_weights(valid, gamma: float) -> np.ndarray:
    """w = valid * exp(-slot / gamma); no decay when gamma <= 0 (dspark.py:124-126)."""
    valid = np.asarray(valid)
    k = valid.shape[-1]
    w = valid.astype(np.float32)
    if gamma > 0:
        slot = np.arange(k, dtype=np.float32)
        w = w * np.exp(-slot / np.float32(gamma)).astype(np.float32)
    return w.astype(np.float32)


def slot_preparation(ids, loss_mask, anchors, keep, block_size: int, gamma: float):
    """Labels, validity and weights for every draft slot (dspark.py:116-127, 143).

    ids [b, s] int64, loss_mask [b, s] float, anchors [b, nb] int64, keep [b, nb] bool.
    Returns dict(target_ids, previous, weights, valid, teacher_indices) with the
    reference's shapes: [b, nb, K] and teacher_indices [b, nb*K].
    """
    ids = np.asarray(ids, dtype=np.int64)
    loss_mask = np.asarray(loss_mask, dtype=np.float32)
    anchors = np.asarray(anchors, dtype=np.int64)
    keep = np.asarray(keep, dtype=bool)
    b, s = ids.shape
    if s < 1:
        raise ValueError("Empty input sequence")
    slot = np.arange(block_size, dtype=np.int64)[None, None, :]
    labels = anchors[:, :, None] + slot + 1
    safe = np.where(keep[:, :, None], np.minimum(labels, s - 1), 0)
    rows = np.arange(b)[:, None, None]
    target_ids = ids[rows, safe]
    supervision = loss_mask[rows, safe]
    ok = keep[:, :, None] & (labels < s) & (supervision > 0.5)
    valid = np.cumprod(ok.astype(np.int64), axis=-1).astype(bool)
    weights = slot_weights(valid, gamma)
    first = ids[np.arange(b)[:, None], anchors]
    previous = np.concatenate([first[:, :, None], target_ids[:, :, :-1]], axis=-1)
    teacher_indices = np.maximum(safe - 1, 0).reshape(b, -1)
    return dict(
        target_ids=target_ids,
        previous=previous,
        weights=weights,
        valid=valid,
        teacher_indices=teacher_indices,
    )


# ---------------------------------------------------------------------------
# A6/A7: per-row objective statistics  objective.py:54-58, 42
# ---------------------------------------------------------------------------


def _lse(x: np.ndarray) -> np.ndarray:
    m = x.max(-1, keepdims=True)
    return (m + np.log(np.exp(x - m).sum(-1, keepdims=True)))[..., 0]


# F.cross_entropy's default ignore_index (objective.py:54): such a row has no CE term.
IGNORE_INDEX = -100


def _checked_labels(labels, v):
    """labels as int64 and the mask of ignored rows; any other label outside [0, V)
    raises, as F.cross_entropy does."""
    labels = np.asarray(labels, dtype=np.int64)
    ignore = labels == IGNORE_INDEX
    if np.any(((labels < 0) | (labels >= v)) & ~ignore):
        raise ValueError(f"label outside [0, {v}) other than the ignore index {IGNORE_INDEX}")
    return labels, ignore


def row_objective(z, u, labels, dtype=np.float64) -> dict:
    """Per-row CE, KL(target || draft) and acceptance rate a = sum_v min(p, t).

    z, u: [R, V] draft / teacher logits; labels [R] (IGNORE_INDEX: CE 0).  Computed in
    ``dtype`` (float64 for parity, float32 for the CPU baseline).  Follows
    objective.py:54 (CE), 55-58 (softmax, log_softmax, KL) and 42 (accept rate).
    """
    z = np.asarray(z, dtype=dtype)
    u = np.asarray(u, dtype=dtype)
    labels, ignore = _checked_labels(labels, z.shape[1])
    r = np.arange(z.shape[0])
    lz, lu = _lse(z), _lse(u)
    logp = z - lz[:, None]
    logt = u - lu[:, None]
    p, t = np.exp(logp), np.exp(logt)
    return dict(
        lse_z=lz,
        lse_u=lu,
        ce=np.where(ignore, 0.0, lz - z[r, np.where(ignore, 0, labels)]).astype(lz.dtype),
        kl=(t * (logt - logp)).sum(-1),
        accept_rate=np.minimum(p, t).sum(-1),
    )


def acceptance_length_counts(accept_rate, valid):
    """(sum of block lengths over valid blocks, number of valid blocks).

    accept_rate, valid: [nb, K].  len_b = 1 + sum_k prod_{j<=k} a_j v_j and a block
    counts only if any slot is valid (objective.py:39-46; README.md:92-102).
    """
    a = np.asarray(accept_rate, dtype=np.float64)
    v = np.asarray(valid).astype(np.float64)
    prefix = np.cumprod(a * v, axis=-1)
    block_valid = np.asarray(valid).astype(bool).any(-1)
    lengths = prefix.sum(-1) + 1.0
    return float((lengths * block_valid).sum()), float(block_valid.sum())


def ce_kl_loss(z, u, weights, labels, valid, c_ce=0.1, c_kl=0.9, dtype=np.float64, chunk_rows=64, workers=1):
    """Forward objective: the six LossMetrics plus per-row statistics.

    z, u [N, V] (or [..., K, V]); weights, labels, valid [..., K] with N rows in
    blocks of K consecutive slots.  Follows
    objective.py:49-67 and the LossMetrics properties at objective.py:20-26.
    Every row statistic is row-local, so chunks of ``chunk_rows`` rows may run on
    ``workers`` host threads (numpy releases the GIL inside its loops); the sums over
    rows are then taken in row order as with one worker.
    """
    valid = np.asarray(valid)
    if valid.ndim < 2:
        raise ValueError("valid must have a trailing block axis [..., K]")
    k = valid.shape[-1]
    weights = np.asarray(weights, dtype=np.float64).reshape(-1)
    labels = np.asarray(labels).reshape(-1)
    n = weights.shape[0]
    z = np.asarray(z).reshape(n, -1)
    u = np.asarray(u).reshape(n, -1)
    rows = {key: np.empty(n, dtype=np.float64) for key in ("lse_z", "lse_u", "ce", "kl", "accept_rate")}

    def chunk(lo):
        hi = min(n, lo + chunk_rows)
        part = row_objective(z[lo:hi], u[lo:hi], labels[lo:hi], dtype=dtype)
        for key in rows:
            rows[key][lo:hi] = part[key]

    if workers > 1:
        from concurrent.futures import ThreadPoolExecutor

        with ThreadPoolExecutor(max_workers=workers) as ex:
            list(ex.map(chunk, range(0, n, chunk_rows)))
    else:
        for lo in range(0, n, chunk_rows):
            chunk(lo)
    return metrics_from_rows(rows, weights, valid, c_ce, c_kl), rows


def metrics_from_rows(rows, weights, valid, c_ce=0.1, c_kl=0.9) -> dict:
    """The six LossMetrics plus ``loss`` and ``accept_len`` from per-row statistics (``rows``
    with "ce", "kl" and "accept_rate" over all N rows, in row order), as objective.py:53-65
    and 20-26 form them.  Rows may come from ``ce_kl_loss`` on chunks of the batch."""
    valid = np.asarray(valid)
    k = valid.shape[-1]
    weights = np.asarray(weights, dtype=np.float64).reshape(-1)
    den = float(weights.sum())
    ce_sum = float((np.asarray(rows["ce"], dtype=np.float64) * weights).sum())
    kl_sum = float((np.asarray(rows["kl"], dtype=np.float64) * weights).sum())
    clamp = max(den, 1e-6)
    v2 = valid.reshape(-1, k)
    acc_sum, acc_tot = acceptance_length_counts(np.asarray(rows["accept_rate"]).reshape(v2.shape), v2)
    metrics = dict(
        ce=ce_sum / clamp,
        kl=kl_sum / clamp,
        numerator=c_ce * ce_sum + c_kl * kl_sum,
        denominator=den,
        accept_len_sum=acc_sum,
        accept_len_total=acc_tot,
    )
    metrics["loss"] = metrics["numerator"] / max(den, 1e-6)
    metrics["accept_len"] = acc_sum / max(acc_tot, 1.0)
    return metrics


def ce_kl_backward(z, u, weights, labels, c_ce=0.1, c_kl=0.9, accumulation_steps=1, dtype=np.float64):
    """dl = (w / acc) [c_ce (p - e_y) + c_kl (p - t)]  (objective.py:70-80).

    The derivative of the *numerator* (not divided by the denominator); the
    pooled normalisation happens in the optimizer (shard.py:318-331).  A row labelled
    IGNORE_INDEX has no CE term, so its dl is (w / acc) c_kl (p - t): the gradient of the
    forward's loss (the reference's scatter_add_ at objective.py:78 rejects that index).
    """
    z = np.asarray(z, dtype=dtype)
    u = np.asarray(u, dtype=dtype)
    n = z.shape[0]
    labels, ignore = _checked_labels(np.asarray(labels).reshape(n), z.shape[1])
    scale = np.asarray(weights, dtype=dtype).reshape(n) / accumulation_steps
    p = np.exp(z - _lse(z)[:, None])
    t = np.exp(u - _lse(u)[:, None])
    dl = np.where(ignore[:, None], c_kl * (p - t), (c_ce + c_kl) * p - c_kl * t)
    keep = np.flatnonzero(~ignore)
    dl[keep, labels[keep]] -= c_ce
    return dl * scale[:, None]


# ---------------------------------------------------------------------------
# A2/A3/A10: LM head projection and its backward  train.py:272-279, 302
# ---------------------------------------------------------------------------


def lm_head_logits(hidden, weight, markov=None, dtype=np.float64):
    """z = hidden . W^T (+ Markov addend), in ``dtype`` (ops.py:34-35, train.py:272-279).

    The fp32 objective keeps z unrounded (the bf16 training path would round z
    to bf16 first; the graded contract is the fp32 objective).
    """
    z = np.asarray(hidden, dtype=dtype) @ np.asarray(weight, dtype=dtype).T
    if markov is not None:
        z = z + np.asarray(markov, dtype=dtype)
    return z


def lm_head_backward(dl, weight, dtype=np.float64):
    """dh = dl . W_lm  (train.py:302)."""
    return np.asarray(dl, dtype=dtype) @ np.asarray(weight, dtype=dtype)


def markov_logits(prev, w1, w2, dtype=np.float64):
    """Markov-head logits w1[prev] . w2^T (train.py:276-279: ops.embedding then
    ops.linear, ops.py:69-70 and 34-35; MarkovHead layers.py:74-78).  The fp32
    objective adds them to the LM-head logits unrounded."""
    e = np.asarray(w1, dtype=dtype)[np.asarray(prev, dtype=np.int64)]
    return e @ np.asarray(w2, dtype=dtype).T


def markov_backward(dl, prev, w1, w2, dtype=np.float64):
    """Gradients of the Markov head given dl (train.py:303-307):
    d(previous) = dl . w2 (ops.linear_backward, ops.py:38-45), d(w2) = dl^T . w1[prev]
    (copied into w2.grad), d(w1) = zeros.index_add(prev, d(previous))
    (ops.embedding_backward, ops.py:73-74).  Returns (d_previous, d_w2, d_w1)."""
    dl = np.asarray(dl, dtype=dtype)
    w2 = np.asarray(w2, dtype=dtype)
    prev = np.asarray(prev, dtype=np.int64)
    e = np.asarray(w1, dtype=dtype)[prev]
    dprev = dl @ w2
    dw2 = dl.T @ e
    dw1 = np.zeros(np.shape(w1), dtype=dtype)
    np.add.at(dw1, prev, dprev)
    return dprev, dw2, dw1


# ---------------------------------------------------------------------------
# final_norm  ops.py:48-66 (train.py:271, 308-310)
# ---------------------------------------------------------------------------


def rms_norm(x, weight, eps):
    """ops.rms_norm (ops.py:48-52) in fp32 with the rounding points of torch's device
    kernels: mean = sum(x*x) * (1/d), inv = 1/sqrt(mean + eps), normalized = bf16(x * inv),
    out = bf16(weight * normalized).  x and weight hold bf16 values.  Returns
    (out, inv [N], normalized)."""
    x = np.asarray(x, dtype=np.float32)
    w = np.asarray(weight, dtype=np.float32)
    d = x.shape[-1]
    sq = (x * x).astype(np.float32)
    mean = (sq.sum(-1, dtype=np.float32) * np.float32(1.0 / np.float32(d))).astype(np.float32)
    inv = (np.float32(1.0) / np.sqrt((mean + np.float32(eps)).astype(np.float32))).astype(np.float32)
    normalized = bf16_round(x * inv[..., None])
    out = bf16_round(w * normalized)
    return out, inv, normalized


def rms_norm_backward(dy, x, inv, weight):
    """ops.rms_norm_backward (ops.py:55-66) in fp32: dw = bf16(sum_rows bf16(dy * normalized)),
    dz = bf16(dy * weight), dinv = sum(dz * x), dvar = dinv * (-0.5 * inv^3),
    dx = bf16(dz * inv + (dvar * (1/d)) * (2 x)).  torch divides by the host scalar d through
    its reciprocal on the device, kept here.  Returns (dx, dw)."""
    dy = np.asarray(dy, dtype=np.float32)
    x = np.asarray(x, dtype=np.float32)
    w = np.asarray(weight, dtype=np.float32)
    inv = np.asarray(inv, dtype=np.float32).reshape(-1, 1)
    d = x.shape[-1]
    normalized = bf16_round(x * inv)
    dw = bf16_round(bf16_round(dy * normalized).sum(0, dtype=np.float32))
    dz = bf16_round(dy * w)
    dinv = (dz * x).astype(np.float32).sum(-1, keepdims=True, dtype=np.float32)
    dvar = (dinv * (np.float32(-0.5) * ((inv * inv) * inv))).astype(np.float32)
    q = (dvar * np.float32(np.float32(1.0) / np.float32(d))).astype(np.float32)
    dx = bf16_round((dz * inv).astype(np.float32) + (q * (np.float32(2.0) * x)).astype(np.float32))
    return dx, dw


# ---------------------------------------------------------------------------
# Pooled-normalisation tail  train.py:525-535, shard.py:318-330
# ---------------------------------------------------------------------------


def pooled_tail(metrics, world_size=1, accumulation_steps=1):
    """Pool [count, 6] LossMetrics buffers (ce, kl, numerator, denominator, accept_len_sum,
    accept_len_total) in fp32 in index order, as the training loop's all-reduce of the last
    four (train.py:525-532) does across ranks; then loss = num / max(den, 1e-6) and
    accept_len = sum / max(total, 1) (train.py:533-534), and the gradient factor of
    adamw_step (shard.py:321-327): world * acc / max(den, 1e-6) if den > 0 else 0, where
    the int-over-tensor division is reciprocal(max(den, 1e-6)) * (world * acc) in fp32.
    Returns fp32 (loss, accept_len, factor, den)."""
    m = np.asarray(metrics, dtype=np.float32).reshape(-1, 6)
    num = den = asum = atot = np.float32(0.0)
    for row in m:
        num = np.float32(num + row[2])
        den = np.float32(den + row[3])
        asum = np.float32(asum + row[4])
        atot = np.float32(atot + row[5])
    loss = np.float32(num / max(den, np.float32(1e-6)))
    accept = np.float32(asum / max(atot, np.float32(1.0)))
    wa = np.float32(world_size * accumulation_steps)
    factor = np.float32(np.float32(1.0) / max(den, np.float32(1e-6)) * wa) if den > 0 else np.float32(0.0)
    return loss, accept, factor, den


def scale_gradient(grad, factor, bf16=False):
    """grad.mul_(factor) (shard.py:330) with a 0-d fp32 factor: for bf16 gradients
    (shard.py:74, zeros_like of the bf16 parameter) torch casts the factor to bf16 first,
    multiplies in fp32 and rounds the product to bf16; fp32 gradients multiply directly."""
    g = np.asarray(grad, dtype=np.float32)
    if bf16:
        return bf16_round(g * bf16_round(np.float32(factor)))
    return g * np.float32(factor)


# ---------------------------------------------------------------------------
# A5: block-FP8 teacher head  ops.py:183-200
# ---------------------------------------------------------------------------


def quantize_activation_blocks(x):
    """1x128 dynamic e4m3 activation quantisation in fp32 (ops.py:189-197).

    Returns (codes uint8 [.., d], scales fp32 [.., d/128]).
    """
    x = np.asarray(x, dtype=np.float32)
    xb = x.reshape(*x.shape[:-1], -1, 128)
    xs = (np.abs(xb).max(-1, keepdims=True) / np.float32(448.0)).astype(np.float32)
    q = np.clip(xb / np.maximum(xs, np.float32(F32_TINY)), -448, 448).astype(np.float32)
    codes = e4m3_encode(q).reshape(x.shape)
    return codes, xs[..., 0]


def quantize_weight_blocks(w):
    """128x128 block e4m3 weight quantisation: s = amax/448, q = clamp(W/s, +-448).

    The recipe of the C4 configuration (weights stored as e4m3 codes plus an
    fp32 scale per 128x128 block that multiplies, qwen.py:43-54, ops.py:198-199).
    """
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    blocks = w.reshape(n // 128, 128, k // 128, 128)
    s = (np.abs(blocks).max(axis=(1, 3)) / np.float32(448.0)).astype(np.float32)
    q = blocks / np.maximum(s, np.float32(F32_TINY))[:, None, :, None]
    codes = e4m3_encode(np.clip(q, -448, 448)).reshape(n, k)
    return codes, s


def fp8_linear(x, weight_codes, scale, dtype=np.float64):
    """Teacher logits with ops.fp8_linear numerics (ops.py:183-200), rounded to bf16.

    x [N, d] (bf16 values), weight_codes [V, d] uint8 e4m3, scale [V/128, d/128] fp32.
    """
    n_out, k = weight_codes.shape
    if n_out % 128 or k % 128:
        raise ValueError("Expected checkpoint's 128x128 FP8 weight blocks")
    codes, xs = quantize_activation_blocks(x)
    dx = (e4m3_decode(codes).reshape(*codes.shape[:-1], -1, 128) * xs[..., None]).astype(np.float32)
    dx = dx.reshape(codes.shape)
    sw = np.repeat(np.repeat(np.asarray(scale, np.float32), 128, axis=0), 128, axis=1)
    dw = (e4m3_decode(weight_codes) * sw).astype(np.float32)
    out = np.asarray(dx, dtype=dtype) @ np.asarray(dw, dtype=dtype).T
    return bf16_round(out.astype(np.float32))


# ---------------------------------------------------------------------------
# Convenience: cosine / relative error metrics (experiments/compare.py:80-89)
# ---------------------------------------------------------------------------


def similarity(actual, expected) -> dict:
    """Row cosine (min and mean over rows of the last axis), whole-tensor cosine,
    relative L2 and max |diff| -- the comparison metrics of experiments/compare.py:80-89."""
    a2 = np.asarray(actual, dtype=np.float64)
    e2 = np.asarray(expected, dtype=np.float64)
    a2 = a2.reshape(-1, a2.shape[-1]) if a2.ndim else a2.reshape(1, 1)
    e2 = e2.reshape(-1, e2.shape[-1]) if e2.ndim else e2.reshape(1, 1)
    dots = (a2 * e2).sum(-1)
    na_r, ne_r = np.linalg.norm(a2, axis=-1), np.linalg.norm(e2, axis=-1)
    live = ne_r > 0   # rows that are exactly zero in the expected tensor have no direction
    row_cos = dots[live] / np.maximum(na_r[live] * ne_r[live], 1e-300)
    if row_cos.size == 0:
        row_cos = np.ones(1)
    a, e = a2.reshape(-1), e2.reshape(-1)
    na, ne = np.linalg.norm(a), np.linalg.norm(e)
    cos = float(a @ e / (na * ne)) if na > 0 and ne > 0 else float("nan")
    diff = a - e
    return dict(
        cosine=cos,
        cosine_min=float(row_cos.min()),
        cosine_mean=float(row_cos.mean()),
        zero_rows_nonzero=int(np.count_nonzero(na_r[~live])),
        relative_l2=float(np.linalg.norm(diff) / max(ne, 1e-30)),
        max_abs=float(np.abs(diff).max()) if diff.size else 0.0,
    )


def log_vocab(v: int) -> float:
    return math.log(v)
