"""GPU parity of the factored Markov head fused into the LM-head GEMM
(ns_lmhead_markov_ce_kl_fwd): z = hidden . W^T + w1[prev] . w2^T, against the oracle.

Tolerances as for the dense path: metrics within 1e-4 relative of the fp32
objective; dl within one bf16 ulp plus fp32 evaluation error.
"""

import numpy as np
import pytest
import torch

from nanospec_amd import head, synthetic
from nanospec_amd.config import Objective
from oracle import objective_ref as ref

from dh_bar import assert_dh_rows

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
FIELDS = ("ce", "kl", "numerator", "denominator", "accept_len_sum", "accept_len_total")


def _np(t):
    return t.detach().float().cpu().numpy()


def _inputs(n, d, v, r, seed):
    hidden, weight, _, teacher, slots = synthetic.head_inputs(n, d, v, seed, DEV)
    prev, w1, w2 = synthetic.markov_factors(n, v, r, seed + 1, DEV)
    return hidden, weight, teacher, slots, head.MarkovFactors(prev, w1, w2)


def _oracle(hidden, weight, teacher, slots, mk, o):
    z = ref.lm_head_logits(_np(hidden), _np(weight)) + ref.markov_logits(mk.previous.cpu().numpy(), _np(mk.w1),
                                                                          _np(mk.w2))
    wt = _np(slots.weights).reshape(-1)
    y = slots.target_ids.reshape(-1).cpu().numpy()
    valid = slots.valid.cpu().numpy()
    k = valid.shape[-1]
    m, rows = ref.ce_kl_loss(z, _np(teacher), wt.reshape(-1, k), y.reshape(-1, k), valid, o.ce, o.kl)
    dl = ref.ce_kl_backward(z, _np(teacher), wt, y, o.ce, o.kl)
    return z, m, rows, dl


@pytest.mark.parametrize("n,d,v,r", [
    (72, 128, 8200, 64),      # partial token and vocab tiles, one Markov K stage
    (256, 256, 4096, 256),    # the reference rank
    (128, 128, 2048, 512),    # eight Markov K stages
])
def test_markov_forward_matches_oracle(gpu_lib, n, d, v, r):
    hidden, weight, teacher, slots, mk = _inputs(n, d, v, r, 40 + n)
    o = Objective(block_size=8)
    m, saved = head.lm_head_ce_kl_loss(hidden, weight, teacher, slots, o, markov=mk)
    torch.cuda.synchronize()
    z, m_ref, rows, dl_ref = _oracle(hidden, weight, teacher, slots, mk, o)
    for f in FIELDS:
        w = m_ref[f]
        assert float(getattr(m, f)) == pytest.approx(w, rel=1e-4, abs=1e-6 * max(1.0, abs(w))), f
    rs = _np(saved.row_stats)
    np.testing.assert_allclose(rs[:, 0], rows["lse_z"], rtol=2e-6, atol=5e-5)
    np.testing.assert_allclose(rs[:, 5], z[np.arange(n), slots.target_ids.reshape(-1).cpu().numpy()],
                               rtol=1e-5, atol=1e-5)
    dl = _np(saved.dlogits).reshape(n, -1)
    diff = np.abs(dl.astype(np.float64) - dl_ref)
    tol = np.abs(dl_ref) * 2.0 ** -7 + 2e-5 * np.abs(dl_ref).max(axis=-1, keepdims=True)
    assert np.all(diff <= tol), float((diff - tol).max())


def test_markov_matches_dense_addend_of_the_same_logits(gpu_lib):
    """The fused factors and a dense fp32-exact addend give the same objective: the dense
    path is fed w1[prev] . w2^T rounded to bf16, so they agree to that rounding."""
    n, d, v, r = 128, 128, 4096, 128
    hidden, weight, teacher, slots, mk = _inputs(n, d, v, r, 7)
    o = Objective(block_size=8)
    m1, _ = head.lm_head_ce_kl_loss(hidden, weight, teacher, slots, o, markov=mk)
    dense = (mk.w1[mk.previous].float() @ mk.w2.float().T).to(torch.bfloat16)
    m2, _ = head.lm_head_ce_kl_loss(hidden, weight, teacher, slots, o, markov_logits=dense)
    torch.cuda.synchronize()
    for f in ("ce", "kl", "accept_len_sum"):
        assert float(getattr(m1, f)) == pytest.approx(float(getattr(m2, f)), rel=2e-3), f


def test_markov_bad_previous_id_poisons_its_row(gpu_lib):
    n, d, v, r = 64, 128, 2048, 64
    hidden, weight, teacher, slots, mk = _inputs(n, d, v, r, 9)
    mk.previous[5] = v            # out of range: that row's logits are NaN, the others are not
    m, saved = head.lm_head_ce_kl_loss(hidden, weight, teacher, slots, Objective(block_size=8), markov=mk)
    torch.cuda.synchronize()
    ce = _np(saved.row_stats)[:, 2]
    assert np.isnan(ce[5]) and np.all(np.isfinite(np.delete(ce, 5)))
    assert np.isnan(float(m.ce))


# ---------------------------------------------------------------------------
# backward: dh, markov_w2.grad (copy_) and markov_w1.grad (index_add_), train.py:302-307
# ---------------------------------------------------------------------------


def _bwd_inputs(n, v, d, r, seed, id_range=None):
    g = torch.Generator(device=DEV).manual_seed(seed)
    dl = (1e-3 * torch.randn((n, v), generator=g, device=DEV)).bfloat16()
    w = (0.02 * torch.randn((v, d), generator=g, device=DEV)).bfloat16()
    prev, w1, w2 = synthetic.markov_factors(n, v, r, seed + 1, DEV)
    if id_range is not None:
        prev = torch.randint(0, id_range, (n,), generator=g, device=DEV)
    g1 = (1e-3 * torch.randn((v, r), generator=g, device=DEV)).bfloat16()   # accumulated into
    return dl, w, head.MarkovFactors(prev, w1, w2), g1


def _run_bwd(dl, w, mk, g1):
    w1_grad = g1.clone()
    w2_grad = torch.full_like(g1, float("nan"))          # overwritten, never read
    dh = head.lm_head_markov_backward(dl, w, mk, w1_grad, w2_grad)
    torch.cuda.synchronize()
    return dh, w1_grad, w2_grad


def _assert_grads(dl, mk, g1, w1_grad, w2_grad, keep=None):
    """w2.grad and w1.grad against the fp64 oracle.  Each is one bf16 rounding of an
    fp32 sum: within 2^-8 relative plus fp32 accumulation error, bounded by 2^-18 of
    the same sum taken over absolute values."""
    dln, prev = _np(dl).astype(np.float64), mk.previous.cpu().numpy()
    w1n, w2n = _np(mk.w1).astype(np.float64), _np(mk.w2).astype(np.float64)
    if keep is None:
        keep = np.ones(len(prev), dtype=bool)
    dprev, dw2, dw1 = ref.markov_backward(dln[keep], prev[keep], w1n, w2n)
    scale2 = np.abs(dln[keep]).T @ np.abs(w1n[prev[keep]])
    got2 = _np(w2_grad)
    assert np.all(np.abs(got2 - dw2) <= np.abs(dw2) * 2.0 ** -8 + 2.0 ** -18 * scale2 + 1e-30), \
        float(np.abs(got2 - dw2).max())
    want1 = _np(g1).astype(np.float64) + dw1
    scale1 = np.zeros_like(dw1)
    np.add.at(scale1, prev[keep], np.abs(dln[keep]) @ np.abs(w2n))
    got1 = _np(w1_grad)
    assert np.all(np.abs(got1 - want1) <= np.abs(want1) * 2.0 ** -8 + 2.0 ** -18 * scale1 + 1e-30), \
        float(np.abs(got1 - want1).max())


@pytest.mark.parametrize("n,v,d,r,id_range", [
    (72, 8200, 128, 64, None),        # ragged vocab tile, two 32-token stages plus an 8-token tail
    (256, 4096, 256, 256, None),      # the reference rank, whole stages only
    (1000, 2048, 192, 128, 16),       # long runs of repeated ids (index_add_ segments of ~60)
    (1536, 16384, 256, 256, None),    # 48 token stages (six unrolled groups of 8), 64 vocab tiles
    (24, 4096, 128, 64, None),        # fewer tokens than one stage: the register path alone
    (1000, 4096, 128, 64, None),      # 31 stages (a partial unrolled group) plus an 8-token tail
    (128, 2048, 128, 512, 8),         # rank 512: two rank tiles in the w2.grad GEMM
    (32768, 2048, 3072, 256, None),   # six rounds of dh tiles, one launch each, then the Markov tiles
])
def test_markov_backward_matches_oracle(gpu_lib, n, v, d, r, id_range):
    dl, w, mk, g1 = _bwd_inputs(n, v, d, r, 60 + n, id_range)
    dh, w1_grad, w2_grad = _run_bwd(dl, w, mk, g1)
    dh_ref = ref.lm_head_backward(_np(dl), _np(w), dtype=np.float32 if n > 1024 else np.float64)
    assert_dh_rows(_np(dh), dh_ref)
    _assert_grads(dl, mk, g1, w1_grad, w2_grad)


def test_markov_backward_deterministic(gpu_lib):
    dl, w, mk, g1 = _bwd_inputs(2048, 8192, 256, 256, 5, id_range=64)
    a = _run_bwd(dl, w, mk, g1)
    b = _run_bwd(dl, w, mk, g1)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_markov_backward_skips_out_of_range_ids(gpu_lib):
    """Rows with a prev id outside [0, V) add nothing to w1.grad (the forward has made
    their loss NaN); dh does not depend on prev."""
    n, v, d, r = 128, 2048, 128, 64
    dl, w, mk, g1 = _bwd_inputs(n, v, d, r, 11)
    mk.previous[3] = v
    mk.previous[77] = -1
    dh, w1_grad, w2_grad = _run_bwd(dl, w, mk, g1)
    keep = np.ones(n, dtype=bool)
    keep[[3, 77]] = False
    dln, prev = _np(dl).astype(np.float64), mk.previous.cpu().numpy()
    _, _, dw1 = ref.markov_backward(dln[keep], prev[keep], _np(mk.w1), _np(mk.w2))
    want1 = _np(g1).astype(np.float64) + dw1
    assert np.all(np.abs(_np(w1_grad) - want1) <= np.abs(want1) * 2.0 ** -8 + 1e-6)
    assert_dh_rows(_np(dh), ref.lm_head_backward(_np(dl), _np(w)))


def test_markov_forward_backward_through_head_step(gpu_lib):
    """head_step with factors: the backward's gradients follow the dl the forward emitted."""
    n, d, v, r = 256, 256, 4096, 256
    hidden, weight, teacher, slots, mk = _inputs(n, d, v, r, 21)
    o = Objective(block_size=8)
    g1 = torch.zeros((v, r), dtype=torch.bfloat16, device=DEV)
    w1_grad, w2_grad = g1.clone(), torch.empty_like(g1)
    m, dh, dl = head.head_step(hidden, weight, teacher, slots, o, markov=mk, markov_grads=(w1_grad, w2_grad))
    torch.cuda.synchronize()
    dl2 = dl.reshape(n, v)
    _, _, _, dl_ref = _oracle(hidden, weight, teacher, slots, mk, o)
    diff = np.abs(_np(dl2).astype(np.float64) - dl_ref)
    assert np.all(diff <= np.abs(dl_ref) * 2.0 ** -7 + 2e-5 * np.abs(dl_ref).max(axis=-1, keepdims=True))
    _assert_grads(dl2, mk, g1, w1_grad, w2_grad)
    assert_dh_rows(_np(dh).reshape(n, d), ref.lm_head_backward(_np(dl2), _np(weight)))


@pytest.mark.parametrize("n,hot", [
    (8192, 4096),     # two sort chunks and one merge pass; one id on half the rows
    (12288, 12000),   # three chunks (a run with no merge partner); one id on almost every row
])
def test_markov_backward_skewed_ids(gpu_lib, n, hot):
    """A skewed previous-token distribution, as dropped anchor blocks give (every slot of a
    dropped block takes the block's first id, dspark.py:120-127): `hot` rows share one id.
    w1.grad matches the oracle and is bitwise reproducible."""
    v, d, r = 4096, 128, 256
    dl, w, mk, g1 = _bwd_inputs(n, v, d, r, 90 + n)
    g = torch.Generator(device=DEV).manual_seed(n)
    hot_rows = torch.randperm(n, generator=g, device=DEV)[:hot]
    mk.previous[hot_rows] = 17
    a = _run_bwd(dl, w, mk, g1)
    b = _run_bwd(dl, w, mk, g1)
    assert torch.equal(a[1], b[1]) and torch.equal(a[2], b[2])
    _assert_grads(dl, mk, g1, a[1], a[2])
