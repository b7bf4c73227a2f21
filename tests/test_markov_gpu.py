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
