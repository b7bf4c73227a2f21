"""GPU parity of final_norm around the LM head (train.py:271, 308-310; ops.py:48-66):
ns_rms_norm_fwd / ns_rms_norm_bwd against the oracle, and the fused dh -> rms-norm
backward (ns_lmhead_norm_bwd, and the Markov backward with a norm) against the unfused
chain, which it must equal bit for bit (same split-K sums, same rounding points).

Tolerances: rms_norm outputs within one bf16 ulp of the oracle (the row sums run in a
different order than numpy's); dx within one bf16 ulp plus 2^-16 of the row's largest
|dx|; the weight gradient (a sum over N of bf16 products) within 2^-7 relative."""

import numpy as np
import pytest
import torch

from nanospec_amd import head, ops, synthetic
from oracle import objective_ref as ref

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
EPS = 1e-6


def _np(t):
    return t.detach().float().cpu().numpy()


def _norm_inputs(n, d, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = (2.0 * torch.randn((n, d), generator=g, device=DEV) + 0.25).bfloat16()
    w = (1.0 + 0.1 * torch.randn(d, generator=g, device=DEV)).bfloat16()
    return x, w, g


def _bf16_ulp(x):
    a = np.abs(np.asarray(x, dtype=np.float64))
    return np.where(a > 0, 2.0 ** (np.floor(np.log2(np.where(a > 0, a, 1.0))) - 7), 2.0 ** -133)


def _within_ulp(got, want, frac=0.999):
    diff = np.abs(got.astype(np.float64) - want)
    assert np.all(diff <= _bf16_ulp(want)), float((diff / _bf16_ulp(want)).max())
    assert np.mean(got == want) >= frac, float(np.mean(got == want))


@pytest.mark.parametrize("n,d", [(300, 320), (4096, 5120)])
def test_rms_norm_forward_matches_oracle(gpu_lib, n, d):
    x, w, _ = _norm_inputs(n, d, n)
    out, saved = ops.rms_norm(x, w, EPS)
    torch.cuda.synchronize()
    o_ref, inv_ref, n_ref = ref.rms_norm(_np(x), _np(w), EPS)
    inv = _np(saved.inverse_rms).reshape(-1)
    assert np.all(np.abs(inv - inv_ref) <= 4 * np.spacing(inv_ref)), float(np.abs(inv - inv_ref).max())
    got_n, got_o = _np(saved.normalized), _np(out)
    _within_ulp(got_n, n_ref)
    # out = bf16(w * normalized): the same product wherever normalized agrees, and one
    # ulp of normalized moves it by at most two ulps elsewhere
    same = got_n == n_ref
    assert np.array_equal(got_o[same], o_ref[same])
    assert np.all(np.abs(got_o - o_ref) <= 2 * _bf16_ulp(o_ref))
    assert saved.input is x and tuple(saved.inverse_rms.shape) == (n, 1)


@pytest.mark.parametrize("n,d", [(300, 320), (4096, 5120), (9000, 2048)])
def test_rms_norm_backward_matches_oracle(gpu_lib, n, d):
    x, w, g = _norm_inputs(n, d, 7 + n)
    _, saved = ops.rms_norm(x, w, EPS)
    dy = (0.7 * saved.normalized.float() + 0.3 * torch.randn((n, d), generator=g, device=DEV)).bfloat16()
    wg = torch.full((d,), float("nan"), dtype=torch.bfloat16, device=DEV)   # overwritten
    dx = ops.rms_norm_backward(dy, saved, w, wg)
    torch.cuda.synchronize()
    dx_ref, dw_ref = ref.rms_norm_backward(_np(dy), _np(x), _np(saved.inverse_rms), _np(w))
    got = _np(dx)
    tol = _bf16_ulp(dx_ref) + 2.0 ** -16 * np.abs(dx_ref).max(axis=-1, keepdims=True)
    assert np.all(np.abs(got - dx_ref) <= tol), float((np.abs(got - dx_ref) - tol).max())
    assert np.mean(got == dx_ref) >= 0.99
    np.testing.assert_allclose(_np(wg), dw_ref, rtol=2.0 ** -7, atol=1e-3 * np.abs(dw_ref).max())


@pytest.mark.parametrize("n,v,d", [(300, 8200, 320), (1024, 8192, 5120)])
def test_fused_norm_backward_equals_unfused(gpu_lib, n, v, d):
    x, w, g = _norm_inputs(n, d, 100 + n)
    _, saved = ops.rms_norm(x, w, EPS)
    dl = (1e-3 * torch.randn((n, v), generator=g, device=DEV)).bfloat16()
    wlm = (0.02 * torch.randn((v, d), generator=g, device=DEV)).bfloat16()
    wg1 = torch.empty(d, dtype=torch.bfloat16, device=DEV)
    wg2 = torch.empty_like(wg1)
    dx1 = head.lm_head_norm_backward(dl, wlm, (saved, w, wg1))
    dh = head.lm_head_linear_backward(dl, wlm)
    dx2 = ops.rms_norm_backward(dh, saved, w, wg2)
    torch.cuda.synchronize()
    assert torch.equal(dx1, dx2) and torch.equal(wg1, wg2)


def test_markov_backward_with_norm_equals_unfused(gpu_lib):
    n, v, d, r = 512, 4096, 320, 64
    x, w, g = _norm_inputs(n, d, 5)
    _, saved = ops.rms_norm(x, w, EPS)
    dl = (1e-3 * torch.randn((n, v), generator=g, device=DEV)).bfloat16()
    wlm = (0.02 * torch.randn((v, d), generator=g, device=DEV)).bfloat16()
    prev, w1, w2 = synthetic.markov_factors(n, v, r, 6, DEV)
    mk = head.MarkovFactors(prev, w1, w2)
    grads = [torch.zeros((v, r), dtype=torch.bfloat16, device=DEV) for _ in range(4)]
    wg1, wg2 = torch.empty(d, dtype=torch.bfloat16, device=DEV), torch.empty(d, dtype=torch.bfloat16, device=DEV)
    dx1 = head.lm_head_markov_backward(dl, wlm, mk, grads[0], grads[1], final_norm=(saved, w, wg1))
    dh = head.lm_head_markov_backward(dl, wlm, mk, grads[2], grads[3])
    dx2 = ops.rms_norm_backward(dh, saved, w, wg2)
    torch.cuda.synchronize()
    assert torch.equal(dx1, dx2) and torch.equal(wg1, wg2)
    assert torch.equal(grads[0], grads[2]) and torch.equal(grads[1], grads[3])


def test_head_backward_with_final_norm(gpu_lib):
    """lm_head_ce_kl_backward(final_norm=...) returns dx: the same as the unfused chain."""
    from nanospec_amd.config import Objective

    n, d, v = 256, 256, 4096
    hidden0, weight, markov, teacher, slots = synthetic.head_inputs(n, d, v, 12, DEV)
    w = torch.ones(d, dtype=torch.bfloat16, device=DEV)
    hidden, saved_norm = ops.rms_norm(hidden0, w, EPS)
    o = Objective(block_size=8)
    _, saved = head.lm_head_ce_kl_loss(hidden, weight, teacher, slots, o, markov_logits=markov)
    wg = torch.empty(d, dtype=torch.bfloat16, device=DEV)
    dx, dl = head.lm_head_ce_kl_backward(saved, return_dlogits=True, final_norm=(saved_norm, w, wg))
    wg2 = torch.empty_like(wg)
    dx2 = ops.rms_norm_backward(head.lm_head_linear_backward(dl.reshape(n, v), weight), saved_norm, w, wg2)
    torch.cuda.synchronize()
    assert torch.equal(dx.reshape(n, d), dx2.reshape(n, d)) and torch.equal(wg, wg2)
