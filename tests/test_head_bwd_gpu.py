"""GPU parity of ce_kl_backward after the fused forward (objective.py:70-80 as train.py:301
calls it, with the backward's accumulation_steps): ns_lmhead_ce_kl_bwd runs pass 2 again from
the forward's row statistics.

It is the forward's own pass-2 kernel on the same inputs, so its dl must equal, bit for bit,
the dl a forward called with that accumulation_steps emits; that dl is checked against the
oracle's ce_kl_backward(accumulation_steps=3) to the fused tests' dl bar.  Also covered: the
empty batch through the fused forward and backward."""

import numpy as np
import pytest
import torch

from nanospec_amd import head, synthetic
from nanospec_amd.config import Objective
from oracle import objective_ref as ref

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _np(t):
    return t.detach().float().cpu().numpy()


def _case(kind):
    """(hidden, weight, target, slots, forward kwargs, dense markov or None) for each form
    of the head's inputs."""
    n, d, v = 136, 128, 4104           # a partial token tile and a vocabulary sliver
    hidden, weight, markov, teacher, slots = synthetic.head_inputs(n, d, v, 501, DEV, ragged=True)
    if kind == "dense":
        return hidden, weight, teacher, slots, dict(markov_logits=markov), markov
    if kind == "fp32_teacher":
        return hidden, weight, teacher.float(), slots, {}, None
    if kind == "factored":
        prev, w1, w2 = synthetic.markov_factors(n, v, 64, 502, DEV)
        return hidden, weight, teacher, slots, dict(markov=head.MarkovFactors(prev, w1, w2)), None
    # teacher rows gathered in the loads with the producer's log-sum-exp (teacher once)
    g = torch.Generator(device=DEV).manual_seed(503)
    xt = (2.0 * torch.randn((300, d), generator=g, device=DEV)).bfloat16()
    full = head.teacher_logits(xt, weight)
    rows = torch.randint(0, 300, (n,), generator=g, device=DEV)
    return hidden, weight, head.TeacherLogits(full.logits, rows, full.lse), slots, dict(markov_logits=markov), markov


@pytest.mark.parametrize("kind", ["dense", "fp32_teacher", "factored", "teacher_once"])
def test_backward_accumulation_steps_reemits_forward_bits(gpu_lib, kind):
    hidden, weight, target, slots, kw, _ = _case(kind)
    o = Objective(block_size=8)
    _, s1 = head.lm_head_ce_kl_loss(hidden, weight, target, slots, o, **kw)
    _, s3 = head.lm_head_ce_kl_loss(hidden, weight, target, slots, o, accumulation_steps=3, **kw)
    dl1, dl3 = s1.dlogits.clone(), s3.dlogits.clone()
    dh3_emitted = head.lm_head_ce_kl_backward(s3, 3)
    # forward emitted for 1 step, backward asks for 3: pass 2 runs again
    dh3, dl3_again = head.lm_head_ce_kl_backward(s1, 3, return_dlogits=True)
    torch.cuda.synchronize()
    assert torch.equal(dl3_again.reshape(dl3.shape), dl3)
    assert torch.equal(dh3, dh3_emitted)
    # a second backward on the same activations re-emits as well
    _, dl1_again = head.lm_head_ce_kl_backward(s1, 1, return_dlogits=True)
    torch.cuda.synchronize()
    assert torch.equal(dl1_again.reshape(dl1.shape), dl1)
    # metrics-only forward, then a backward
    _, s0 = head.lm_head_ce_kl_loss(hidden, weight, target, slots, o, emit_dlogits=False, **kw)
    assert s0.dlogits is None
    _, dl1_late = head.lm_head_ce_kl_backward(s0, 1, return_dlogits=True)
    torch.cuda.synchronize()
    assert torch.equal(dl1_late.reshape(dl1.shape), dl1)


def test_reemitted_dl_matches_oracle(gpu_lib):
    hidden, weight, target, slots, kw, markov = _case("dense")
    o = Objective(block_size=8)
    _, saved = head.lm_head_ce_kl_loss(hidden, weight, target, slots, o, emit_dlogits=False, **kw)
    _, dl = head.lm_head_ce_kl_backward(saved, 3, return_dlogits=True)
    torch.cuda.synchronize()
    z = ref.lm_head_logits(_np(hidden), _np(weight), _np(markov))
    want = ref.ce_kl_backward(z, _np(target), _np(slots.weights).reshape(-1), slots.target_ids.reshape(-1).cpu().numpy(),
                              o.ce, o.kl, accumulation_steps=3)
    got = _np(dl).reshape(want.shape).astype(np.float64)
    scale = np.abs(want).max(axis=-1, keepdims=True)
    tol = np.abs(want) * 2.0 ** -7 + 2e-5 * scale
    assert np.all(np.abs(got - want) <= tol)
    masked = ~slots.valid.reshape(-1).cpu().numpy()
    assert masked.any() and np.all(got[masked] == 0.0)      # w = 0 rows vanish


def test_ignore_index_rows(gpu_lib):
    """Label -100 in the fused head: CE 0 and dl without the CE term, against the oracle,
    in the forward's emission and in the backward's re-emission."""
    hidden, weight, target, slots, kw, markov = _case("dense")
    y = slots.target_ids.clone()
    y.view(-1)[[0, 7, 64, 135]] = -100
    slots = synthetic.Slots(slots.weights, y, slots.valid)
    o = Objective(block_size=8)
    m, saved = head.lm_head_ce_kl_loss(hidden, weight, target, slots, o, accumulation_steps=2, **kw)
    dl2 = saved.dlogits.clone()
    head.lm_head_ce_kl_backward(saved, 2)                                   # hands the emitted dl over
    _, dl2_again = head.lm_head_ce_kl_backward(saved, 2, return_dlogits=True)   # pass 2 again
    torch.cuda.synchronize()
    assert torch.equal(dl2_again.reshape(dl2.shape), dl2)
    assert np.all(_np(saved.row_stats)[[0, 7, 64, 135], 2] == 0.0)
    z = ref.lm_head_logits(_np(hidden), _np(weight), _np(markov))
    wt = _np(slots.weights).reshape(-1)
    yy = y.reshape(-1).cpu().numpy()
    m_ref, _ = ref.ce_kl_loss(z, _np(target), wt.reshape(-1, 8), yy.reshape(-1, 8), slots.valid.cpu().numpy(),
                              o.ce, o.kl)
    for f in ("ce", "kl", "numerator", "accept_len_sum"):
        assert float(getattr(m, f)) == pytest.approx(m_ref[f], rel=1e-4, abs=1e-6), f
    want = ref.ce_kl_backward(z, _np(target), wt, yy, o.ce, o.kl, accumulation_steps=2)
    got = _np(dl2).reshape(want.shape).astype(np.float64)
    tol = np.abs(want) * 2.0 ** -7 + 2e-5 * np.abs(want).max(axis=-1, keepdims=True)
    assert np.all(np.abs(got - want) <= tol)


def test_empty_batch(gpu_lib):
    d, v = 128, 4096
    hidden = torch.empty((0, 8, d), dtype=torch.bfloat16, device=DEV)
    weight = (0.02 * torch.randn((v, d), device=DEV)).bfloat16()
    teacher = torch.empty((0, 8, v), dtype=torch.bfloat16, device=DEV)
    slots = synthetic.Slots(torch.empty((0, 8), device=DEV), torch.empty((0, 8), dtype=torch.int64, device=DEV),
                            torch.empty((0, 8), dtype=torch.bool, device=DEV))
    m, saved = head.lm_head_ce_kl_loss(hidden, weight, teacher, slots, Objective(block_size=8))
    dh = head.lm_head_ce_kl_backward(saved, 2)
    torch.cuda.synchronize()
    assert dh.shape == (0, 8, d)
    assert float(m.denominator) == 0.0 and float(m.loss) == 0.0 and float(m.accept_len_total) == 0.0


@pytest.mark.parametrize("kind", ["dense", "factored"])
@pytest.mark.parametrize("fwd_steps,bwd_steps", [(1, 4), (4, 2), (2, 8)])
def test_power_of_two_steps_rescale_the_emitted_dl(gpu_lib, kind, fwd_steps, bwd_steps):
    """The reference passes accumulation_steps to the backward only (train.py:291, 301): a
    forward that emitted dl for one count and a backward for another differing by a power of
    two scale the emitted dl in place, with the bits a forward for that count emits."""
    hidden, weight, target, slots, kw, _ = _case(kind)
    o = Objective(block_size=8)
    _, s_want = head.lm_head_ce_kl_loss(hidden, weight, target, slots, o, accumulation_steps=bwd_steps, **kw)
    want = s_want.dlogits.clone()
    _, saved = head.lm_head_ce_kl_loss(hidden, weight, target, slots, o, accumulation_steps=fwd_steps, **kw)
    emitted = saved.dlogits
    dh, dl = head.lm_head_ce_kl_backward(saved, bwd_steps, return_dlogits=True)
    torch.cuda.synchronize()
    assert dl.data_ptr() == emitted.data_ptr()          # scaled in place, pass 2 not rerun
    assert torch.equal(dl.reshape(want.shape), want)
    assert torch.equal(dh, head.lm_head_ce_kl_backward(s_want, bwd_steps))
