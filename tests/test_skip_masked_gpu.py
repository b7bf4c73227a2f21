"""lm_head_ce_kl_loss(skip_masked_rows=True): pass 2 and the dh GEMM on the rows whose dl is not
all zero only.  Against the full pass on the same inputs: CE, KL, numerator, denominator and
accept_len_total bit for bit, accept_len_sum within 1e-6 (the accept rates of the rows kept come
from a pass over a different split of the vocabulary), dl bit for bit (zero rows where skipped,
as the reference's 0 * p - 0 * t), dh within the per-row dhidden bar and exactly zero on skipped
rows; against the oracle at the usual bars; NaN statistics in an unsupervised row keep it."""

import numpy as np
import pytest
import torch

from nanospec_amd import head, synthetic
from nanospec_amd.config import Objective

from dh_bar import assert_dh_rows

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
EXACT = ("ce", "kl", "numerator", "denominator", "accept_len_total")


def _both(hidden, weight, markov, teacher, slots, o, acc=1, bwd_acc=None):
    bwd_acc = acc if bwd_acc is None else bwd_acc
    out = []
    for skip in (False, True):
        m, saved = head.lm_head_ce_kl_loss(hidden, weight, teacher, slots, o, markov_logits=markov,
                                           accumulation_steps=acc, skip_masked_rows=skip)
        dh, dl = head.lm_head_ce_kl_backward(saved, bwd_acc, return_dlogits=True)
        out.append((m, saved, dh, dl))
    torch.cuda.synchronize()
    return out


def _assert_same(full, skip, masked):
    (mf, sf, dhf, dlf), (ms, ss, dhs, dls) = full, skip
    for f in EXACT:
        assert torch.equal(getattr(mf, f), getattr(ms, f)), f
    a, b = float(mf.accept_len_sum), float(ms.accept_len_sum)
    assert b == pytest.approx(a, rel=1e-6, abs=1e-6), (a, b)
    assert torch.equal(dlf, dls)
    n = dlf.reshape(-1, dlf.shape[-1]).shape[0]
    dhs2 = dhs.reshape(n, -1)
    assert torch.equal(dhs2[masked], torch.zeros_like(dhs2[masked]))
    assert_dh_rows(dhs2.float().cpu().numpy(), dhf.reshape(n, -1).float().cpu().numpy())
    np.testing.assert_array_equal(sf.row_stats[:, :4].cpu().numpy(), ss.row_stats[:, :4].cpu().numpy())


def _masked(slots):
    return ((slots.valid.reshape(-1) == 0) & (slots.weights.reshape(-1) == 0)).cpu()


@pytest.mark.parametrize("n,d,v,markov,fp32_teacher", [
    (512, 256, 8192, True, False),
    (264, 192, 2056, False, True),
    (3072, 128, 16384, True, False),
])
def test_skip_matches_full_pass(gpu_lib, n, d, v, markov, fp32_teacher):
    hidden, weight, mk, teacher, slots = synthetic.head_inputs(n, d, v, 5100 + n, DEV, ragged=True, gamma=2.0)
    if fp32_teacher:
        teacher = teacher.float()
    o = Objective(block_size=8, gamma=2.0)
    full, skip = _both(hidden, weight, mk if markov else None, teacher, slots, o)
    masked = _masked(slots)
    assert 0 < int(masked.sum()) < n
    _assert_same(full, skip, masked)


def test_skip_against_the_oracle(gpu_lib):
    from oracle import objective_ref as ref
    from test_lmhead_gpu import _assert_dl, _assert_metrics, _metrics, _oracle_head

    hidden, weight, markov, teacher, slots = synthetic.head_inputs(256, 256, 4096, 5201, DEV, ragged=True)
    o = Objective(block_size=8)
    m, saved = head.lm_head_ce_kl_loss(hidden, weight, teacher, slots, o, markov_logits=markov,
                                       skip_masked_rows=True)
    dh, dl = head.lm_head_ce_kl_backward(saved, return_dlogits=True)
    torch.cuda.synchronize()
    z, m_ref, rows, dl_ref, dh_ref = _oracle_head(hidden, weight, markov, teacher, slots, o)
    _assert_metrics(_metrics(m), m_ref)
    _assert_dl(dl.float().cpu().numpy().reshape(256, -1), dl_ref)
    assert_dh_rows(dh.float().cpu().numpy().reshape(256, -1), dh_ref)
    del ref


def test_skip_keeps_unsupervised_rows_with_nan(gpu_lib):
    """A NaN in the hidden row of an unsupervised slot makes its statistics NaN: the row goes
    through pass 2 (dl and dh NaN there, as the reference's 0 * NaN), and the metrics match the
    full pass's NaN pattern."""
    n, d, v = 256, 256, 4096
    hidden, weight, markov, teacher, slots = synthetic.head_inputs(n, d, v, 5301, DEV, ragged=True)
    masked = _masked(slots)
    r = int(torch.nonzero(masked)[0])
    hidden = hidden.clone()
    hidden[r, 7] = float("nan")
    o = Objective(block_size=8)
    full, skip = _both(hidden, weight, markov, teacher, slots, o)
    (mf, _, dhf, dlf), (ms, _, dhs, dls) = full, skip
    for f in EXACT + ("accept_len_sum",):
        a, b = getattr(mf, f), getattr(ms, f)
        assert bool(torch.isnan(a)) == bool(torch.isnan(b)), f
    assert torch.equal(torch.isnan(dlf), torch.isnan(dls))
    assert torch.isnan(dls[r]).all() and torch.isnan(dhs[r]).all()
    assert torch.equal(torch.isnan(dhf), torch.isnan(dhs))


def test_skip_with_every_row_supervised_and_other_counts(gpu_lib):
    """No row to skip: the same kernels as the full pass, bit for bit.  Then a backward with
    another accumulation count: a power-of-two ratio rescales the kept dl (and its compact
    rows) in place, any other count re-runs pass 2 over every row."""
    hidden, weight, markov, teacher, slots = synthetic.head_inputs(256, 256, 4096, 5401, DEV)
    o = Objective(block_size=8)
    full, skip = _both(hidden, weight, markov, teacher, slots, o)
    for f in EXACT + ("accept_len_sum",):
        assert torch.equal(getattr(full[0], f), getattr(skip[0], f)), f
    assert torch.equal(full[2], skip[2]) and torch.equal(full[3], skip[3])
    hidden, weight, markov, teacher, slots = synthetic.head_inputs(256, 256, 4096, 5402, DEV, ragged=True)
    masked = _masked(slots)
    for bwd_acc in (4, 3):
        full, skip = _both(hidden, weight, markov, teacher, slots, o, acc=2, bwd_acc=bwd_acc)
        _assert_same(full, skip, masked)


def test_skip_at_c3(gpu_lib):
    """C3 (N = 32,768, ragged masks, gamma 2): the skipping pass against the full one."""
    hidden, weight, markov, teacher, slots = synthetic.c3(DEV)
    o = Objective(block_size=8, gamma=2.0)
    full, skip = _both(hidden, weight, markov, teacher, slots, o)
    masked = _masked(slots)
    (mf, sf, dhf, dlf), (ms, ss, dhs, dls) = full, skip
    for f in EXACT:
        assert torch.equal(getattr(mf, f), getattr(ms, f)), f
    assert float(ms.accept_len_sum) == pytest.approx(float(mf.accept_len_sum), rel=1e-6)
    assert torch.equal(dlf, dls)
    dhs2, dhf2 = dhs.reshape(-1, dhs.shape[-1]), dhf.reshape(-1, dhf.shape[-1])
    assert not dhs2[masked.to(DEV)].any()
    rows = torch.arange(0, dhs2.shape[0], 61, device=DEV)   # every 61st row through the dh bar
    assert_dh_rows(dhs2[rows].float().cpu().numpy(), dhf2[rows].float().cpu().numpy())


def test_skip_with_every_row_unsupervised(gpu_lib):
    """Nothing supervised: pass 2 runs on no row, dl and dh are all zero, the metrics those of
    the full pass."""
    hidden, weight, markov, teacher, slots = synthetic.head_inputs(128, 128, 2048, 5501, DEV)
    slots = synthetic.Slots(torch.zeros_like(slots.weights), slots.target_ids, torch.zeros_like(slots.valid))
    o = Objective(block_size=8)
    full, skip = _both(hidden, weight, markov, teacher, slots, o)
    for f in EXACT + ("accept_len_sum",):
        assert torch.equal(getattr(full[0], f), getattr(skip[0], f)), f
    assert not skip[3].any() and not skip[2].any()
    assert torch.equal(full[3], skip[3])


def test_skip_with_final_norm_and_dl_formed_on_request(gpu_lib):
    """The skipping forward keeps the compact dl; a backward that needs the [N, V] dl (the fused
    final_norm backward, or return_dlogits) forms it from the kept rows: dx, the norm weight's
    gradient and dl bit for bit those of the full pass, also after a power-of-two rescale."""
    from nanospec_amd import ops

    n, d, v = 512, 256, 4096
    hidden0, weight, markov, teacher, slots = synthetic.head_inputs(n, d, v, 5601, DEV, ragged=True)
    w = torch.ones(d, dtype=torch.bfloat16, device=DEV)
    hidden, saved_norm = ops.rms_norm(hidden0, w, 1e-6)
    o = Objective(block_size=8)
    for bwd_acc in (1, 2):
        out = []
        for skip in (False, True):
            _, saved = head.lm_head_ce_kl_loss(hidden, weight, teacher, slots, o, markov_logits=markov,
                                               skip_masked_rows=skip)
            if skip:
                assert saved.dlogits is None and saved.compact is not None
            wg = torch.empty(d, dtype=torch.bfloat16, device=DEV)
            dx, dl = head.lm_head_ce_kl_backward(saved, bwd_acc, return_dlogits=True,
                                                 final_norm=(saved_norm, w, wg))
            out.append((dx, dl, wg))
        torch.cuda.synchronize()
        (dxf, dlf, wgf), (dxs, dls, wgs) = out
        assert torch.equal(dlf, dls)
        assert torch.equal(dxf, dxs) and torch.equal(wgf, wgs)
