"""NaN and inf inputs propagate through every metric as in the reference: a NaN, +inf or
-inf logit in the draft (z) or teacher (u) row of a valid or a masked slot, at the logits
level (ns_ce_kl_logits_fwd) and through the fused head (ns_lmhead_ce_kl_fwd, the Markov
and teacher variants).

The reference forms accept_rate = torch.minimum(p, t).sum(-1) and
(accept_rate * valid).cumprod(-1) (objective.py:42-43), and the weighted sums
(ce * weights).sum() (objective.py:59): a NaN in a masked slot still reaches the
metrics (NaN * 0 = NaN), and -inf in u gives KL = 0 * (-inf) = NaN.  The oracle follows
those lines (np.minimum, cumprod of a * v) and is pinned to torch's evaluation of them in
tests/test_oracle.py.  Every check below: the six metrics, loss and accept_len are NaN
exactly where the oracle's are, equal where infinite, and within 1e-4 relative where
finite; the per-row CE, KL and accept rate have the oracle's NaN pattern.

A previous id outside [0, V) and a teacher row outside the teacher tensor make the
reference raise (an index error in F.embedding / gather).  The library reports them as
a NaN row instead: the oracle is fed the same row as NaN logits.
"""

import math

import numpy as np
import pytest
import torch

from nanospec_amd import head
from nanospec_amd import objective as nobj
from nanospec_amd import synthetic
from nanospec_amd.config import Objective
from oracle import objective_ref as ref

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
FIELDS = ("ce", "kl", "numerator", "denominator", "accept_len_sum", "accept_len_total")
NAN, INF = float("nan"), float("inf")
VALID_ROW, MASKED_ROW = 18, 11        # block 2 slot 2 (valid) and block 1 slot 3 (masked)

# (tensor, value, row, where): where = "entry" (one non-label entry), "label" (the label
# entry) or "row" (every entry of the row)
CASES = [(tensor, value, row, "entry") for tensor in ("z", "u") for value in (NAN, INF, -INF)
         for row in (VALID_ROW, MASKED_ROW)]
CASES += [("z", -INF, VALID_ROW, "label"), ("z", -INF, VALID_ROW, "row"), ("u", -INF, MASKED_ROW, "row")]


def _case_id(c):
    return f"{c[0]}{c[1]}-{'valid' if c[2] == VALID_ROW else 'masked'}-{c[3]}"


def _np(t):
    return t.detach().float().cpu().numpy()


def _slots(n, v, seed, k=8):
    """All slots valid except MASKED_ROW and two more in other blocks (w = 0 there)."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    valid = torch.ones((n // k, k), dtype=torch.bool, device=DEV)
    for r in (MASKED_ROW, 37, 52):
        valid.view(-1)[r] = False
    labels = torch.randint(0, v, (n // k, k), generator=g, device=DEV)
    return synthetic.Slots(synthetic.position_weights(valid, 4.0), labels, valid)


def _poison(x, case, labels):
    """x[row] poisoned in place as the case says (x is [N, V] bf16 or fp32)."""
    tensor, value, row, where = case
    y = int(labels.view(-1)[row])
    if where == "row":
        x[row] = value
    elif where == "label":
        x[row, y] = value
    else:
        x[row, (y + 101) % x.shape[1]] = value


def _same(got, want, what, rel=1e-4):
    if math.isnan(want):
        assert math.isnan(got), (what, got, want)
    elif math.isinf(want):
        assert got == want, (what, got, want)
    else:
        assert got == pytest.approx(want, rel=rel, abs=1e-6 * max(1.0, abs(want))), (what, got, want)


def _check(m, saved_rows, z, u, slots, o):
    """Metrics and row NaN patterns against the oracle on the same (poisoned) inputs."""
    w = _np(slots.weights)
    y = slots.target_ids.cpu().numpy()
    valid = slots.valid.cpu().numpy()
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        m_ref, rows = ref.ce_kl_loss(z, u, w, y, valid, o.ce, o.kl)
    for f in FIELDS:
        _same(float(getattr(m, f)), m_ref[f], f)
    _same(float(m.loss), m_ref["loss"], "loss")
    _same(float(m.accept_len), m_ref["accept_len"], "accept_len")
    rs = _np(saved_rows)
    for col, key in ((2, "ce"), (3, "kl"), (4, "accept_rate")):
        np.testing.assert_array_equal(np.isnan(rs[:, col]), np.isnan(rows[key]), err_msg=key)
        fin = np.isfinite(rows[key])
        np.testing.assert_array_equal(np.isfinite(rs[:, col]), fin, err_msg=key)
    return m_ref


@pytest.mark.parametrize("case", CASES, ids=_case_id)
def test_logits_level(gpu_lib, case):
    """C0 shape (N = 64, V = 8192), bf16 logits given directly."""
    n, v = 64, 8192
    z, u, _ = synthetic.logits_inputs(n, v, 70, DEV)
    slots = _slots(n, v, 71)
    _poison(z if case[0] == "z" else u, case, slots.target_ids)
    o = Objective(block_size=8)
    m, saved = nobj.ce_kl_loss(z, u, slots, o)
    dl = nobj.ce_kl_backward(saved)
    torch.cuda.synchronize()
    zn, un = _np(z), _np(u)
    m_ref = _check(m, saved.row_stats, zn, un, slots, o)
    assert math.isnan(m_ref["accept_len"]) == (case[1] != -INF or case[3] == "row")
    # dl: NaN in exactly the rows where the oracle's derivative is NaN
    with np.errstate(invalid="ignore", over="ignore"):
        dl_ref = ref.ce_kl_backward(zn, un, _np(slots.weights).reshape(-1), slots.target_ids.reshape(-1).cpu().numpy(),
                                    o.ce, o.kl)
    np.testing.assert_array_equal(np.isnan(_np(dl)).any(-1), np.isnan(dl_ref).any(-1))


def _head_oracle_z(hidden, weight, markov):
    return ref.lm_head_logits(_np(hidden), _np(weight), _np(markov))


@pytest.mark.parametrize("n,d,v", [(64, 256, 8192), (512, 128, 4096)])
@pytest.mark.parametrize("case", CASES, ids=_case_id)
def test_fused_head(gpu_lib, case, n, d, v):
    """z poisoned through the dense Markov addend (z = hidden . W^T + markov), u through the
    teacher logits.  N = 64 runs the general epilogue (a partial token tile), N = 512 the
    whole-tile one."""
    hidden, weight, markov, teacher, _ = synthetic.head_inputs(n, d, v, 72, DEV)
    slots = _slots(n, v, 73)
    _poison(markov if case[0] == "z" else teacher, case, slots.target_ids)
    o = Objective(block_size=8)
    m, saved = head.lm_head_ce_kl_loss(hidden, weight, teacher, slots, o, markov_logits=markov)
    torch.cuda.synchronize()
    _check(m, saved.row_stats, _head_oracle_z(hidden, weight, markov), _np(teacher), slots, o)


@pytest.mark.parametrize("row", [VALID_ROW, MASKED_ROW], ids=["valid", "masked"])
def test_bad_markov_id(gpu_lib, row):
    n, d, v, r = 64, 128, 2048, 64
    hidden, weight, _, teacher, _ = synthetic.head_inputs(n, d, v, 74, DEV)
    prev, w1, w2 = synthetic.markov_factors(n, v, r, 75, DEV)
    slots = _slots(n, v, 76)
    prev[row] = v
    o = Objective(block_size=8)
    m, saved = head.lm_head_ce_kl_loss(hidden, weight, teacher, slots, o, markov=head.MarkovFactors(prev, w1, w2))
    torch.cuda.synchronize()
    ok = prev.clone()
    ok[row] = 0
    z = ref.lm_head_logits(_np(hidden), _np(weight)) + ref.markov_logits(ok.cpu().numpy(), _np(w1), _np(w2))
    z[row] = np.nan
    _check(m, saved.row_stats, z, _np(teacher), slots, o)


@pytest.mark.parametrize("with_lse", [False, True], ids=["gathered", "teacher-once"])
@pytest.mark.parametrize("row", [VALID_ROW, MASKED_ROW], ids=["valid", "masked"])
def test_teacher_row_out_of_range(gpu_lib, row, with_lse):
    """A gathered teacher row past the teacher tensor, read in pass 1 (gathered) or with the
    producer's log-normalisers (teacher-once: pass 1 reads no teacher)."""
    n, d, v = 64, 128, 2048
    hidden, weight, markov, teacher, _ = synthetic.head_inputs(n, d, v, 77, DEV)
    slots = _slots(n, v, 78)
    rows = torch.arange(n, device=DEV)
    rows[row] = n
    lse = None
    if with_lse:
        lse = torch.logsumexp(teacher.float(), dim=-1)
    spec = head.TeacherLogits(teacher, rows, lse)
    o = Objective(block_size=8)
    m, saved = head.lm_head_ce_kl_loss(hidden, weight, spec, slots, o, markov_logits=markov)
    torch.cuda.synchronize()
    u = _np(teacher)
    u[row] = np.nan
    _check(m, saved.row_stats, _head_oracle_z(hidden, weight, markov), u, slots, o)
