"""GPU parity of the teacher-logit side of the head (train.py:172-173, 280-290):
the teacher_indices gather done inside the head kernels' loads (ns_teacher_args.rows),
the teacher-logit producer with its per-row log-sum-exp (ns_lmhead_teacher_logits), and
the teacher-once forward that consumes that log-sum-exp (ns_teacher_args.lse).

A gathered load reads the same bytes as a gathered copy, so those results are bit-exact.
The teacher-once forward forms KL in the second pass (sum t (u - z) - lse_u + lse_z), so
its metrics are checked against the oracle at the usual 1e-4 relative bar."""

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


def _run(hidden, weight, teacher, slots, o, **kw):
    m, saved = head.lm_head_ce_kl_loss(hidden, weight, teacher, slots, o, **kw)
    torch.cuda.synchronize()
    return m, saved


def _lse64(x):
    x = np.asarray(x, dtype=np.float64)
    mx = x.max(-1, keepdims=True)
    return (mx + np.log(np.exp(x - mx).sum(-1, keepdims=True)))[..., 0]


@pytest.mark.parametrize("tdtype", [torch.bfloat16, torch.float32])
def test_gathered_teacher_rows_equal_a_gathered_copy(gpu_lib, tdtype):
    n, d, v, rows_total = 256, 128, 4096, 700
    hidden, weight, markov, _, slots = synthetic.head_inputs(n, d, v, 31, DEV)
    g = torch.Generator(device=DEV).manual_seed(32)
    full = (3.0 * torch.randn((rows_total, v), generator=g, device=DEV)).to(tdtype)
    rows = torch.randint(0, rows_total, (n,), generator=g, device=DEV)
    rows[5] = rows[6] = 17                      # repeated rows, as overlapping anchors give
    o = Objective(block_size=8)
    m1, s1 = _run(hidden, weight, head.TeacherLogits(full, rows), slots, o, markov_logits=markov)
    m2, s2 = _run(hidden, weight, full[rows].contiguous(), slots, o, markov_logits=markov)
    for f in FIELDS:
        assert torch.equal(getattr(m1, f), getattr(m2, f)), f
    assert torch.equal(s1.row_stats, s2.row_stats) and torch.equal(s1.dlogits, s2.dlogits)


def test_gathered_teacher_rows_more_than_4gib_apart(gpu_lib):
    # A bf16 teacher of 270,000 x 8192 (4.4 GB): gathered rows near both ends are more than
    # 4 GiB apart, so the head reads them itself instead of loading them into LDS (whose
    # loads take 32-bit offsets).  Same bar as above: equal to a gathered copy, bit for bit.
    n, d, v, rows_total = 256, 128, 8192, 270_000
    hidden, weight, markov, _, slots = synthetic.head_inputs(n, d, v, 36, DEV)
    g = torch.Generator(device=DEV).manual_seed(37)
    rows = torch.randint(0, 64, (n,), generator=g, device=DEV)
    rows[1::2] += rows_total - 64               # alternate between the first and last rows
    full = torch.empty((rows_total, v), dtype=torch.bfloat16, device=DEV)
    full[rows] = (3.0 * torch.randn((n, v), generator=g, device=DEV)).bfloat16()
    o = Objective(block_size=8)
    m1, s1 = _run(hidden, weight, head.TeacherLogits(full, rows), slots, o, markov_logits=markov)
    m2, s2 = _run(hidden, weight, full[rows].contiguous(), slots, o, markov_logits=markov)
    del full
    for f in FIELDS:
        assert torch.equal(getattr(m1, f), getattr(m2, f)), f
    assert torch.equal(s1.row_stats, s2.row_stats) and torch.equal(s1.dlogits, s2.dlogits)


def test_teacher_row_out_of_range_poisons_its_row(gpu_lib):
    n, d, v = 64, 128, 2048
    hidden, weight, markov, teacher, slots = synthetic.head_inputs(n, d, v, 33, DEV)
    rows = torch.arange(n, device=DEV)
    rows[9] = n                                 # past the teacher tensor
    m, saved = _run(hidden, weight, head.TeacherLogits(teacher, rows), slots, Objective(block_size=8),
                    markov_logits=markov)
    kl = _np(saved.row_stats)[:, 3]
    assert np.isnan(kl[9]) and np.all(np.isfinite(np.delete(kl, 9)))


def test_teacher_rows_helper_matches_torch_gather(gpu_lib):
    b, s, nbk, v = 2, 40, 16, 64
    g = torch.Generator(device=DEV).manual_seed(34)
    logits = torch.randn((b, s, v), generator=g, device=DEV)
    idx = torch.randint(0, s, (b, nbk), generator=g, device=DEV)
    want = logits.gather(1, idx.unsqueeze(-1).expand(-1, -1, v)).reshape(-1, v)     # train.py:286-290
    got = logits.reshape(-1, v)[head.teacher_rows(idx, s)]
    assert torch.equal(got, want)


@pytest.mark.parametrize("n,d,v,gathered", [(300, 128, 8200, False), (256, 256, 4096, True)])
def test_teacher_producer_logits_and_lse(gpu_lib, n, d, v, gathered):
    g = torch.Generator(device=DEV).manual_seed(35)
    rows_total = 2 * n if gathered else n
    x = torch.randn((rows_total, d), generator=g, device=DEV).bfloat16()
    w = (0.05 * torch.randn((v, d), generator=g, device=DEV)).bfloat16()
    rows = torch.randint(0, rows_total, (n,), generator=g, device=DEV) if gathered else None
    t = head.teacher_logits(x, w, rows)
    plain = head.lm_head_linear(x[rows].contiguous() if gathered else x, w)
    torch.cuda.synchronize()
    assert torch.equal(t.logits, plain)
    want = _lse64(_np(t.logits))
    np.testing.assert_allclose(_np(t.lse), want, rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("factored", [False, True])
def test_teacher_once_forward_matches_oracle(gpu_lib, factored):
    """Teacher logits from the producer (teacher hidden gathered at teacher rows through
    the LM head), consumed with their log-sum-exp: pass 1 reads no teacher."""
    n, d, v = 256, 256, 4096
    hidden, weight, markov, _, slots = synthetic.head_inputs(n, d, v, 36, DEV)
    g = torch.Generator(device=DEV).manual_seed(37)
    xt = (2.0 * torch.randn((3 * n, d), generator=g, device=DEV)).bfloat16()
    rows = torch.randint(0, 3 * n, (n,), generator=g, device=DEV)
    spec = head.teacher_logits(xt, weight, rows)
    o = Objective(block_size=8)
    kw = {}
    if factored:
        prev, w1, w2 = synthetic.markov_factors(n, v, 64, 38, DEV)
        kw["markov"] = head.MarkovFactors(prev, w1, w2)
    else:
        kw["markov_logits"] = markov
    m1, s1 = _run(hidden, weight, spec, slots, o, **kw)
    m2, s2 = _run(hidden, weight, spec.logits, slots, o, **kw)    # LSE formed in pass 1
    # the oracle on the same z and u
    z = ref.lm_head_logits(_np(hidden), _np(weight))
    if factored:
        z = z + ref.markov_logits(kw["markov"].previous.cpu().numpy(), _np(kw["markov"].w1), _np(kw["markov"].w2))
    else:
        z = z + _np(markov)
    u = _np(spec.logits)
    wt = _np(slots.weights).reshape(-1)
    y = slots.target_ids.reshape(-1).cpu().numpy()
    valid = slots.valid.cpu().numpy()
    m_ref, rows_ref = ref.ce_kl_loss(z, u, wt.reshape(-1, 8), y.reshape(-1, 8), valid, o.ce, o.kl)
    for f in FIELDS:
        w_ = m_ref[f]
        for m in (m1, m2):
            assert float(getattr(m, f)) == pytest.approx(w_, rel=1e-4, abs=1e-6 * max(1.0, abs(w_))), f
    np.testing.assert_allclose(_np(s1.row_stats)[:, 3], rows_ref["kl"], rtol=1e-4, atol=2e-5)
    dl_ref = ref.ce_kl_backward(z, u, wt, y, o.ce, o.kl)
    dl = _np(s1.dlogits).reshape(n, -1)
    tol = np.abs(dl_ref) * 2.0 ** -7 + 2e-5 * np.abs(dl_ref).max(axis=-1, keepdims=True)
    assert np.all(np.abs(dl.astype(np.float64) - dl_ref) <= tol)


def test_teacher_once_with_gathered_rows_and_per_row_lse(gpu_lib):
    """The verifier's layout (train.py:172-173, 285-290): logits and lse for all B*S
    teacher positions, gathered at the objective's rows inside the kernels."""
    n, d, v, rows_total = 256, 128, 4096, 640
    hidden, weight, markov, _, slots = synthetic.head_inputs(n, d, v, 39, DEV)
    g = torch.Generator(device=DEV).manual_seed(40)
    xt = (2.0 * torch.randn((rows_total, d), generator=g, device=DEV)).bfloat16()
    full = head.teacher_logits(xt, weight)                    # [R, V] with lse [R]
    rows = torch.randint(0, rows_total, (n,), generator=g, device=DEV)
    o = Objective(block_size=8)
    m1, s1 = _run(hidden, weight, head.TeacherLogits(full.logits, rows, full.lse), slots, o, markov_logits=markov)
    m2, s2 = _run(hidden, weight, full.logits[rows].contiguous(), slots, o, markov_logits=markov)
    for f in FIELDS:
        a, b = float(getattr(m1, f)), float(getattr(m2, f))
        assert a == pytest.approx(b, rel=2e-5, abs=1e-6), f
    np.testing.assert_allclose(_np(s1.row_stats)[:, 1], _np(s2.row_stats)[:, 1], rtol=1e-6, atol=1e-5)
