"""Seeded random shapes and settings, each against the fp64 oracle: the logits-level objective
(any V, bf16 or fp32 draft and teacher, independently) and the fused head (d a multiple of 64,
V a multiple of 8, with or without the dense Markov addend, bf16 or fp32 teacher, ragged or full
masks, gamma 0, 2 or 4).  The fixed shapes elsewhere pin each tiling edge on purpose; this sweep
looks for combinations nobody thought of.  Same bars as test_objective_gpu.py and
test_lmhead_gpu.py."""

import numpy as np
import pytest
import torch

from nanospec_amd import synthetic
from nanospec_amd.config import Objective

from test_lmhead_gpu import _check_full
from test_objective_gpu import _assert_dl_bf16, _assert_metrics, _metrics, _np, _oracle, _run

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _logits_case(i):
    r = np.random.default_rng(5000 + i)
    n = 8 * int(r.integers(1, 33))
    v = int(r.choice([int(r.integers(8, 64)), int(r.integers(64, 5000)), int(r.integers(5000, 260_000))]))
    tz = torch.bfloat16 if r.random() < 0.6 else torch.float32
    tu = torch.bfloat16 if r.random() < 0.6 else torch.float32
    gamma = float(r.choice([0.0, 2.0, 4.0]))
    return n, v, tz, tu, gamma


@pytest.mark.parametrize("i", range(12))
def test_logits_random(gpu_lib, i):
    n, v, tz, tu, gamma = _logits_case(i)
    z, u, slots = synthetic.logits_inputs(n, v, 6000 + i, DEV, gamma=gamma)
    z, u = z.to(tz), u.to(tu)
    o = Objective(block_size=8, gamma=gamma)
    m, saved, dl = _run(z, u, slots, o)
    m_ref, rows, dl_ref = _oracle(z, u, slots, o)
    _assert_metrics(_metrics(m), m_ref)
    rs = _np(saved.row_stats)
    np.testing.assert_allclose(rs[:, 0], rows["lse_z"], rtol=2e-6, atol=2e-5)
    np.testing.assert_allclose(rs[:, 1], rows["lse_u"], rtol=2e-6, atol=2e-5)
    np.testing.assert_allclose(rs[:, 4], rows["accept_rate"], atol=5e-6)
    zy = _np(z).reshape(n, v)[np.arange(n), slots.target_ids.reshape(-1).cpu().numpy()]
    np.testing.assert_array_equal(rs[:, 5], zy)
    if tz == torch.bfloat16:
        _assert_dl_bf16(_np(dl).reshape(n, v), dl_ref)
    else:
        _assert_dl_fp32(_np(dl).reshape(n, v), dl_ref, _np(z).reshape(n, v), _np(u).reshape(n, v), rows, slots, o)


def _assert_dl_fp32(dl, dl_ref, z, u, rows, slots, o):
    """fp32 dl = (w/acc) [(c_ce + c_kl) p - c_kl t - c_ce e_y]: within 1e-4 of itself plus
    2^-17 of the two terms it is the difference of.  Where (c_ce + c_kl) p and c_kl t nearly
    cancel, the error of p and t (each relative: from the log-normalisers, held to 2e-6 above,
    and from the per-entry exponential) stays that of the terms, not of their small difference
    (one such entry of 7296 at V = 38 missed a plain 1e-4 relative bar by 6x)."""
    w = _np(slots.weights).reshape(-1, 1).astype(np.float64)
    p = np.exp(z.astype(np.float64) - rows["lse_z"][:, None])
    t = np.exp(u.astype(np.float64) - rows["lse_u"][:, None])
    terms = w * ((o.ce + o.kl) * p + o.kl * t)
    diff = np.abs(dl.astype(np.float64) - dl_ref)
    tol = 1e-4 * np.abs(dl_ref) + 2.0 ** -17 * terms + 1e-30
    worst = float(((diff - 1e-4 * np.abs(dl_ref)) / (terms + 1e-30)).max())
    assert np.all(diff <= tol), f"needs {worst:.3g} of the terms"


def _head_case(i):
    r = np.random.default_rng(7000 + i)
    n = 8 * int(r.integers(1, 90))
    d = 64 * int(r.integers(1, 8))
    v = 8 * int(r.integers(1, 2500))
    markov = r.random() < 0.6
    fp32_teacher = r.random() < 0.3
    ragged = r.random() < 0.5
    gamma = float(r.choice([0.0, 2.0, 4.0]))
    return n, d, v, markov, fp32_teacher, ragged, gamma


@pytest.mark.parametrize("i", range(10))
def test_head_random(gpu_lib, i):
    n, d, v, markov, fp32_teacher, ragged, gamma = _head_case(i)
    hidden, weight, mk, teacher, slots = synthetic.head_inputs(n, d, v, 8000 + i, DEV, ragged=ragged, gamma=gamma)
    if fp32_teacher:
        teacher = teacher.float()
    _check_full(hidden, weight, mk if markov else None, teacher, slots, Objective(block_size=8, gamma=gamma))
