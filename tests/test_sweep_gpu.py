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


def _fp8_case(i):
    r = np.random.default_rng(9000 + i)
    return int(r.integers(1, 1300)), 128 * int(r.integers(1, 7)), 128 * int(r.integers(1, 120))


@pytest.mark.parametrize("i", range(6))
def test_fp8_random(gpu_lib, i):
    """fp8_linear against the oracle's fp8_linear bound, and the producer's row LSE against fp64."""
    from nanospec_amd import ops
    from test_fp8_gpu import _assert_fp8_logits, _lse64

    n, d, v = _fp8_case(i)
    x, codes, scale = synthetic.fp8_teacher_inputs(n, d, v, 9100 + i, DEV)
    w8 = codes.view(torch.float8_e4m3fn)
    plain = ops.fp8_linear(x, w8, scale)
    spec = ops.fp8_teacher_logits(x, w8, scale)
    torch.cuda.synchronize()
    assert torch.equal(spec.logits, plain)
    _assert_fp8_logits(_np(plain), _np(x), codes.cpu().numpy(), scale.cpu().numpy())
    np.testing.assert_allclose(_np(spec.lse), _lse64(_np(plain)), rtol=2e-6, atol=2e-6)


def _markov_case(i):
    r = np.random.default_rng(9500 + i)
    return (8 * int(r.integers(1, 80)), 64 * int(r.integers(1, 6)), 8 * int(r.integers(8, 2000)),
            64 * int(r.integers(1, 6)))


@pytest.mark.parametrize("i", range(5))
def test_markov_factored_random(gpu_lib, i):
    """The factored Markov head (a second K segment of the head GEMM) forward and backward
    against the fp64 oracle: metrics, lse_z, z at the label, dl, dh, W2.grad and W1.grad."""
    from dh_bar import assert_dh_rows
    from nanospec_amd import head
    from oracle import objective_ref as ref
    from test_markov_gpu import _assert_grads, _inputs, _oracle

    n, d, v, r = _markov_case(i)
    hidden, weight, teacher, slots, mk = _inputs(n, d, v, r, 9600 + i)
    o = Objective(block_size=8)
    m, saved = head.lm_head_ce_kl_loss(hidden, weight, teacher, slots, o, markov=mk)
    g1 = (1e-3 * torch.randn((v, r), generator=torch.Generator(device=DEV).manual_seed(i), device=DEV)).bfloat16()
    w1_grad, w2_grad = g1.clone(), torch.full_like(g1, float("nan"))
    dh, dl = head.lm_head_ce_kl_backward(saved, return_dlogits=True, markov_grads=(w1_grad, w2_grad))
    torch.cuda.synchronize()
    z, m_ref, rows, dl_ref = _oracle(hidden, weight, teacher, slots, mk, o)
    got = {f: float(getattr(m, f)) for f in ("ce", "kl", "numerator", "denominator", "accept_len_sum",
                                              "accept_len_total")}
    for f, w in got.items():
        assert w == pytest.approx(m_ref[f], rel=1e-4, abs=1e-6 * max(1.0, abs(m_ref[f]))), f
    rs = _np(saved.row_stats)
    np.testing.assert_allclose(rs[:, 0], rows["lse_z"], rtol=2e-6, atol=5e-5)
    np.testing.assert_allclose(rs[:, 5], z[np.arange(n), slots.target_ids.reshape(-1).cpu().numpy()],
                               rtol=1e-5, atol=1e-5)
    dln = _np(dl).reshape(n, -1)
    diff = np.abs(dln.astype(np.float64) - dl_ref)
    assert np.all(diff <= np.abs(dl_ref) * 2.0 ** -7 + 2e-5 * np.abs(dl_ref).max(axis=-1, keepdims=True))
    # the backward from the kernel's own dl: dh = dl . W_lm and the Markov gradients
    assert_dh_rows(_np(dh).reshape(n, -1), ref.lm_head_backward(dln, _np(weight)))
    _assert_grads(dl.reshape(n, -1), mk, g1, w1_grad, w2_grad)
