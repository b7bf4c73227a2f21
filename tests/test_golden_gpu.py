"""The HIP library against the torch-made golden fixtures of the head region
(tests/golden/head_small.npz, norm_small.npz), at the north-star tolerances: metrics within
1e-4 relative, dl within one bf16 ulp plus fp32 evaluation error, dh cosine >= 0.9999 and
max error <= 2e-2 of max |dh|, Markov gradients within bf16 output rounding, rms_norm within
one bf16 ulp (forward) and its propagation (backward)."""

import os

import numpy as np
import pytest
import torch

from nanospec_amd import head, ops
from nanospec_amd.config import Objective
from nanospec_amd.synthetic import Slots
from oracle import objective_ref as ref

from dh_bar import assert_dh_rows

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
HERE = os.path.join(os.path.dirname(__file__), "golden")
FIELDS = ("ce", "kl", "numerator", "denominator", "accept_len_sum", "accept_len_total")


def _bf16(bits):
    return torch.from_numpy(np.asarray(bits, dtype=np.uint16).view(np.int16)).view(torch.bfloat16).to(DEV)


def _np(t):
    return t.detach().float().cpu().numpy()


def test_head_golden_markov_teacher_rows(gpu_lib):
    gd = dict(np.load(os.path.join(HERE, "head_small.npz"), allow_pickle=False))
    hidden, weight = _bf16(gd["hidden"]), _bf16(gd["weight"])
    w1, w2 = _bf16(gd["w1"]), _bf16(gd["w2"])
    prev = torch.from_numpy(gd["prev"]).to(DEV)
    teacher = head.TeacherLogits(_bf16(gd["teacher"]), torch.from_numpy(gd["teacher_rows"]).to(DEV))
    k = gd["valid"].shape[-1]
    slots = Slots(torch.from_numpy(gd["weights"]).to(DEV), torch.from_numpy(gd["labels"].reshape(-1, k)).to(DEV),
                  torch.from_numpy(gd["valid"]).to(DEV))
    o = Objective(block_size=k, ce=float(gd["c_ce"]), kl=float(gd["c_kl"]))
    g1, g2 = torch.zeros_like(w1), torch.empty_like(w2)
    m, dh, dl = head.head_step(hidden, weight, teacher, slots, o, markov=head.MarkovFactors(prev, w1, w2),
                               markov_grads=(g1, g2))
    torch.cuda.synchronize()
    for f in FIELDS:
        w_ = float(gd[f])
        assert float(getattr(m, f)) == pytest.approx(w_, rel=1e-4, abs=1e-6 * max(1.0, abs(w_))), f
    dl_ref = gd["dl"].astype(np.float64)
    got = _np(dl).reshape(dl_ref.shape)
    tol = np.abs(dl_ref) * 2.0 ** -7 + 2e-5 * np.abs(dl_ref).max(axis=-1, keepdims=True)
    assert np.all(np.abs(got - dl_ref) <= tol), float((np.abs(got - dl_ref) - tol).max())
    assert_dh_rows(_np(dh).reshape(gd["dh"].shape), gd["dh"])
    # the Markov gradients follow the library's bf16 dl; bf16 output rounding plus that dl's error
    for got_g, want in ((g1, gd["dw1"]), (g2, gd["dw2"])):
        sim = ref.similarity(_np(got_g), want)
        assert sim["cosine"] >= 0.9999 and sim["relative_l2"] <= 1e-2, sim


def test_rms_norm_golden(gpu_lib):
    gd = dict(np.load(os.path.join(HERE, "norm_small.npz"), allow_pickle=False))
    x, w, dy = _bf16(gd["x"]), _bf16(gd["weight"]), _bf16(gd["dy"])
    out, saved = ops.rms_norm(x, w, float(gd["eps"]))
    wg = torch.empty_like(w)
    dx = ops.rms_norm_backward(dy, saved, w, wg)
    torch.cuda.synchronize()
    np.testing.assert_allclose(_np(out), gd["out"], rtol=2.0 ** -7, atol=1e-6)
    sim = ref.similarity(_np(dx), gd["dx"])
    assert sim["cosine_min"] >= 0.9999 and sim["relative_l2"] <= 1e-2, sim
    np.testing.assert_allclose(_np(wg), gd["dweight"], rtol=2e-2, atol=2e-2 * np.abs(gd["dweight"]).max())
