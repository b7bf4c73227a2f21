"""The oracle against the library-made golden vectors (tests/golden/)."""

import os

import numpy as np
import pytest

from oracle import objective_ref as ref

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "objective_small.npz")


@pytest.fixture(scope="module")
def gold():
    return dict(np.load(GOLDEN, allow_pickle=False))


def test_oracle_matches_golden_rows_and_metrics(gold):
    z, u, y = gold["z"], gold["u"], gold["labels"]
    k = gold["valid"].shape[-1]
    m, rows = ref.ce_kl_loss(z, u, gold["weights"], y.reshape(-1, k), gold["valid"],
                             float(gold["c_ce"]), float(gold["c_kl"]))
    np.testing.assert_allclose(rows["ce"], gold["ce_rows"], rtol=1e-12)
    np.testing.assert_allclose(rows["kl"], gold["kl_rows"], rtol=1e-10, atol=1e-13)
    np.testing.assert_allclose(rows["accept_rate"], gold["accept_rows"], rtol=1e-12)
    for key in ("ce", "kl", "numerator", "denominator", "accept_len_sum", "accept_len_total"):
        assert m[key] == pytest.approx(float(gold[key]), rel=1e-12), key


def test_oracle_matches_golden_dl(gold):
    dl = ref.ce_kl_backward(gold["z"], gold["u"], gold["weights"].reshape(-1), gold["labels"],
                            float(gold["c_ce"]), float(gold["c_kl"]), int(gold["accumulation_steps"]))
    np.testing.assert_allclose(dl, gold["dl"], rtol=1e-9, atol=1e-16)


HEAD = os.path.join(os.path.dirname(__file__), "golden", "head_small.npz")
NORM = os.path.join(os.path.dirname(__file__), "golden", "norm_small.npz")


def bf16_values(bits):
    """float32 values of bf16 bit patterns stored as uint16."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


@pytest.fixture(scope="module")
def head_gold():
    return dict(np.load(HEAD, allow_pickle=False))


@pytest.fixture(scope="module")
def norm_gold():
    return dict(np.load(NORM, allow_pickle=False))


def test_oracle_matches_golden_head_with_markov_and_teacher_rows(head_gold):
    """Dense head + factored Markov head + gathered teacher rows (train.py:271-307),
    against torch float64 autograd."""
    gd = head_gold
    h, w = bf16_values(gd["hidden"]), bf16_values(gd["weight"])
    w1, w2 = bf16_values(gd["w1"]), bf16_values(gd["w2"])
    z = ref.lm_head_logits(h, w) + ref.markov_logits(gd["prev"], w1, w2)
    u = bf16_values(gd["teacher"])[gd["teacher_rows"]]
    k = gd["valid"].shape[-1]
    m, _ = ref.ce_kl_loss(z, u, gd["weights"], gd["labels"].reshape(-1, k), gd["valid"],
                          float(gd["c_ce"]), float(gd["c_kl"]))
    for key in ("ce", "kl", "numerator", "denominator", "accept_len_sum", "accept_len_total"):
        assert m[key] == pytest.approx(float(gd[key]), rel=1e-10), key
    dl = ref.ce_kl_backward(z, u, gd["weights"].reshape(-1), gd["labels"], float(gd["c_ce"]), float(gd["c_kl"]))
    np.testing.assert_allclose(dl, gd["dl"], rtol=1e-5, atol=1e-9)
    np.testing.assert_allclose(ref.lm_head_backward(dl, w), gd["dh"], rtol=1e-5, atol=1e-8)
    _, dw2, dw1 = ref.markov_backward(dl, gd["prev"], w1, w2)
    np.testing.assert_allclose(dw2, gd["dw2"], rtol=1e-5, atol=1e-8)
    np.testing.assert_allclose(dw1, gd["dw1"], rtol=1e-5, atol=1e-8)


def test_oracle_matches_golden_rms_norm(norm_gold):
    """The oracle's rms_norm keeps the reference's bf16 roundings; the golden is exact
    float64, so they agree to bf16 rounding (forward) and to its propagation (backward)."""
    gd = norm_gold
    x, w, dy = bf16_values(gd["x"]), bf16_values(gd["weight"]), bf16_values(gd["dy"])
    out, inv, _ = ref.rms_norm(x, w, float(gd["eps"]))
    np.testing.assert_allclose(out, gd["out"], rtol=2.0 ** -7, atol=1e-6)
    dx, dw = ref.rms_norm_backward(dy, x, inv, w)
    sim = ref.similarity(dx, gd["dx"])
    assert sim["cosine_min"] >= 0.9999 and sim["relative_l2"] <= 1e-2, sim
    np.testing.assert_allclose(dw, gd["dweight"], rtol=2e-2, atol=2e-2 * np.abs(gd["dweight"]).max())
