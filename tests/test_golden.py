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
