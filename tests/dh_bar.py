"""The north star's dhidden bar, applied per row (shared by the GPU tests).

On every row: max |dh - dh_ref| <= 2e-2 of that row's largest |dh_ref| and cosine >= 0.9999;
a row whose reference is exactly zero (a masked slot) is exactly zero.  This is the
compare.py:80-89 metric set (cosine, max_abs) taken row by row, which a whole-tensor
max_abs bar would let a small-norm row escape."""

import numpy as np


def assert_dh_rows(dh_gpu, dh_ref):
    g = np.asarray(dh_gpu, dtype=np.float64).reshape(-1, np.shape(dh_ref)[-1])
    w = np.asarray(dh_ref, dtype=np.float64).reshape(g.shape)
    rmax = np.abs(w).max(-1)
    live = rmax > 0
    assert np.all(g[~live] == 0.0)
    err = np.abs(g - w).max(-1)[live] / rmax[live]
    assert err.max() <= 2e-2, float(err.max())
    cos = (g * w).sum(-1)[live] / (np.linalg.norm(g, axis=-1)[live] * np.linalg.norm(w, axis=-1)[live])
    assert cos.min() >= 0.9999, float(cos.min())
