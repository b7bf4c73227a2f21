"""Pins for the CPU oracle (oracle/objective_ref.py).

Each check is independent of the oracle's own formulas: torch library routines
(cross_entropy, kl_div, autograd, matmul, dtype casts), closed forms,
known answers worked by hand, and pure-Python brute force on tiny inputs.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import objective_ref as ref


def _logits(seed, n, v, scale=2.0, peak=6.0):
    g = np.random.default_rng(seed)
    z = scale * g.standard_normal((n, v))
    z[np.arange(n), g.integers(0, v, n)] += peak
    return z


# --------------------------------------------------------------------- CE / KL


def test_ce_matches_torch_cross_entropy():
    z = _logits(0, 32, 300)
    y = np.random.default_rng(1).integers(0, 300, 32)
    rows = ref.row_objective(z, z * 0.5, y)
    lib = F.cross_entropy(torch.from_numpy(z), torch.from_numpy(y), reduction="none").numpy()
    np.testing.assert_allclose(rows["ce"], lib, rtol=1e-12, atol=1e-12)


def test_kl_matches_torch_kl_div():
    z, u = _logits(2, 24, 257), _logits(3, 24, 257, scale=3.0, peak=8.0)
    y = np.zeros(24, dtype=np.int64)
    rows = ref.row_objective(z, u, y)
    zt, ut = torch.from_numpy(z), torch.from_numpy(u)
    lib = F.kl_div(zt.log_softmax(-1), ut.softmax(-1), reduction="none").sum(-1).numpy()
    np.testing.assert_allclose(rows["kl"], lib, rtol=1e-10, atol=1e-12)


def test_constant_logits_ce_is_log_vocab_and_equal_logits_kl_zero():
    v = 1000
    z = np.full((3, v), 1.7)
    rows = ref.row_objective(z, z, np.array([0, 5, 999]))
    np.testing.assert_allclose(rows["ce"], math.log(v), rtol=1e-14)
    np.testing.assert_allclose(rows["kl"], 0.0, atol=1e-14)
    np.testing.assert_allclose(rows["accept_rate"], 1.0, rtol=1e-12)


def test_accept_rate_total_variation_identity():
    z, u = _logits(4, 16, 500), _logits(5, 16, 500, scale=3.0, peak=8.0)
    rows = ref.row_objective(z, u, np.zeros(16, dtype=np.int64))
    p = torch.from_numpy(z).softmax(-1)
    t = torch.from_numpy(u).softmax(-1)
    tv = 0.5 * (p - t).abs().sum(-1)
    np.testing.assert_allclose(rows["accept_rate"], (1.0 - tv).numpy(), rtol=1e-10, atol=1e-12)


def test_accept_rate_brute_force_tiny():
    g = np.random.default_rng(6)
    z, u = g.standard_normal((3, 7)), g.standard_normal((3, 7))
    rows = ref.row_objective(z, u, np.zeros(3, dtype=np.int64))
    for i in range(3):
        ez = [math.exp(x) for x in z[i]]
        eu = [math.exp(x) for x in u[i]]
        sz, su = sum(ez), sum(eu)
        expect = sum(min(a / sz, b / su) for a, b in zip(ez, eu))
        assert abs(rows["accept_rate"][i] - expect) < 1e-12


def test_far_peaks_accept_near_zero():
    v = 64
    z = np.zeros((2, v))
    u = np.zeros((2, v))
    z[:, 3] = 60.0
    u[:, 40] = 60.0
    rows = ref.row_objective(z, u, np.zeros(2, dtype=np.int64))
    assert np.all(rows["accept_rate"] < 1e-20)


# ------------------------------------------------------------------ accept_len


def _brute_accept(a, valid):
    total, blocks = 0.0, 0
    for ab, vb in zip(a, valid):
        if not any(vb):
            continue
        blocks += 1
        length, prod = 1.0, 1.0
        for ai, vi in zip(ab, vb):
            prod *= ai * (1.0 if vi else 0.0)
            length += prod
        total += length
    return total, blocks


def test_acceptance_known_answers():
    valid = np.array([[1, 1, 1, 1], [1, 0, 1, 1], [0, 0, 0, 0], [1, 1, 0, 0]], dtype=bool)
    ones = np.ones((4, 4))
    s, tot = ref.acceptance_length_counts(ones, valid)
    # a = 1: length = 1 + leading run of valid slots -> 5, 2, (excluded), 3
    assert (s, tot) == (10.0, 3.0)
    zeros = np.zeros((4, 4))
    s, tot = ref.acceptance_length_counts(zeros, valid)
    assert (s, tot) == (3.0, 3.0)
    half = np.full((1, 3), 0.5)
    s, tot = ref.acceptance_length_counts(half, np.ones((1, 3), dtype=bool))
    assert s == pytest.approx(1 + 0.5 + 0.25 + 0.125) and tot == 1.0


def test_acceptance_brute_force_random():
    g = np.random.default_rng(7)
    a = g.uniform(0, 1, (9, 5))
    valid = g.uniform(0, 1, (9, 5)) > 0.3
    assert ref.acceptance_length_counts(a, valid) == pytest.approx(_brute_accept(a, valid), rel=1e-14)


def _torch_objective(z, u, w, y, valid, c_ce, c_kl):
    """torch's evaluation (fp64) of the forward objective as objective.py:42-46 and 53-60
    form it: torch.minimum, cumprod of accept_rate * valid, lengths * block_valid, and the
    weighted sums.  Its NaN and inf semantics (softmax of an inf, 0 * inf, minimum with a
    NaN) are torch's own."""
    k = valid.shape[-1]
    zt, ut = torch.from_numpy(z), torch.from_numpy(u)
    wt, vt = torch.from_numpy(w.reshape(-1).astype(np.float64)), torch.from_numpy(valid)
    ce = F.cross_entropy(zt, torch.from_numpy(y.reshape(-1)), reduction="none")
    probs, target = zt.softmax(-1), ut.softmax(-1)
    kl = (target * (ut.log_softmax(-1) - zt.log_softmax(-1))).sum(-1)
    accept = torch.minimum(probs, target).sum(-1)
    prefix = (accept.view(-1, k) * vt).cumprod(-1)
    block_valid = vt.any(-1)
    den = wt.sum()
    ce_s, kl_s = (ce * wt).sum(), (kl * wt).sum()
    acc_sum = ((prefix.sum(-1) + 1.0) * block_valid).sum()
    return dict(ce=float(ce_s / den.clamp_min(1e-6)), kl=float(kl_s / den.clamp_min(1e-6)),
                numerator=float(c_ce * ce_s + c_kl * kl_s), denominator=float(den), accept_len_sum=float(acc_sum),
                accept_len_total=float(block_valid.double().sum())), accept.numpy(), kl.numpy(), ce.numpy()


@pytest.mark.parametrize("tensor", ["z", "u"])
@pytest.mark.parametrize("value", [np.nan, np.inf, -np.inf])
@pytest.mark.parametrize("where", ["entry", "label", "row"])
@pytest.mark.parametrize("masked", [False, True])
def test_non_finite_logits_match_torch(tensor, value, where, masked):
    """A NaN, +inf or -inf logit in z or u, in a valid or a masked slot: the oracle's metrics
    and per-row CE, KL and accept rate are NaN / inf exactly where torch's evaluation of the
    reference's lines is, and equal elsewhere (a masked slot's NaN accept rate still poisons
    accept_len_sum through cumprod(accept * valid))."""
    n, v, k = 16, 97, 8
    z, u = _logits(30, n, v), _logits(31, n, v, scale=3.0, peak=8.0)
    y = np.random.default_rng(32).integers(0, v, n)
    valid = np.ones((n // k, k), dtype=bool)
    valid[1, 6] = False
    row = 14 if masked else 5
    valid[row // k, row % k] = not masked
    w = ref.slot_weights(valid, 4.0)
    x = z if tensor == "z" else u
    if where == "row":
        x[row] = value
    elif where == "label":
        x[row, y[row]] = value
    else:
        x[row, (y[row] + 7) % v] = value
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        m, rows = ref.ce_kl_loss(z, u, w, y.reshape(-1, k), valid, 0.1, 0.9)
    want, accept, kl, ce = _torch_objective(z, u, w, y, valid, 0.1, 0.9)
    for key, val in want.items():
        if math.isnan(val):
            assert math.isnan(m[key]), key
        else:
            assert m[key] == pytest.approx(val, rel=1e-12), key
    for got, lib in ((rows["accept_rate"], accept), (rows["kl"], kl), (rows["ce"], ce)):
        np.testing.assert_array_equal(np.isnan(got), np.isnan(lib))
        fin = np.isfinite(lib)
        np.testing.assert_array_equal(np.isfinite(got), fin)
        np.testing.assert_array_equal(got[~fin & ~np.isnan(lib)], lib[~fin & ~np.isnan(lib)])
        np.testing.assert_allclose(got[fin], lib[fin], rtol=1e-12, atol=1e-12)


def test_metrics_from_chunked_rows_equal_the_whole_batch():
    """Row statistics formed chunk by chunk give the whole batch's metrics (every row
    statistic is row-local), bit for bit."""
    n, v, k = 48, 301, 8
    z, u = _logits(40, n, v), _logits(41, n, v, scale=3.0, peak=8.0)
    y = np.random.default_rng(42).integers(0, v, n).reshape(-1, k)
    valid = np.random.default_rng(43).uniform(size=(n // k, k)) > 0.2
    w = ref.slot_weights(valid, 2.0)
    m, rows = ref.ce_kl_loss(z, u, w, y, valid, 0.1, 0.9)
    parts = [ref.ce_kl_loss(z[i:i + 16], u[i:i + 16], w[i // k:(i + 16) // k], y[i // k:(i + 16) // k],
                            valid[i // k:(i + 16) // k], 0.1, 0.9)[1] for i in range(0, n, 16)]
    joined = {key: np.concatenate([p[key] for p in parts]) for key in rows}
    assert ref.metrics_from_rows(joined, w, valid, 0.1, 0.9) == m


def test_empty_batch_metrics():
    v, k = 16, 4
    z = np.zeros((2 * k, v))
    m, _ = ref.ce_kl_loss(z, z, np.zeros((2, k)), np.zeros((2, k), dtype=np.int64), np.zeros((2, k), dtype=bool))
    assert m["denominator"] == 0.0 and m["accept_len_total"] == 0.0
    assert m["loss"] == 0.0 and m["accept_len"] == 0.0


# ------------------------------------------------------------------ loss / dl


def _library_loss(z, u, w, y, c_ce, c_kl, acc=1):
    zt = torch.from_numpy(z).requires_grad_(True)
    ut = torch.from_numpy(u)
    wt = torch.from_numpy(w.astype(np.float64))
    ce = F.cross_entropy(zt, torch.from_numpy(y), reduction="none")
    kl = F.kl_div(zt.log_softmax(-1), ut.softmax(-1), reduction="none").sum(-1)
    num = c_ce * (ce * wt).sum() + c_kl * (kl * wt).sum()
    (num / acc).backward()
    return num.item(), (ce * wt).sum().item(), (kl * wt).sum().item(), zt.grad.numpy()


def test_loss_and_dl_match_torch_library_and_autograd():
    n, v, k = 24, 333, 8
    z, u = _logits(8, n, v), _logits(9, n, v, scale=3.0, peak=8.0)
    g = np.random.default_rng(10)
    y = g.integers(0, v, n)
    valid = np.ones((n // k, k), dtype=bool)
    valid[1, 5:] = False
    w = ref.slot_weights(valid, 4.0).reshape(-1)
    m, _ = ref.ce_kl_loss(z, u, w.reshape(-1, k), y.reshape(-1, k), valid, 0.1, 0.9)
    num, ce_sum, kl_sum, grad = _library_loss(z, u, w, y, 0.1, 0.9, acc=3)
    den = float(w.astype(np.float64).sum())
    assert m["numerator"] == pytest.approx(num, rel=1e-12)
    assert m["ce"] == pytest.approx(ce_sum / den, rel=1e-12)
    assert m["kl"] == pytest.approx(kl_sum / den, rel=1e-12)
    dl = ref.ce_kl_backward(z, u, w, y, 0.1, 0.9, accumulation_steps=3)
    np.testing.assert_allclose(dl, grad, rtol=1e-9, atol=1e-15)


def test_ignore_index_matches_torch_cross_entropy_and_autograd():
    """Label -100 is F.cross_entropy's default ignore_index (objective.py:54): CE 0 in the
    forward, and dl is the gradient of that loss (no CE term on the row)."""
    n, v, k = 16, 211, 8
    z, u = _logits(20, n, v), _logits(21, n, v, scale=3.0, peak=8.0)
    y = np.random.default_rng(22).integers(0, v, n)
    y[[1, 6, 9]] = ref.IGNORE_INDEX
    valid = np.ones((n // k, k), dtype=bool)
    w = ref.slot_weights(valid, 4.0).reshape(-1)
    rows = ref.row_objective(z, u, y)
    lib = F.cross_entropy(torch.from_numpy(z), torch.from_numpy(y), reduction="none").numpy()
    np.testing.assert_allclose(rows["ce"], lib, rtol=1e-12, atol=1e-12)
    assert np.all(rows["ce"][[1, 6, 9]] == 0.0)
    m, _ = ref.ce_kl_loss(z, u, w.reshape(-1, k), y.reshape(-1, k), valid, 0.1, 0.9)
    num, _, _, grad = _library_loss(z, u, w, y, 0.1, 0.9, acc=2)
    assert m["numerator"] == pytest.approx(num, rel=1e-12)
    dl = ref.ce_kl_backward(z, u, w, y, 0.1, 0.9, accumulation_steps=2)
    np.testing.assert_allclose(dl, grad, rtol=1e-9, atol=1e-15)
    with pytest.raises(ValueError):
        ref.row_objective(z, u, np.full(n, -1))
    with pytest.raises(ValueError):
        ref.ce_kl_backward(z, u, w, np.full(n, v), 0.1, 0.9)


def test_dl_invariants():
    n, v = 16, 129
    z, u = _logits(11, n, v), _logits(12, n, v)
    y = np.random.default_rng(13).integers(0, v, n)
    w = np.linspace(0, 1, n).astype(np.float32)
    dl = ref.ce_kl_backward(z, u, w, y, 0.1, 0.9)
    np.testing.assert_allclose(dl.sum(-1), 0.0, atol=1e-12)
    assert np.all(dl[0] == 0.0)
    dl4 = ref.ce_kl_backward(z, u, w, y, 0.1, 0.9, accumulation_steps=4)
    np.testing.assert_allclose(dl4 * 4, dl, rtol=1e-13, atol=1e-18)


def test_den_clamp():
    k, v = 2, 8
    z = np.random.default_rng(14).standard_normal((k, v))
    w = np.full((1, k), 1e-9, dtype=np.float32)
    m, _ = ref.ce_kl_loss(z, z, w, np.zeros((1, k), dtype=np.int64), np.ones((1, k), dtype=bool))
    assert m["loss"] == pytest.approx(m["numerator"] / 1e-6)


# --------------------------------------------------------------- GEMM / head


def test_lm_head_matches_torch_matmul():
    g = np.random.default_rng(15)
    h, w, mk = g.standard_normal((5, 64)), 0.02 * g.standard_normal((96, 64)), g.standard_normal((5, 96))
    z = ref.lm_head_logits(h, w, mk)
    lib = (torch.from_numpy(h) @ torch.from_numpy(w).T + torch.from_numpy(mk)).numpy()
    np.testing.assert_allclose(z, lib, rtol=1e-12, atol=1e-12)
    dl = g.standard_normal((5, 96))
    dh = ref.lm_head_backward(dl, w)
    np.testing.assert_allclose(dh, (torch.from_numpy(dl) @ torch.from_numpy(w)).numpy(), rtol=1e-12)
    np.testing.assert_allclose(ref.lm_head_backward(2 * dl, w), 2 * dh, rtol=1e-13)


def test_markov_head_matches_torch_embedding_linear_and_autograd():
    """Forward = F.linear(F.embedding(prev, w1), w2) (train.py:278-279); the three
    gradients = torch.autograd of sum(dl * logits), which is what the reference's
    handwritten linear_backward / embedding_backward compute (ops.py:38-45, 73-74)."""
    g = np.random.default_rng(33)
    n, v, r = 12, 40, 8
    prev = g.integers(0, v, n)
    prev[3] = prev[7] = prev[9] = 5            # repeated ids: index_add sums their rows
    w1, w2, dl = g.standard_normal((v, r)), g.standard_normal((v, r)), g.standard_normal((n, v))
    tw1 = torch.from_numpy(w1).requires_grad_()
    tw2 = torch.from_numpy(w2).requires_grad_()
    tprev = torch.from_numpy(prev)
    e = F.embedding(tprev, tw1)
    e.retain_grad()
    logits = F.linear(e, tw2)
    np.testing.assert_allclose(ref.markov_logits(prev, w1, w2), logits.detach().numpy(), rtol=1e-12, atol=1e-12)
    (logits * torch.from_numpy(dl)).sum().backward()
    dprev, dw2, dw1 = ref.markov_backward(dl, prev, w1, w2)
    np.testing.assert_allclose(dprev, e.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dw2, tw2.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dw1, tw1.grad.numpy(), rtol=1e-12, atol=1e-12)
    # hand-worked index_add: row 5 collects rows 3, 7 and 9 of d(previous) (plus any other 5s)
    hits = np.flatnonzero(prev == 5)
    np.testing.assert_allclose(dw1[5], dprev[hits].sum(axis=0), rtol=1e-12)
    untouched = np.setdiff1d(np.arange(v), prev)
    assert np.all(dw1[untouched] == 0)


# --------------------------------------------------------------- formats / fp8


def test_bf16_round_matches_torch():
    g = np.random.default_rng(16)
    x = (g.standard_normal(10000) * np.exp(g.uniform(-20, 20, 10000))).astype(np.float32)
    x[:4] = [0.0, -0.0, 1e-40, 3.0e38]
    lib = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(ref.bf16_round(x), lib)


def test_e4m3_encode_matches_torch_cast():
    g = np.random.default_rng(17)
    x = np.concatenate([
        g.uniform(-448, 448, 20000),
        g.standard_normal(20000) * 0.01,
        ref.E4M3_VALUES[np.isfinite(ref.E4M3_VALUES)],
        # exact midpoints between neighbouring codes exercise ties-to-even
        0.5 * (ref._POS_VALUES[1:] + ref._POS_VALUES[:-1]),
    ]).astype(np.float32)
    codes = ref.e4m3_encode(x)
    lib = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(codes, lib)


def test_fp8_linear_exact_on_grid_with_power_of_two_scales():
    g = np.random.default_rng(18)
    n, d, v = 4, 256, 128
    finite = ref.E4M3_VALUES[np.isfinite(ref.E4M3_VALUES) & (np.abs(ref.E4M3_VALUES) <= 16)]
    # activations: per 1x128 block, include +-448 so the dynamic scale is exactly 1
    x = g.choice(finite, (n, d)).astype(np.float32)
    x[:, 0], x[:, 128] = 448.0, -448.0
    wc = ref.e4m3_encode(g.choice(finite, (v, d)))
    scale = np.array([[2.0 ** -3, 2.0 ** 2]], dtype=np.float32)
    out = ref.fp8_linear(x, wc, scale)
    sw = np.repeat(np.repeat(scale, 128, 0), 128, 1)
    exact = x.astype(np.float64) @ (ref.e4m3_decode(wc) * sw).astype(np.float64).T
    np.testing.assert_array_equal(out, ref.bf16_round(exact.astype(np.float32)))


def test_fp8_linear_matches_torch_float8_semantics():
    g = np.random.default_rng(19)
    n, d, v = 3, 256, 256
    x = ref.bf16_round(g.standard_normal((n, d)).astype(np.float32))
    w = (0.02 * g.standard_normal((v, d))).astype(np.float32)
    wc, s = ref.quantize_weight_blocks(w)
    # library restatement with torch's float8 cast
    xt = torch.from_numpy(x)
    xb = xt.float().reshape(n, -1, 128)
    xs = xb.abs().amax(-1, keepdim=True) / 448.0
    qx = (xb / xs.clamp_min(torch.finfo(torch.float32).tiny)).clamp(-448, 448).to(torch.float8_e4m3fn)
    dx = (qx.float() * xs).reshape(n, d)
    wq = torch.from_numpy(wc).view(torch.float8_e4m3fn)
    dw = (wq.float().view(v // 128, 128, d // 128, 128) * torch.from_numpy(s)[:, None, :, None]).reshape(v, d)
    lib = (dx.double() @ dw.double().T).float().to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(ref.fp8_linear(x, wc, s), lib)


def _torch_activation_codes(x):
    """ops.py:189-196 as torch tensor ops: (codes, scales) of x [n, d]."""
    xb = torch.from_numpy(x).reshape(x.shape[0], -1, 128)
    xs = xb.abs().amax(-1, keepdim=True) / 448.0
    q = (xb / xs.clamp_min(torch.finfo(torch.float32).tiny)).clamp(-448, 448).to(torch.float8_e4m3fn)
    return q.view(torch.uint8).reshape(x.shape).numpy(), xs[..., 0].numpy()


def test_fp8_non_finite_activation_poisons_its_row():
    """A NaN activation makes its block's scale and codes NaN, an infinity makes the scale
    inf and its own code NaN (inf / inf), as torch's amax / clamp / float8 cast do; either
    way that row's logits are NaN and the other rows are untouched."""
    g = np.random.default_rng(20)
    n, d, v = 4, 256, 256
    x = ref.bf16_round(g.standard_normal((n, d)).astype(np.float32))
    x[1, 5] = np.nan
    x[2, 130] = -np.inf
    codes, xs = ref.quantize_activation_blocks(x)
    t_codes, t_xs = _torch_activation_codes(x)
    np.testing.assert_array_equal(xs, t_xs)          # NaN at [1, 0], inf at [2, 1]
    nan_code = (codes & 0x7F) == 0x7F
    np.testing.assert_array_equal(nan_code, (t_codes & 0x7F) == 0x7F)   # NaN codes of either sign
    np.testing.assert_array_equal(codes[~nan_code], t_codes[~nan_code])
    assert nan_code[1, :128].all() and nan_code[2].sum() == 1
    wc, s = ref.quantize_weight_blocks((0.02 * g.standard_normal((v, d))).astype(np.float32))
    with np.errstate(invalid="ignore"):
        out = ref.fp8_linear(x, wc, s)
    assert np.isnan(out[1]).all() and np.isnan(out[2]).all()
    assert np.isfinite(out[[0, 3]]).all()


# ------------------------------------------------------------ slot preparation


def test_slot_preparation_known_answer():
    ids = np.array([[10, 11, 12, 13, 14, 15]])
    mask = np.array([[1, 1, 1, 0, 1, 1]], dtype=np.float32)
    anchors = np.array([[0, 3, 0]])
    keep = np.array([[True, True, False]])
    out = ref.slot_preparation(ids, mask, anchors, keep, block_size=3, gamma=2.0)
    # anchor 0: labels 1,2,3 -> ids 11,12,13; mask at 3 is 0 -> valid 1,1,0
    # anchor 3: labels 4,5,6 -> 6 >= s: ids 14,15,15(clamped); valid 1,1,0
    # not kept: safe index 0 everywhere, all invalid
    np.testing.assert_array_equal(out["target_ids"], [[[11, 12, 13], [14, 15, 15], [10, 10, 10]]])
    np.testing.assert_array_equal(out["valid"], [[[1, 1, 0], [1, 1, 0], [0, 0, 0]]])
    np.testing.assert_array_equal(out["previous"], [[[10, 11, 12], [13, 14, 15], [10, 10, 10]]])
    np.testing.assert_array_equal(out["teacher_indices"], [[0, 1, 2, 3, 4, 4, 0, 0, 0]])
    e = math.exp(-0.5)
    np.testing.assert_allclose(out["weights"], [[[1, e, 0], [1, e, 0], [0, 0, 0]]], rtol=1e-6)


def test_slot_preparation_brute_force():
    g = np.random.default_rng(20)
    b, s, nb, k = 2, 19, 5, 4
    ids = g.integers(0, 1000, (b, s))
    mask = (g.uniform(0, 1, (b, s)) > 0.2).astype(np.float32)
    anchors = g.integers(0, s, (b, nb))
    keep = g.uniform(0, 1, (b, nb)) > 0.25
    out = ref.slot_preparation(ids, mask, anchors, keep, k, 0.0)
    for i in range(b):
        for j in range(nb):
            alive = True
            for t in range(k):
                label = anchors[i, j] + t + 1
                idx = min(label, s - 1) if keep[i, j] else 0
                assert out["target_ids"][i, j, t] == ids[i, idx]
                alive = alive and keep[i, j] and label < s and mask[i, idx] > 0.5
                assert out["valid"][i, j, t] == alive
                assert out["weights"][i, j, t] == (1.0 if alive else 0.0)
                assert out["teacher_indices"][i, j * k + t] == max(idx - 1, 0)
                prev = ids[i, anchors[i, j]] if t == 0 else out["target_ids"][i, j, t - 1]
                assert out["previous"][i, j, t] == prev


def test_similarity_metrics():
    a = np.array([[1.0, 0.0], [0.0, 2.0]])
    e = np.array([[1.0, 0.0], [2.0, 0.0]])
    sim = ref.similarity(a, e)
    assert sim["cosine_min"] == pytest.approx(0.0, abs=1e-12)
    assert sim["cosine_mean"] == pytest.approx(0.5)
    assert sim["max_abs"] == pytest.approx(2.0)
    same = ref.similarity(e, e)
    assert same["cosine_min"] == pytest.approx(1.0) and same["relative_l2"] == 0.0
    z = np.array([[0.0, 0.0], [1.0, 1.0]])
    assert ref.similarity(z, z)["cosine_min"] == pytest.approx(1.0)
    assert ref.similarity(np.array([[1e-3, 0.0], [1.0, 1.0]]), z)["zero_rows_nonzero"] == 1


# --------------------------------------------------------------- pooled tail


def test_pooled_tail_hand_worked():
    """Two buffers: num 3 + 1, den 2 + 2, accept 10 + 6 over 4 + 4 blocks; world 2, acc 3."""
    m = np.array([[0.5, 0.25, 3.0, 2.0, 10.0, 4.0], [0.7, 0.1, 1.0, 2.0, 6.0, 4.0]], np.float32)
    loss, accept, factor, den = ref.pooled_tail(m, world_size=2, accumulation_steps=3)
    assert (loss, accept, factor, den) == (1.0, 2.0, 1.5, 4.0)
    # nothing supervised: factor 0, the 1e-6 clamp on the loss, accept total clamped to 1
    loss, accept, factor, den = ref.pooled_tail([[0, 0, 0.5, 0, 0, 0]], 4, 2)
    assert factor == 0.0 and den == 0.0 and accept == 0.0
    assert loss == np.float32(np.float32(0.5) / np.float32(1e-6))


def test_pooled_tail_matches_torch_evaluation_of_adamw_step():
    """shard.py:321-327 and train.py:533-534 evaluated by torch on fp32 tensors: the int
    over tensor division rounds twice (reciprocal, then product), which the oracle keeps."""
    g = np.random.default_rng(5)
    mismatch_if_divided = 0
    for trial in range(400):
        count = int(g.integers(1, 5))
        m = np.zeros((count, 6), np.float32)
        m[:, 2] = g.uniform(0, 50, count)
        m[:, 3] = g.uniform(0, 7, count) if trial % 10 else 0.0
        m[:, 4] = g.integers(0, 600, count)
        m[:, 5] = g.integers(0, 100, count)
        world, acc = int(g.integers(1, 9)), int(g.integers(1, 9))
        loss, accept, factor, den = ref.pooled_tail(m, world, acc)
        pooled = torch.zeros(4, dtype=torch.float32)
        for row in torch.from_numpy(m):
            pooled += row[2:]
        t_den = pooled[1].clone()
        t_factor = torch.where(t_den > 0, world * acc / t_den.clamp_min(1e-6), 0.0)
        assert float(pooled[0] / pooled[1].clamp_min(1e-6)) == loss
        assert float(pooled[2] / pooled[3].clamp_min(1.0)) == accept
        assert float(t_factor) == factor and float(t_den) == den
        if den > 0 and np.float32(world * acc) / max(den, np.float32(1e-6)) != factor:
            mismatch_if_divided += 1
        if den >= 1e-6:
            assert abs(float(factor) * float(den) - world * acc) <= 1e-6 * world * acc
    # the two-rounding form is observable: a plain division would differ on some inputs
    assert mismatch_if_divided > 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_scale_gradient_matches_torch_mul(dtype):
    """shard.py:330 grad.mul_(factor), bit-exact against torch's own products: fp32 times
    the 0-d fp32 factor; bf16 times the factor cast to bf16 (what the device kernel of
    mul_ computes for a bf16 tensor and a 0-d fp32 device tensor -- torch's CPU kernel
    keeps the fp32 factor instead, so the device semantics are pinned by the GPU test
    against torch's device mul_)."""
    g = torch.randn(5000, generator=torch.Generator().manual_seed(2)).to(dtype)
    for f in (1.0 / 3.7, 0.0, 2.0 ** -20 * 1.2345, 7.0):
        factor = torch.tensor(f, dtype=torch.float32)
        want = g.clone().mul_(factor.to(dtype)).float().numpy()
        got = ref.scale_gradient(g.float().numpy(), factor.item(), bf16=dtype == torch.bfloat16)
        assert np.array_equal(got, want), f


# --------------------------------------------------------------- final_norm


def _norm_case(n, d, seed):
    g = torch.Generator().manual_seed(seed)
    x = (2.0 * torch.randn(n, d, generator=g) + 0.5).bfloat16()
    w = (1.0 + 0.1 * torch.randn(d, generator=g)).bfloat16()
    return x.float().numpy(), w.float().numpy(), g


@pytest.mark.parametrize("n,d", [(7, 64), (33, 320)])
def test_rms_norm_matches_closed_form(n, d):
    x, w, _ = _norm_case(n, d, 3)
    eps = 1e-6
    out, inv, normalized = ref.rms_norm(x, w, eps)
    x64 = x.astype(np.float64)
    inv64 = 1.0 / np.sqrt((x64 ** 2).mean(-1) + eps)
    assert np.all(np.abs(inv - inv64) <= 4 * np.spacing(inv.astype(np.float32)))
    exact_n = x64 * inv64[:, None]
    assert np.all(np.abs(normalized - exact_n) <= np.abs(exact_n) * 2.0 ** -8 + 1e-30)
    exact_o = w.astype(np.float64) * exact_n
    assert np.all(np.abs(out - exact_o) <= np.abs(exact_o) * 2.0 ** -7 + 1e-30)
    # torch's own rms_norm (fp64) agrees with the closed form
    t = F.rms_norm(torch.from_numpy(x64), (d,), torch.from_numpy(w.astype(np.float64)), eps)
    np.testing.assert_allclose(t.numpy(), w * exact_n, rtol=1e-12)


@pytest.mark.parametrize("n,d", [(9, 64), (40, 320)])
def test_rms_norm_backward_matches_autograd(n, d):
    x, w, g = _norm_case(n, d, 4)
    eps = 1e-6
    _, inv, normalized = ref.rms_norm(x, w, eps)
    # dy correlated with the normalized input: the projection term is O(1) of dx
    dy = torch.from_numpy(normalized * w).clone()
    dy = (dy * 0.7 + 0.3 * torch.randn(n, d, generator=g)).bfloat16().float().numpy()
    dx, dw = ref.rms_norm_backward(dy, x, inv, w)
    tx = torch.from_numpy(x.astype(np.float64)).requires_grad_()
    tw = torch.from_numpy(w.astype(np.float64)).requires_grad_()
    y = tw * (tx * torch.rsqrt(tx.pow(2).mean(-1, keepdim=True) + eps))
    (y * torch.from_numpy(dy.astype(np.float64))).sum().backward()
    sim = ref.similarity(dx, tx.grad.numpy())
    assert sim["cosine_min"] >= 0.9999 and sim["relative_l2"] <= 5e-3, sim
    np.testing.assert_allclose(dw, tw.grad.numpy(), rtol=2e-2, atol=2e-2 * np.abs(tw.grad.numpy()).max())
    # a planted mistake (the dvar term dropped) is caught by the same bar
    dz = ref.bf16_round(dy * w)
    wrong = ref.bf16_round(dz * inv[:, None])
    assert ref.similarity(wrong, tx.grad.numpy())["cosine_min"] < 0.9999
