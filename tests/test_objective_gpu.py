"""GPU parity of the logits-level objective (ns_ce_kl_logits_fwd / _bwd) against
the CPU oracle and the library-made golden vectors.

Tolerances (north star): loss, ce, kl, accept_len within 1e-4 relative of the
fp32 objective; token-index work (label pick) exact; dl within one bf16 ulp of
the exact value (bf16 logits) or 1e-4 relative (fp32 logits).
"""

import os

import numpy as np
import pytest
import torch

from nanospec_amd import objective as nobj
from nanospec_amd import synthetic
from nanospec_amd.config import Objective
from oracle import objective_ref as ref

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
FIELDS = ("ce", "kl", "numerator", "denominator", "accept_len_sum", "accept_len_total")
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "objective_small.npz")


def _np(t):
    return t.detach().float().cpu().numpy()


def _metrics(m):
    out = {f: float(getattr(m, f)) for f in FIELDS}
    out["loss"] = float(m.loss)
    out["accept_len"] = float(m.accept_len)
    return out


def _assert_metrics(got, want, rel=1e-4):
    for key in FIELDS + ("loss", "accept_len"):
        w = want[key]
        assert got[key] == pytest.approx(w, rel=rel, abs=1e-6 * max(1.0, abs(w))), (key, got[key], w)


def _assert_dl_bf16(dl_gpu, dl_ref):
    """bf16 dl: within one bf16 ulp of the exact value, and nearly always the
    correctly rounded value itself."""
    exact = ref.bf16_round(dl_ref.astype(np.float32))
    diff = np.abs(dl_gpu.astype(np.float64) - dl_ref)
    # one bf16 ulp, plus fp32-evaluation error where (c_ce+c_kl) p and c_kl t cancel
    scale = np.abs(dl_ref).max(axis=-1, keepdims=True)
    tol = np.abs(dl_ref) * 2.0 ** -7 + 1e-6 * scale
    assert np.all(diff <= tol), float((diff - tol).max())
    assert np.mean(dl_gpu == exact) > 0.999


def _run(z, u, slots, o, acc=1):
    metrics, saved = nobj.ce_kl_loss(z, u, slots, o, accumulation_steps=acc)
    dl = nobj.ce_kl_backward(saved, acc)
    torch.cuda.synchronize()
    return metrics, saved, dl


def _oracle(z, u, slots, o, acc=1):
    zn, un = _np(z).reshape(-1, z.shape[-1]), _np(u).reshape(-1, u.shape[-1])
    w, y, v = _np(slots.weights), slots.target_ids.cpu().numpy(), slots.valid.cpu().numpy()
    m, rows = ref.ce_kl_loss(zn, un, w, y, v, o.ce, o.kl)
    dl = ref.ce_kl_backward(zn, un, w.reshape(-1), y.reshape(-1), o.ce, o.kl, acc)
    return m, rows, dl


def test_golden_vectors(gpu_lib):
    g = dict(np.load(GOLDEN, allow_pickle=False))
    k = g["valid"].shape[-1]
    z = torch.from_numpy(g["z"]).to(DEV)
    u = torch.from_numpy(g["u"]).to(DEV)
    slots = synthetic.Slots(torch.from_numpy(g["weights"]).to(DEV),
                            torch.from_numpy(g["labels"]).view(-1, k).to(DEV),
                            torch.from_numpy(g["valid"]).to(DEV))
    o = Objective(block_size=k, ce=float(g["c_ce"]), kl=float(g["c_kl"]))
    acc = int(g["accumulation_steps"])
    for dtype in (torch.float32, torch.bfloat16):   # inputs are bf16-exact: identical values
        m, saved, dl = _run(z.to(dtype), u.to(dtype), slots, o, acc)
        want = {f: float(g[f]) for f in FIELDS}
        want["loss"] = want["numerator"] / max(want["denominator"], 1e-6)
        want["accept_len"] = want["accept_len_sum"] / max(want["accept_len_total"], 1.0)
        _assert_metrics(_metrics(m), want)
        rs = _np(saved.row_stats)
        np.testing.assert_allclose(rs[:, 2], g["ce_rows"], rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(rs[:, 3], g["kl_rows"], rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(rs[:, 4], g["accept_rows"], atol=2e-6)
        if dtype == torch.float32:
            np.testing.assert_allclose(_np(dl), g["dl"], rtol=1e-4, atol=1e-7)
        else:
            _assert_dl_bf16(_np(dl), g["dl"])


@pytest.mark.parametrize("n,v,dtype", [
    (64, 8192, torch.bfloat16),      # C0 shape
    (64, 8192, torch.float32),
    (32, 1001, torch.bfloat16),      # odd V: unaligned rows -> scalar path
    (16, 40000, torch.bfloat16),     # several vocab splits with a ragged last split
    (8, 250_008, torch.bfloat16),    # a bf16 row within the on-chip capacity (253,952): group path
    (8, 253_960, torch.bfloat16),    # a bf16 row past the on-chip capacity: two passes
])
def test_parity_small(gpu_lib, n, v, dtype):
    z, u, slots = synthetic.logits_inputs(n, v, 7 + n + v, DEV)
    z, u = z.to(dtype), u.to(dtype)
    o = Objective(block_size=8)
    m, saved, dl = _run(z, u, slots, o)
    m_ref, rows, dl_ref = _oracle(z, u, slots, o)
    _assert_metrics(_metrics(m), m_ref)
    rs = _np(saved.row_stats)
    np.testing.assert_allclose(rs[:, 0], rows["lse_z"], rtol=2e-6, atol=2e-5)
    np.testing.assert_allclose(rs[:, 1], rows["lse_u"], rtol=2e-6, atol=2e-5)
    np.testing.assert_allclose(rs[:, 4], rows["accept_rate"], atol=5e-6)
    # label pick is index work: z at the label is reproduced exactly
    zy = _np(z).reshape(n, v)[np.arange(n), slots.target_ids.reshape(-1).cpu().numpy()]
    np.testing.assert_array_equal(rs[:, 5], zy)
    if dtype == torch.bfloat16:
        _assert_dl_bf16(_np(dl).reshape(n, v), dl_ref)
    else:
        np.testing.assert_allclose(_np(dl).reshape(n, v), dl_ref, rtol=1e-4, atol=1e-8)


@pytest.mark.parametrize("n,v", [(32, 8), (32, 24), (32, 1000), (64, 8192), (24, 40000), (16, 248_320), (8, 253_952)])
def test_row_resident_path_matches_the_two_pass_path(gpu_lib, n, v):
    """bf16 rows within the on-chip capacity run four workgroups per row, each keeping its
    quarter of z and u on chip; the same values with an fp32 teacher run the two split passes.  Both restate
    objective.py:49-80 with the same per-entry formulas: metrics within 2e-6 relative, row
    statistics within fp32 summation-order error, dl equal except where an lse's last bit
    moves one entry's rounding."""
    z, u, slots = synthetic.logits_inputs(n, v, 300 + n, DEV)
    o = Objective(block_size=8)
    m_row, s_row, dl_row = _run(z, u, slots, o)
    m_two, s_two, dl_two = _run(z, u.float(), slots, o)
    for f in FIELDS:
        a, b = float(getattr(m_row, f)), float(getattr(m_two, f))
        assert a == pytest.approx(b, rel=2e-6, abs=1e-6), f
    np.testing.assert_allclose(_np(s_row.row_stats)[:, :5], _np(s_two.row_stats)[:, :5], rtol=2e-6, atol=2e-5)
    np.testing.assert_array_equal(_np(s_row.row_stats)[:, 5], _np(s_two.row_stats)[:, 5])
    assert float((dl_row == dl_two).float().mean()) > 0.999
    m_ref, _, _ = _oracle(z, u, slots, o)
    _assert_metrics(_metrics(m_row), m_ref)


@pytest.mark.parametrize("v", [8192, 40000])
def test_label_pick_at_vector_and_row_edges(gpu_lib, v):
    """Labels at the first and last entry of a row, at the edges of a 16-byte vector, on both
    sides of the boundaries between the four workgroups that share a row, at a column edge
    and in the last, partly filled column of the last member (V = 40000: 5000 vectors, 1250 per
    member, 4 full columns of 256 threads and 226 vectors in the fifth): z_label, CE and dl[y]
    exact against the oracle's pick."""
    n = 16
    z, u, slots = synthetic.logits_inputs(n, v, 400 + v, DEV)
    # member h holds vectors h * share .. (h + 1) * share - 1; its vector h * share + 256 i + t
    # (entries 8 q .. 8 q + 7) is column i of thread t
    threads, members = 256, 4
    nvec = v // 8
    share = -(-nvec // members)
    starts = [8 * share * h for h in range(1, members)]
    last_cols = (nvec - (members - 1) * share) // threads * threads
    last_partial = 8 * ((members - 1) * share + last_cols) % v
    picks = [0, v - 1, 7, 8, 1, 2] + [e for s in starts for e in (s - 1, s)] + \
        [8 * threads - 1, 8 * threads, last_partial, last_partial + 9]
    y = torch.tensor(picks, dtype=torch.int64, device=DEV).view(-1, 8)
    slots = synthetic.Slots(slots.weights, y, slots.valid)
    o = Objective(block_size=8)
    m, saved, dl = _run(z, u, slots, o)
    m_ref, rows, dl_ref = _oracle(z, u, slots, o)
    _assert_metrics(_metrics(m), m_ref)
    rs = _np(saved.row_stats)
    zy = _np(z)[np.arange(n), np.array(picks)]
    np.testing.assert_array_equal(rs[:, 5], zy)
    np.testing.assert_allclose(rs[:, 2], rows["ce"], rtol=2e-6, atol=2e-5)
    _assert_dl_bf16(_np(dl).reshape(n, v), dl_ref)


def test_accumulation_steps_and_reemission(gpu_lib):
    z, u, slots = synthetic.logits_inputs(32, 4096, 11, DEV)
    o = Objective(block_size=8)
    m, saved = nobj.ce_kl_loss(z, u, slots, o)
    dl1 = nobj.ce_kl_backward(saved, 1)          # the forward's own dl
    dl1b = nobj.ce_kl_backward(saved, 1)         # recomputed by the backward entry
    dl3 = nobj.ce_kl_backward(saved, 3)
    torch.cuda.synchronize()
    assert torch.equal(dl1, dl1b)
    _, _, dl_ref3 = _oracle(z, u, slots, o, acc=3)
    _assert_dl_bf16(_np(dl3).reshape(32, -1), dl_ref3)


def test_4d_layout_and_deterministic(gpu_lib):
    b, nb, k, v = 2, 3, 8, 5000
    z, u, slots = synthetic.logits_inputs(b * nb * k, v, 12, DEV)
    z4, u4 = z.view(b, nb, k, v), u.view(b, nb, k, v)
    slots4 = synthetic.Slots(slots.weights.view(b, nb, k), slots.target_ids.view(b, nb, k),
                             slots.valid.view(b, nb, k))
    o = Objective(block_size=k)
    m1, _, dl1 = _run(z4, u4, slots4, o)
    m2, _, dl2 = _run(z4, u4, slots4, o)
    assert dl1.shape == z4.shape and dl1.dtype == z4.dtype
    assert torch.equal(dl1, dl2)
    for f in FIELDS:
        assert torch.equal(getattr(m1, f), getattr(m2, f))


def test_empty_supervision(gpu_lib):
    z, u, slots = synthetic.logits_inputs(16, 2048, 13, DEV)
    slots = synthetic.Slots(torch.zeros_like(slots.weights), slots.target_ids, torch.zeros_like(slots.valid))
    m, _, dl = _run(z, u, slots, Objective(block_size=8))
    got = _metrics(m)
    assert got["denominator"] == 0.0 and got["accept_len_total"] == 0.0
    assert got["loss"] == 0.0 and got["accept_len"] == 0.0
    assert torch.count_nonzero(dl) == 0


def test_ignore_index_and_out_of_range_labels(gpu_lib):
    """Label -100 (F.cross_entropy's ignore_index, objective.py:54): CE 0 and no CE term in
    dl, as the oracle (pinned to torch's cross_entropy and autograd); any other label
    outside [0, V) makes the loss NaN instead of raising on the device."""
    z, u, slots = synthetic.logits_inputs(32, 3000, 15, DEV)
    y = slots.target_ids.clone()
    y.view(-1)[[2, 9, 17]] = -100
    slots = synthetic.Slots(slots.weights, y, slots.valid)
    o = Objective(block_size=8)
    m, saved, dl = _run(z, u, slots, o, acc=2)
    m_ref, rows, dl_ref = _oracle(z, u, slots, o, acc=2)
    _assert_metrics(_metrics(m), m_ref)
    assert np.all(_np(saved.row_stats)[[2, 9, 17], 2] == 0.0)
    _assert_dl_bf16(_np(dl).reshape(32, -1), dl_ref)
    y.view(-1)[4] = 3000
    m, _, _ = _run(z, u, synthetic.Slots(slots.weights, y, slots.valid), o)
    assert np.isnan(float(m.loss))


def test_nan_propagates(gpu_lib):
    """A NaN draft logit poisons ce, loss and accept_len whether or not its slot is valid
    (NaN * 0 = NaN in (ce * weights).sum() and cumprod(accept_rate * valid), objective.py:43,
    59); the full NaN / inf matrix is in test_nan_gpu.py."""
    z, u, slots = synthetic.logits_inputs(16, 2048, 14, DEV)
    for row in range(16):
        zr = z.clone()
        zr[row, 100] = float("nan")
        m, _, _ = _run(zr, u, slots, Objective(block_size=8))
        assert np.isnan(float(m.ce)) and np.isnan(float(m.loss)) and np.isnan(float(m.accept_len)), row
        assert np.isfinite(float(m.denominator)) and np.isfinite(float(m.accept_len_total)), row


def test_c1_full_size(gpu_lib):
    """C1 (N = 4096, V = 248,320): oracle parity on two whole blocks, and
    size-independent properties on every row."""
    z, u, slots = synthetic.c1(DEV)
    n, v = z.shape
    o = Objective(block_size=8)
    m, saved, dl = _run(z, u, slots, o)
    rs = _np(saved.row_stats)
    w = _np(slots.weights).reshape(-1).astype(np.float64)
    valid = slots.valid.cpu().numpy()
    # metrics are consistent with the per-row statistics
    den = w.sum()
    got = _metrics(m)
    assert got["denominator"] == pytest.approx(den, rel=1e-6)
    assert got["ce"] == pytest.approx((w * rs[:, 2]).sum() / den, rel=1e-5)
    assert got["kl"] == pytest.approx((w * rs[:, 3]).sum() / den, rel=1e-5)
    s, tot = ref.acceptance_length_counts(rs[:, 4].reshape(-1, 8), valid)
    assert got["accept_len_sum"] == pytest.approx(s, rel=1e-5) and got["accept_len_total"] == tot
    # oracle on whole blocks (row-local and block-local quantities)
    for blk in (0, 137):
        sl = slice(blk * 8, blk * 8 + 8)
        zs, us = _np(z[sl]), _np(u[sl])
        ys = slots.target_ids.reshape(-1)[sl].cpu().numpy()
        rows = ref.row_objective(zs, us, ys)
        np.testing.assert_allclose(rs[sl, 2], rows["ce"], rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(rs[sl, 3], rows["kl"], rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(rs[sl, 4], rows["accept_rate"], atol=5e-6)
        dl_ref = ref.ce_kl_backward(zs, us, w[sl], ys, o.ce, o.kl)
        _assert_dl_bf16(_np(dl[sl]), dl_ref)
    # every row of dl sums to ~0 and masked rows are exactly 0
    dlf = dl.float()
    row_sum = dlf.sum(-1).abs()
    row_abs = dlf.abs().sum(-1).clamp_min(1e-30)
    assert float((row_sum / row_abs).max()) < 1e-2
    masked = ~slots.valid.reshape(-1)
    assert torch.count_nonzero(dl[masked]) == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_power_of_two_steps_rescale_the_emitted_dl(gpu_lib, dtype):
    """ce_kl_loss emits dl for its accumulation_steps (1 when the caller passes none, as
    train.py:291 does); ce_kl_backward(saved, 4) then scales it in place, with the bits the
    forward would have emitted for 4; a count that is not a power-of-two multiple (3) runs the
    emit pass again."""
    z, u, slots = synthetic.logits_inputs(32, 4096, 16, DEV)
    z, u = z.to(dtype), u.to(dtype)
    o = Objective(block_size=8)
    _, s4 = nobj.ce_kl_loss(z, u, slots, o, accumulation_steps=4)
    want = nobj.ce_kl_backward(s4, 4)
    _, saved = nobj.ce_kl_loss(z, u, slots, o)
    emitted = saved.dlogits
    dl = nobj.ce_kl_backward(saved, 4)
    torch.cuda.synchronize()
    assert dl.data_ptr() == emitted.data_ptr() and torch.equal(dl, want)
    _, saved = nobj.ce_kl_loss(z, u, slots, o)
    dl3 = nobj.ce_kl_backward(saved, 3)
    _, s3 = nobj.ce_kl_loss(z, u, slots, o, accumulation_steps=3)
    torch.cuda.synchronize()
    assert torch.equal(dl3, nobj.ce_kl_backward(s3, 3))
