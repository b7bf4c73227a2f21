"""Row-strided inputs: callers hand the library views of wider tensors (a leading dimension
above the row length), which the Python layer passes as ld without copying.  Every kernel that
reads rows by a pitch must then give the bits it gives for contiguous copies of the same values."""

import pytest
import torch

from nanospec_amd import head, objective, ops, synthetic
from nanospec_amd.config import Objective

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _padded(t, pad):
    """A view of `t` whose rows sit `pad` elements apart beyond their length (the padding NaN)."""
    rows = t.reshape(-1, t.shape[-1])
    wide = torch.full((rows.shape[0], rows.shape[1] + pad), float("nan"), dtype=t.dtype, device=t.device)
    wide[:, : rows.shape[1]] = rows
    v = wide[:, : rows.shape[1]]
    assert v.stride(0) == rows.shape[1] + pad
    return v.view(*t.shape[:-1], t.shape[-1]) if t.dim() == 2 else v


@pytest.mark.parametrize("n,v,dtype", [(64, 8192, torch.bfloat16), (48, 40000, torch.float32),
                                        (16, 248_320, torch.bfloat16)])
def test_logits_strided_rows(gpu_lib, n, v, dtype):
    z, u, slots = synthetic.logits_inputs(n, v, 4400 + n, DEV)
    z, u = z.to(dtype), u.to(dtype)
    o = Objective(block_size=8)
    m0, s0 = objective.ce_kl_loss(z, u, slots, o)
    dl0 = objective.ce_kl_backward(s0)
    zp, up = _padded(z, 24), _padded(u, 40)
    m1, s1 = objective.ce_kl_loss(zp, up, slots, o)
    dl1 = objective.ce_kl_backward(s1)
    torch.cuda.synchronize()
    for f in ("ce", "kl", "numerator", "denominator", "accept_len_sum", "accept_len_total"):
        assert torch.equal(getattr(m0, f), getattr(m1, f)), f
    assert torch.equal(s0.row_stats, s1.row_stats)
    assert torch.equal(dl0, dl1)


@pytest.mark.parametrize("n,d,v", [(64, 256, 8192), (520, 128, 4104)])
def test_head_strided_rows(gpu_lib, n, d, v):
    hidden, weight, markov, teacher, slots = synthetic.head_inputs(n, d, v, 4500 + n, DEV, ragged=True)
    o = Objective(block_size=8)
    m0, dh0, dl0 = head.head_step(hidden, weight, teacher, slots, o, markov_logits=markov)
    m1, dh1, dl1 = head.head_step(_padded(hidden, 64), _padded(weight, 128), _padded(teacher, 8), slots, o,
                                  markov_logits=_padded(markov, 16))
    torch.cuda.synchronize()
    for f in ("ce", "kl", "numerator", "denominator", "accept_len_sum", "accept_len_total"):
        assert torch.equal(getattr(m0, f), getattr(m1, f)), f
    assert torch.equal(dh0, dh1)
    assert torch.equal(dl0, dl1)


def test_dh_and_fp8_strided_rows(gpu_lib):
    g = torch.Generator(device=DEV).manual_seed(46)
    dl = (1e-3 * torch.randn((300, 8200), generator=g, device=DEV)).bfloat16()
    w = (0.02 * torch.randn((8200, 320), generator=g, device=DEV)).bfloat16()
    a = head.lm_head_linear_backward(dl, w)
    b = head.lm_head_linear_backward(_padded(dl, 56), _padded(w, 64))
    x, codes, scale = synthetic.fp8_teacher_inputs(200, 384, 2048, 47, DEV)
    w8 = codes.view(torch.float8_e4m3fn)
    c = ops.fp8_linear(x, w8, scale)
    e = ops.fp8_linear(_padded(x, 128), w8, scale)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert torch.equal(c, e)
