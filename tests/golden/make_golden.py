"""Write small golden vectors for the draft objective from torch library routines.

Independent of both the oracle and the HIP library: CE from
``F.cross_entropy``, KL from ``F.kl_div`` (the formulation of
experiments/reference.py:67), acceptance from softmax + minimum, and dl from
``torch.autograd`` on the weighted library loss, all in float64.  Inputs are
bf16-representable float32 values so every implementation sees identical
inputs.  Run: ``python tests/golden/make_golden.py`` (writes objective_small.npz,
head_small.npz and norm_small.npz; the first is unchanged by the other two).
"""

import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))


def make(seed=4242, nb=3, k=8, v=384, c_ce=0.1, c_kl=0.9, gamma=4.0, acc=2):
    g = torch.Generator().manual_seed(seed)
    n = nb * k
    z = (2.0 * torch.randn(n, v, generator=g)).bfloat16().float()
    u = (3.0 * torch.randn(n, v, generator=g)).bfloat16().float()
    peaks = torch.randint(0, v, (n,), generator=g)
    z[torch.arange(n), peaks] += 6.0
    u[torch.arange(n), torch.where(torch.rand(n, generator=g) < 0.6, peaks, torch.randint(0, v, (n,), generator=g))] += 8.0
    z, u = z.bfloat16().float(), u.bfloat16().float()
    y = torch.randint(0, v, (n,), generator=g)
    valid = torch.ones(nb, k, dtype=torch.bool)
    valid[1, 5:] = False          # truncated block
    valid[2, :] = False           # block with no supervision
    valid[0, 3] = False           # gap: later slots no longer count toward accept_len
    w = valid.float() * torch.exp(-torch.arange(k, dtype=torch.float32) / gamma)

    zd = z.double().requires_grad_(True)
    ud, wd = u.double(), w.reshape(-1).double()
    ce = F.cross_entropy(zd, y, reduction="none")
    kl = F.kl_div(zd.log_softmax(-1), ud.softmax(-1), reduction="none").sum(-1)
    num = c_ce * (ce * wd).sum() + c_kl * (kl * wd).sum()
    (num / acc).backward()
    with torch.no_grad():
        a = torch.minimum(zd.softmax(-1), ud.softmax(-1)).sum(-1)
        vf = valid.double()
        prefix = (a.view(nb, k) * vf).cumprod(-1)
        block_valid = valid.any(-1).double()
        acc_sum = ((prefix.sum(-1) + 1.0) * block_valid).sum()
        acc_tot = block_valid.sum()
        den = wd.sum()
    return dict(
        z=z.numpy(), u=u.numpy(), labels=y.numpy(), weights=w.numpy(), valid=valid.numpy(),
        c_ce=np.float64(c_ce), c_kl=np.float64(c_kl), accumulation_steps=np.int64(acc),
        ce_rows=ce.detach().numpy(), kl_rows=kl.detach().numpy(), accept_rows=a.numpy(),
        ce=(ce * wd).sum().item() / max(den.item(), 1e-6), kl=(kl * wd).sum().item() / max(den.item(), 1e-6),
        numerator=num.item(), denominator=den.item(), accept_len_sum=acc_sum.item(),
        accept_len_total=acc_tot.item(), dl=zd.grad.numpy(),
    )


def bf16_bits(t):
    """bf16 values as their uint16 bit patterns (half the bytes of float32)."""
    return t.bfloat16().view(torch.int16).numpy().view(np.uint16)


def make_head(seed=777, nb=8, k=8, d=128, v=512, r=64, rows_total=100, c_ce=0.1, c_kl=0.9, gamma=4.0):
    """The head region of train() (train.py:271-307) on a small case, from torch library
    routines in float64: z = hidden . W^T + linear(embedding(prev, w1), w2) (train.py:272-279),
    teacher logits gathered at teacher rows (train.py:285-290), the weighted CE + KL loss and
    acceptance as in make(), and torch.autograd for dl, dh, d(w1) and d(w2)."""
    g = torch.Generator().manual_seed(seed)
    n = nb * k
    hidden = torch.randn(n, d, generator=g).bfloat16()
    weight = (0.05 * torch.randn(v, d, generator=g)).bfloat16()
    prev = torch.randint(0, v, (n,), generator=g)
    prev[10] = prev[20] = prev[30] = 7             # repeated previous ids (index_add)
    w1 = torch.randn(v, r, generator=g).bfloat16()
    w2 = (0.05 * torch.randn(v, r, generator=g)).bfloat16()
    teacher = (3.0 * torch.randn(rows_total, v, generator=g)).bfloat16()
    rows = torch.randint(0, rows_total, (n,), generator=g)
    y = torch.randint(0, v, (n,), generator=g)
    valid = torch.ones(nb, k, dtype=torch.bool)
    valid[3, 4:] = False
    w = valid.float() * torch.exp(-torch.arange(k, dtype=torch.float32) / gamma)

    hd = hidden.double().requires_grad_(True)
    wd = weight.double()
    w1d = w1.double().requires_grad_(True)
    w2d = w2.double().requires_grad_(True)
    z = F.linear(hd, wd) + F.linear(F.embedding(prev, w1d), w2d)
    z.retain_grad()
    u = teacher.double()[rows]
    wts = w.reshape(-1).double()
    ce = F.cross_entropy(z, y, reduction="none")
    kl = F.kl_div(z.log_softmax(-1), u.softmax(-1), reduction="none").sum(-1)
    num = c_ce * (ce * wts).sum() + c_kl * (kl * wts).sum()
    num.backward()
    with torch.no_grad():
        a = torch.minimum(z.softmax(-1), u.softmax(-1)).sum(-1)
        prefix = (a.view(nb, k) * valid.double()).cumprod(-1)
        block_valid = valid.any(-1).double()
        den = wts.sum().item()
    return dict(
        hidden=bf16_bits(hidden), weight=bf16_bits(weight), prev=prev.numpy(), w1=bf16_bits(w1),
        w2=bf16_bits(w2), teacher=bf16_bits(teacher), teacher_rows=rows.numpy(), labels=y.numpy(),
        weights=w.numpy(), valid=valid.numpy(), c_ce=np.float64(c_ce), c_kl=np.float64(c_kl),
        ce=(ce * wts).sum().item() / den, kl=(kl * wts).sum().item() / den, numerator=num.item(),
        denominator=den, accept_len_sum=((prefix.sum(-1) + 1.0) * block_valid).sum().item(),
        accept_len_total=block_valid.sum().item(),
        dl=z.grad.float().numpy(), dh=hd.grad.float().numpy(), dw1=w1d.grad.float().numpy(),
        dw2=w2d.grad.float().numpy(),
    )


def make_norm(seed=778, n=48, d=320, eps=1e-6):
    """final_norm (ops.py:48-66) from torch in float64: out = weight * x / sqrt(mean(x^2) +
    eps) and torch.autograd of sum(dy * out) for dx and the weight gradient."""
    g = torch.Generator().manual_seed(seed)
    x = (2.0 * torch.randn(n, d, generator=g) + 0.25).bfloat16()
    weight = (1.0 + 0.1 * torch.randn(d, generator=g)).bfloat16()
    dy = torch.randn(n, d, generator=g).bfloat16()
    xd = x.double().requires_grad_(True)
    wd = weight.double().requires_grad_(True)
    out = F.rms_norm(xd, (d,), wd, eps)
    (out * dy.double()).sum().backward()
    return dict(x=bf16_bits(x), weight=bf16_bits(weight), dy=bf16_bits(dy), eps=np.float64(eps),
                out=out.detach().float().numpy(), dx=xd.grad.float().numpy(), dweight=wd.grad.float().numpy())


if __name__ == "__main__":
    for name, data in (("objective_small.npz", make()), ("head_small.npz", make_head()),
                       ("norm_small.npz", make_norm())):
        out = os.path.join(HERE, name)
        np.savez_compressed(out, **data)
        print("wrote", out)
