"""Write small golden vectors for the draft objective from torch library routines.

Independent of both the oracle and the HIP library: CE from
``F.cross_entropy``, KL from ``F.kl_div`` (the formulation of
experiments/reference.py:67), acceptance from softmax + minimum, and dl from
``torch.autograd`` on the weighted library loss, all in float64.  Inputs are
bf16-representable float32 values so every implementation sees identical
inputs.  Run: ``python tests/golden/make_golden.py`` (writes objective_small.npz).
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


if __name__ == "__main__":
    out = os.path.join(HERE, "objective_small.npz")
    np.savez_compressed(out, **make())
    print("wrote", out)
