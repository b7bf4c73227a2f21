"""GPU parity of the pooled-normalisation tail (ns_pooled_tail, ns_scale_gradient)
against the oracle (train.py:525-535, shard.py:318-330): scalar fp32 arithmetic in a
fixed order, so the results are bit-exact."""

import numpy as np
import pytest
import torch

from nanospec_amd import pooled
from nanospec_amd.objective import LossMetrics
from oracle import objective_ref as ref

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.mark.parametrize("count,world,acc", [(1, 1, 1), (3, 2, 4), (64, 8, 1)])
def test_pooled_tail_matches_oracle(gpu_lib, count, world, acc):
    g = np.random.default_rng(count)
    m = np.zeros((count, 6), np.float32)
    m[:, :2] = g.uniform(0, 10, (count, 2))
    m[:, 2] = g.uniform(0, 500, count)
    m[:, 3] = g.uniform(0, 60, count)
    m[:, 4] = g.integers(0, 4000, count)
    m[:, 5] = g.integers(0, 512, count)
    out = pooled.pooled_tail(torch.from_numpy(m).to(DEV), world, acc)
    want = ref.pooled_tail(m, world, acc)
    got = (out.loss, out.accept_len, out.factor, out.denominator)
    for x, y in zip(got, want):
        assert float(x) == float(y)


def test_pooled_tail_nothing_supervised_and_metrics_objects(gpu_lib):
    buf = torch.tensor([0.0, 0.0, 0.25, 0.0, 0.0, 0.0], device=DEV)
    out = pooled.pooled_tail([LossMetrics.from_buffer(buf), LossMetrics.from_buffer(buf.clone())], 2, 3)
    want = ref.pooled_tail(np.stack([buf.cpu().numpy()] * 2), 2, 3)
    assert float(out.factor) == 0.0 and float(out.accept_len) == 0.0
    assert float(out.loss) == float(want[0])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_scale_gradients_matches_torch_mul(gpu_lib, dtype):
    gen = torch.Generator(device=DEV).manual_seed(4)
    grads = [torch.randn(n, generator=gen, device=DEV).to(dtype) for n in (1, 7, 8, 4099, 1 << 20)]
    factor = torch.tensor(1.0 / 3.7, device=DEV)
    orig = [g.clone() for g in grads]
    want = [g.clone().mul_(factor) for g in grads]
    pooled.scale_gradients_(grads, factor)
    torch.cuda.synchronize()
    for g, w, o in zip(grads, want, orig):
        assert torch.equal(g, w)
        exact = ref.scale_gradient(o.float().cpu().numpy(), float(factor), bf16=dtype == torch.bfloat16)
        assert np.array_equal(exact, g.float().cpu().numpy())
