"""GPU parity of the block-FP8 teacher head (ns_fp8_quantize_rows,
ns_fp8_teacher_logits) against the oracle's ops.fp8_linear restatement.

Activation codes and scales are integer/format work: bit-exact.  Teacher logits
are bf16 of an fp32 sum whose order differs from the reference's fp32 GEMM:
within one bf16 ulp everywhere and identical for almost every entry.
"""

import numpy as np
import pytest
import torch

from nanospec_amd import head, ops, synthetic
from nanospec_amd.config import Objective
from oracle import objective_ref as ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _np(t):
    return t.detach().float().cpu().numpy()


def test_activation_quantisation_bit_exact(gpu_lib):
    g = torch.Generator(device=DEV).manual_seed(5)
    x = (torch.randn((96, 512), generator=g, device=DEV) * torch.logspace(-3, 2, 512, device=DEV)).bfloat16()
    x[3, 128:256] = 0.0              # an all-zero block quantises to exact zeros
    x[4, :128] = -0.0
    q, xs = ops.fp8_quantize_rows(x)
    torch.cuda.synchronize()
    q_ref, xs_ref = ref.quantize_activation_blocks(_np(x))
    np.testing.assert_array_equal(xs.cpu().numpy(), xs_ref)
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)


@pytest.mark.parametrize("n,d,v", [(64, 256, 1024), (200, 384, 2048)])
def test_fp8_linear_matches_oracle(gpu_lib, n, d, v):
    x, codes, scale = synthetic.fp8_teacher_inputs(n, d, v, 11 + n, DEV)
    out = ops.fp8_linear(x, codes.view(torch.float8_e4m3fn), scale)
    torch.cuda.synchronize()
    want = ref.fp8_linear(_np(x), codes.cpu().numpy(), scale.cpu().numpy())
    got = _np(out)
    ulp = np.abs(want) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(got - want) <= ulp), float((np.abs(got - want) - ulp).max())
    assert np.mean(got == want) > 0.99


def test_fp8_rejects_unblocked_shapes(gpu_lib):
    x = torch.zeros((4, 200), dtype=torch.bfloat16, device=DEV)
    w = torch.zeros((256, 200), dtype=torch.uint8, device=DEV).view(torch.float8_e4m3fn)
    with pytest.raises(ValueError, match="128x128"):
        ops.fp8_linear(x, w, torch.ones((2, 2), device=DEV))


def test_c4_teacher_fused_with_draft_path(gpu_lib):
    """C4 shape (N = 4096, d = 5120, V = 248,320): fp8 teacher logits on whole
    blocks against the oracle, then the fused objective on them."""
    hidden, weight, markov, (xt, codes, scale), slots = synthetic.c4(DEV)
    teacher = ops.fp8_linear(xt, codes.view(torch.float8_e4m3fn), scale)
    m, saved = head.lm_head_ce_kl_loss(hidden, weight, teacher, slots, Objective(block_size=8),
                                       markov_logits=markov)
    torch.cuda.synchronize()
    rows = np.arange(8 * 77, 8 * 78)
    want = ref.fp8_linear(_np(xt[rows]), codes.cpu().numpy(), scale.cpu().numpy())
    got = _np(teacher[rows])
    ulp = np.abs(want) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(got - want) <= ulp)
    assert np.mean(got == want) > 0.99
    assert np.isfinite(float(m.loss)) and 1.0 <= float(m.accept_len) <= 9.0
