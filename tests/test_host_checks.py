"""Host-side argument checks of the Python layer that must fire before any launch (no GPU
needed): a tensor whose raw pointer would reach a kernel must live on the device."""

import pytest
import torch

from nanospec_amd import head, ops

DEV = torch.device("cuda:0")   # only compared against, never allocated on


def test_markov_factors_on_the_host_are_refused():
    v, r, n = 64, 64, 8
    mk = head.MarkovFactors(torch.zeros(n, dtype=torch.int64), torch.zeros((v, r), dtype=torch.bfloat16),
                            torch.zeros((v, r), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="HIP device"):
        head._markov_inputs(mk, v, n, DEV)


def test_rms_norm_saved_state_on_the_host_is_refused():
    n, d = 4, 64
    x = torch.zeros((n, d), dtype=torch.bfloat16)
    saved = ops.RMSActivations(x, torch.ones((n, 1)), x.clone())
    w = torch.ones(d, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="HIP device"):
        ops.norm_args(saved, w, torch.zeros(d, dtype=torch.bfloat16), torch.empty((n, d), dtype=torch.bfloat16))
