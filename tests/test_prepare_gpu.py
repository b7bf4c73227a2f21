"""GPU slot preparation (ns_prepare_slots) against the oracle: integer outputs
bit-exact, weights within a few fp32 ulp (exp implementations differ)."""

import numpy as np
import pytest
import torch

from nanospec_amd.config import Objective
from nanospec_amd.prepare import prepare_slots
from oracle import objective_ref as ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("b,s,nb,k,gamma", [(2, 19, 5, 4, 0.0), (3, 128, 32, 7, 4.0), (1, 6, 3, 3, 2.0),
                                            (4, 1000, 64, 8, 2.0)])
def test_prepare_matches_oracle(gpu_lib, b, s, nb, k, gamma):
    g = np.random.default_rng(b * 1000 + s)
    ids = g.integers(0, 248320, (b, s))
    mask = (g.uniform(0, 1, (b, s)) > 0.15).astype(np.float32)
    anchors = g.integers(0, s, (b, nb))
    keep = g.uniform(0, 1, (b, nb)) > 0.2
    o = Objective(block_size=k, num_anchors=nb, gamma=gamma)
    out = prepare_slots(torch.from_numpy(ids).to(DEV), torch.from_numpy(mask).to(DEV),
                        o, torch.from_numpy(anchors).to(DEV), torch.from_numpy(keep).to(DEV))
    torch.cuda.synchronize()
    want = ref.slot_preparation(ids, mask, anchors, keep, k, gamma)
    for key in ("target_ids", "previous", "valid", "teacher_indices"):
        np.testing.assert_array_equal(getattr(out, key).cpu().numpy(), want[key], err_msg=key)
    np.testing.assert_allclose(out.weights.cpu().numpy(), want["weights"], rtol=4e-7, atol=0)


def test_prepare_known_answer(gpu_lib):
    ids = torch.tensor([[10, 11, 12, 13, 14, 15]], device=DEV)
    mask = torch.tensor([[1, 1, 1, 0, 1, 1]], dtype=torch.float32, device=DEV)
    out = prepare_slots(ids, mask, Objective(block_size=3, gamma=2.0), torch.tensor([[0, 3, 0]], device=DEV),
                        torch.tensor([[True, True, False]], device=DEV))
    assert out.target_ids.tolist() == [[[11, 12, 13], [14, 15, 15], [10, 10, 10]]]
    assert out.valid.int().tolist() == [[[1, 1, 0], [1, 1, 0], [0, 0, 0]]]
    assert out.teacher_indices.tolist() == [[0, 1, 2, 3, 4, 4, 0, 0, 0]]


def test_prepare_empty_sequence_raises(gpu_lib):
    ids = torch.zeros((1, 0), dtype=torch.int64, device=DEV)
    with pytest.raises(ValueError, match="Empty input sequence"):
        prepare_slots(ids, torch.zeros((1, 0), device=DEV), Objective(block_size=3),
                      torch.zeros((1, 2), dtype=torch.int64, device=DEV),
                      torch.zeros((1, 2), dtype=torch.bool, device=DEV))
