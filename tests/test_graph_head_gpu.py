"""The fused head step (ns_lmhead_ce_kl_fwd + ns_lmhead_bwd through head.head_step) under HIP
graph capture.

The library allocates nothing and sets no memory with hipMemset: every launch, the dh GEMM's
launches by round included, is an ordinary kernel node.  A captured step replayed three times,
with eager fills of its outputs and synchronisations between the replays, must equal the eager
step bit for bit each time.
"""

import pytest
import torch

from nanospec_amd import head, synthetic
from nanospec_amd.config import Objective

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.mark.parametrize("n,d,v", [
    (64, 256, 8192),      # C0
    (32768, 3072, 2048),  # six rounds of dh tiles: one launch per round
])
def test_head_step_under_graph_capture(gpu_lib, n, d, v):
    hidden, weight, markov, teacher, slots = synthetic.head_inputs(n, d, v, 80 + d, DEV, ragged=True)
    o = Objective(block_size=8)

    def step():
        return head.head_step(hidden, weight, teacher, slots, o, markov_logits=markov)

    m0, dh0, dl0 = step()   # eager: also raises each kernel's LDS limit before the capture
    want = (torch.stack([m0.ce, m0.kl, m0.numerator, m0.denominator, m0.accept_len_sum, m0.accept_len_total]),
            dh0.clone(), dl0.clone())
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        m, dh, dl = step()
        got_m = torch.stack([m.ce, m.kl, m.numerator, m.denominator, m.accept_len_sum, m.accept_len_total])
    for rep in range(3):
        for t in (got_m, dh, dl):
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got_m, want[0]), rep
        assert torch.equal(dh, want[1]), rep
        assert torch.equal(dl, want[2]), rep
