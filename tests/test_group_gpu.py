"""The logits path's group kernel (four workgroups per row exchanging partial statistics
through the workspace) under HIP graph capture and on two streams at once.

Its per-call state (ticket counter, per-row finish counters, exchange words) is zeroed by a
kernel inside each call, so replays of a captured call and concurrent calls with their own
workspaces must each give the eager single-call result, bit for bit.
"""

import ctypes

import pytest
import torch

from nanospec_amd import _lib, synthetic
from nanospec_amd.objective import _slot_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _inputs(n, v, seed):
    z, u, slots = synthetic.logits_inputs(n, v, seed, DEV)
    w, y, valid, k = _slot_inputs(slots, n, torch.device(DEV))
    return z, u, w, y, valid, k


def _outputs(n, v):
    ws = torch.empty(int(_lib.load().ns_workspace_bytes(_lib.NS_WS_LOGITS, n, v, 0)), dtype=torch.uint8, device=DEV)
    return (torch.empty(6, device=DEV), torch.empty((n, 8), device=DEV),
            torch.empty((n, v), dtype=torch.bfloat16, device=DEV), ws)


def _call(lib, inp, out, stream):
    z, u, w, y, valid, k = inp
    metrics, row_stats, dl, ws = out
    n, v = z.shape
    return lib.ns_ce_kl_logits_fwd(
        _lib.ptr(z), _lib.NS_BF16, v, _lib.ptr(u), _lib.NS_BF16, v, _lib.ptr(y), _lib.ptr(w), _lib.ptr(valid),
        n, v, k, 0.1, 0.9, 1.0, _lib.ptr(dl), v, _lib.ptr(row_stats), _lib.ptr(metrics), _lib.ptr(ws),
        ws.numel(), stream)


def _eager(lib, inp):
    n, v = inp[0].shape
    out = _outputs(n, v)
    _lib.check(_call(lib, inp, out, _lib.stream(torch.device(DEV))), "ns_ce_kl_logits_fwd")
    torch.cuda.synchronize()
    return out[:3]


def test_group_path_under_graph_capture(gpu_lib):
    """ns_ce_kl_logits_fwd on bf16 rows (the group kernel) captured with torch.cuda.graph and
    replayed three times, with eager NaN fills of the outputs and synchronisations between the
    replays: every replay equals the eager call, bit for bit."""
    lib = gpu_lib
    n, v = 96, 40000
    inp = _inputs(n, v, 71)
    want = _eager(lib, inp)
    out = _outputs(n, v)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    status = []
    with torch.cuda.graph(graph):
        status.append(_call(lib, inp, out, _lib.stream(torch.device(DEV))))
    _lib.check(status[0], "ns_ce_kl_logits_fwd (captured)")
    for rep in range(3):
        for t in out[:3]:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for g, w_ in zip(out[:3], want):
            assert torch.equal(g, w_), rep


def test_group_path_on_two_streams(gpu_lib):
    """Two calls with their own inputs and workspaces, enqueued on two streams without a
    synchronisation between them, three times over: each equals its eager result, bit for bit.
    The group kernels' workgroups share the GPU; each call's tickets come from its own
    workspace."""
    lib = gpu_lib
    shapes = [(128, 248_320), (64, 40000)]
    inps = [_inputs(n, v, 90 + i) for i, (n, v) in enumerate(shapes)]
    wants = [_eager(lib, inp) for inp in inps]
    outs = [_outputs(n, v) for n, v in shapes]
    streams = [torch.cuda.Stream(device=DEV), torch.cuda.Stream(device=DEV)]
    for rep in range(3):
        for out in outs:
            for t in out[:3]:
                t.fill_(float("nan"))
        torch.cuda.synchronize()
        for inp, out, s in zip(inps, outs, streams):
            _lib.check(_call(lib, inp, out, ctypes.c_void_p(s.cuda_stream)), "ns_ce_kl_logits_fwd")
        torch.cuda.synchronize()
        for out, want in zip(outs, wants):
            for g, w_ in zip(out[:3], want):
                assert torch.equal(g, w_), rep


def test_group_wait_runs_out_to_nan_and_the_next_call_is_exact(gpu_lib, monkeypatch):
    """The exchange's bounded wait, forced from the host: member 1 of every row publishes nothing
    (NS_DEBUG_GROUP_DROP_MEMBER=1) and each poll loop gives up after 64 polls
    (NS_DEBUG_GROUP_SPIN_LIMIT=64).  The call returns; the members that waited take NaN
    statistics, so dl holds NaN and accept_len_sum is NaN.  The next call without the settings
    (its counters and words cleared again) equals the eager result bit for bit."""
    lib = gpu_lib
    n, v = 64, 40000
    inp = _inputs(n, v, 17)
    want = _eager(lib, inp)
    monkeypatch.setenv("NS_DEBUG_GROUP_DROP_MEMBER", "1")
    monkeypatch.setenv("NS_DEBUG_GROUP_SPIN_LIMIT", "64")
    metrics, row_stats, dl = _eager(lib, inp)
    assert torch.isnan(metrics[4]).item()            # accept_len_sum
    assert torch.isnan(row_stats[:, 4]).all().item()  # every row's accept rate
    assert torch.isnan(dl.float()).any().item()
    monkeypatch.delenv("NS_DEBUG_GROUP_DROP_MEMBER")
    monkeypatch.delenv("NS_DEBUG_GROUP_SPIN_LIMIT")
    again = _eager(lib, inp)
    for g, w_ in zip(again, want):
        assert torch.equal(g, w_)
