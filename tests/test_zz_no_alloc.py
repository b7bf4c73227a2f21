"""The allocation-free fused forward (ns_lmhead_ce_kl_fwd_noalloc) against the workspace
entry point it mirrors (ns_lmhead_ce_kl_fwd), through the C ABI: bit-identical metrics, row
statistics and dl on two calls in a row, the second smaller (the shared static scratch keeps
the first call's contents), and sizes beyond its scratch refused before any launch."""

import ctypes

import pytest
import torch

from nanospec_amd import _lib, synthetic
from nanospec_amd.objective import _slot_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _args(n, d, v, seed):
    hidden, weight, markov, teacher, slots = synthetic.head_inputs(n, d, v, seed, DEV, ragged=True)
    w, y, valid, k = _slot_inputs(slots, n, torch.device(DEV))
    return hidden, weight, markov, teacher, w, y, valid, k


def _call(lib, noalloc, hidden, weight, markov, teacher, w, y, valid, k, acc=2):
    n, d = hidden.shape
    v = weight.shape[0]
    metrics = torch.full((6,), float("nan"), device=DEV)
    row_stats = torch.full((n, 8), float("nan"), device=DEV)
    dl = torch.full((n, v), float("nan"), dtype=torch.bfloat16, device=DEV)
    head = (_lib.ptr(hidden), d, _lib.ptr(weight), d, _lib.ptr(markov), v, _lib.ptr(teacher), _lib.NS_BF16, v, None,
            _lib.ptr(y), _lib.ptr(w), _lib.ptr(valid), n, d, v, k, 0.1, 0.9, 1.0 / acc, _lib.ptr(dl), v,
            _lib.ptr(row_stats), _lib.ptr(metrics))
    stream = _lib.stream(torch.device(DEV))
    if noalloc:
        status = lib.ns_lmhead_ce_kl_fwd_noalloc(*head, stream)
        _lib.check(status, "ns_lmhead_ce_kl_fwd_noalloc")
    else:
        ws = _lib.workspace(_lib.NS_WS_LMHEAD, n, v, d, torch.device(DEV))
        status = lib.ns_lmhead_ce_kl_fwd(*head, _lib.ptr(ws), ws.numel(), stream)
        _lib.check(status, "ns_lmhead_ce_kl_fwd")
    torch.cuda.synchronize()
    return metrics, row_stats, dl


def test_noalloc_matches_the_workspace_entry_point(gpu_lib):
    lib = gpu_lib
    for n, d, v, seed in ((1024, 256, 16384, 31), (264, 192, 2056, 32)):   # the second call is smaller
        a = _args(n, d, v, seed)
        got = _call(lib, True, *a)
        want = _call(lib, False, *a)
        for g, w_ in zip(got, want):
            assert torch.equal(g, w_), (n, d, v)
        assert bool(torch.isfinite(got[0]).all())


def test_noalloc_under_graph_capture(gpu_lib):
    """ns_device_init before capture, then ns_lmhead_ce_kl_fwd_noalloc captured with
    torch.cuda.graph and replayed three times, with eager fills of the outputs and
    synchronisations between the replays: every replay equals the workspace entry point's
    result on the same inputs, bit for bit."""
    lib = gpu_lib
    assert lib.ns_device_init() == 0, lib.ns_last_error()
    n, d, v = 512, 128, 8192
    hidden, weight, markov, teacher, w, y, valid, k = _args(n, d, v, 33)
    want = _call(lib, False, hidden, weight, markov, teacher, w, y, valid, k)
    metrics = torch.empty(6, device=DEV)
    row_stats = torch.empty((n, 8), device=DEV)
    dl = torch.empty((n, v), dtype=torch.bfloat16, device=DEV)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    status = []
    with torch.cuda.graph(graph):
        status.append(lib.ns_lmhead_ce_kl_fwd_noalloc(
            _lib.ptr(hidden), d, _lib.ptr(weight), d, _lib.ptr(markov), v, _lib.ptr(teacher), _lib.NS_BF16, v, None,
            _lib.ptr(y), _lib.ptr(w), _lib.ptr(valid), n, d, v, k, 0.1, 0.9, 0.5, _lib.ptr(dl), v,
            _lib.ptr(row_stats), _lib.ptr(metrics), _lib.stream(torch.device(DEV))))
    _lib.check(status[0], "ns_lmhead_ce_kl_fwd_noalloc (captured)")
    for rep in range(3):
        for t in (metrics, row_stats, dl):
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for g, w_ in zip((metrics, row_stats, dl), want):
            assert torch.equal(g, w_), rep


def test_noalloc_refuses_sizes_beyond_its_scratch(gpu_lib):
    n, d, v = 65536, 64, 248320
    status = gpu_lib.ns_lmhead_ce_kl_fwd_noalloc(
        ctypes.c_void_p(256), d, ctypes.c_void_p(256), d, None, v, ctypes.c_void_p(256), _lib.NS_BF16, v, None,
        ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.c_void_p(256), n, d, v, 8, 0.1, 0.9, 1.0, None, v,
        ctypes.c_void_p(256), ctypes.c_void_p(256), None)
    assert status == -4   # NS_EWORKSPACE, before any device work
    assert "static scratch" in gpu_lib.ns_last_error().decode()
