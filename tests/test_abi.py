"""The C ABI surface: the library loads, exports every header symbol and
rejects bad arguments before any device work (no GPU needed)."""

import ctypes

import pytest

from nanospec_amd import _lib


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_exports_every_header_symbol(lib):
    names = _lib.header_symbols()
    assert "ns_ce_kl_logits_fwd" in names and "ns_last_error" in names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(_lib.SIGNATURES), "ctypes signature table out of sync with the header"


def test_abi_version(lib):
    assert lib.ns_abi_version() == _lib.ABI_VERSION


def test_workspace_query(lib):
    small = lib.ns_workspace_bytes(_lib.NS_WS_LOGITS, 64, 8192, 0)
    big = lib.ns_workspace_bytes(_lib.NS_WS_LOGITS, 4096, 248320, 0)
    assert 0 < small < big
    assert big % 256 == 0


def _fwd(lib, **over):
    args = dict(z=1, zdt=0, ldz=16, u=1, udt=0, ldu=16, labels=1, weights=1, valid=1, n=8, v=16, k=8,
                c_ce=0.1, c_kl=0.9, inv_acc=1.0, dl=None, ldd=16, row_stats=1, metrics=1, ws=256,
                wsb=1 << 20, stream=None)
    args.update(over)
    p = lambda x: None if x is None else ctypes.c_void_p(x)
    return lib.ns_ce_kl_logits_fwd(
        p(args["z"]), args["zdt"], args["ldz"], p(args["u"]), args["udt"], args["ldu"], p(args["labels"]),
        p(args["weights"]), p(args["valid"]), args["n"], args["v"], args["k"], args["c_ce"], args["c_kl"],
        args["inv_acc"], p(args["dl"]), args["ldd"], p(args["row_stats"]), p(args["metrics"]), p(args["ws"]),
        args["wsb"], p(args["stream"]))


@pytest.mark.parametrize("over,code,text", [
    (dict(zdt=7), -2, "dtype"),
    (dict(n=12), -1, "multiple of the block size"),
    (dict(k=0), -1, "block size"),
    (dict(ldz=8), -1, "leading dimension"),
    (dict(ldu=(1 << 23) + 1), -1, "exceeds"),     # tiles use 32-bit byte offsets
    (dict(z=None), -5, "z is NULL"),
    (dict(labels=None), -5, "non-NULL"),
    (dict(wsb=16), -4, "workspace"),
    (dict(v=0), -1, "vocabulary"),
])
def test_argument_validation(lib, over, code, text):
    assert _fwd(lib, **over) == code
    assert text in lib.ns_last_error().decode()


def test_status_mapping(lib):
    _fwd(lib, zdt=9)
    with pytest.raises(ValueError, match="dtype"):
        _lib.check(-2, "ns_ce_kl_logits_fwd")


def _norm_args(**over):
    a = dict(x=256, ldx=64, inv=256, weight=256, dx=512, lddx=64, weight_grad=768)
    a.update(over)
    return _lib.RmsNormBwd(a["x"], a["ldx"], a["inv"], a["weight"], a["dx"], a["lddx"], a["weight_grad"])


@pytest.mark.parametrize("over,d,code,text", [
    (dict(), 60, -1, "multiple of 8"),
    (dict(), 16392, -1, "up to 16384"),
    (dict(ldx=32), 64, -1, "leading dimension"),
    (dict(inv=None), 64, -5, "non-NULL"),
    (dict(dx=520), 64, -3, "aligned"),
    (dict(), 64, -4, "workspace"),
])
def test_rms_norm_bwd_validation(lib, over, d, code, text):
    args = _norm_args(**over)
    rc = lib.ns_rms_norm_bwd(ctypes.c_void_p(256), d, ctypes.byref(args), 4, d, None, 0, None)
    assert rc == code
    assert text in lib.ns_last_error().decode()


def test_markov_and_pooled_validation(lib):
    p = ctypes.c_void_p
    # rank not a multiple of 64
    rc = lib.ns_lmhead_markov_bwd(p(256), 64, p(256), 64, p(256), p(256), 64, p(256), 64, 32, p(256), 64, None,
                                  p(256), 64, p(256), 64, 8, 64, 64, p(256), 1 << 20, None)
    assert rc == -1 and "Markov rank" in lib.ns_last_error().decode()
    # dh may be NULL only with a norm
    rc = lib.ns_lmhead_markov_bwd(p(256), 64, p(256), 64, p(256), p(256), 64, p(256), 64, 64, None, 64, None,
                                  p(256), 64, p(256), 64, 8, 64, 64, p(256), 1 << 20, None)
    assert rc == -5 and "dh is NULL" in lib.ns_last_error().decode()
    assert lib.ns_pooled_tail(p(256), 0, 1, 1, p(256), None) == -1
    assert lib.ns_pooled_tail(p(256), 1, 0, 1, p(256), None) == -1
    assert lib.ns_scale_gradient(p(256), 5, 8, p(256), None) == -2
    assert lib.ns_scale_gradient(p(260), 0, 8, p(256), None) == -3
    assert lib.ns_lmhead_markov_bwd_workspace_bytes(4096, 248320, 5120, 256) > \
        lib.ns_workspace_bytes(_lib.NS_WS_LMHEAD_BWD, 4096, 248320, 5120)
    assert lib.ns_workspace_bytes(_lib.NS_WS_LMHEAD_NORM_BWD, 4096, 248320, 5120) > \
        lib.ns_workspace_bytes(_lib.NS_WS_LMHEAD_BWD, 4096, 248320, 5120)


def _head_bwd(lib, **over):
    """ns_lmhead_ce_kl_bwd with fake (never dereferenced) pointers: n=8, d=64, V=64."""
    a = dict(hidden=256, ldh=64, weight=256, ldw=64, markov=None, ldm=64, prev=None, w1=None, ldw1=0, w2=None,
             ldw2=0, r=0, teacher=256, tdt=0, ldt=64, labels=256, weights=256, n=8, d=64, v=64, inv_acc=0.5,
             row_stats=256, dl=512, ldd=64, ws=256, wsb=1 << 24)
    a.update(over)
    p = lambda x: None if x is None else ctypes.c_void_p(x)
    return lib.ns_lmhead_ce_kl_bwd(
        p(a["hidden"]), a["ldh"], p(a["weight"]), a["ldw"], p(a["markov"]), a["ldm"], p(a["prev"]), p(a["w1"]),
        a["ldw1"], p(a["w2"]), a["ldw2"], a["r"], p(a["teacher"]), a["tdt"], a["ldt"], None, p(a["labels"]),
        p(a["weights"]), a["n"], a["d"], a["v"], 0.1, 0.9, a["inv_acc"], p(a["row_stats"]), p(a["dl"]), a["ldd"],
        p(a["ws"]), a["wsb"], None)


@pytest.mark.parametrize("over,code,text", [
    (dict(dl=None), -5, "dl is NULL"),                       # the re-emission has no other output
    (dict(row_stats=None), -5, "row_stats"),                 # it is the input here
    (dict(markov=256, r=64, prev=256, w1=256, ldw1=64, w2=256, ldw2=64), -1, "not both"),
    (dict(r=32, prev=256, w1=256, ldw1=64, w2=256, ldw2=64), -1, "Markov rank"),
    (dict(r=-64), -1, "Markov rank"),
    (dict(d=96), -1, "hidden size"),
    (dict(tdt=3), -2, "teacher dtype"),
    (dict(ldd=60), -1, "leading dimension"),
    (dict(dl=520), -3, "aligned"),
    (dict(wsb=16), -4, "workspace"),
    (dict(labels=None), -5, "non-NULL"),
])
def test_lmhead_ce_kl_bwd_validation(lib, over, code, text):
    assert _head_bwd(lib, **over) == code
    assert text in lib.ns_last_error().decode()


def test_lmhead_ce_kl_bwd_empty(lib):
    # no rows: nothing to emit, and no pointer is needed
    assert _head_bwd(lib, n=0, hidden=None, dl=None, row_stats=None, labels=None, weights=None, ws=None,
                     wsb=0) == 0


@pytest.mark.parametrize("kind", range(7))
@pytest.mark.parametrize("n,v,d", [(0, 248320, 5120), (0, 0, 0), (8, 0, 64), (8, 64, 0)])
def test_workspace_query_degenerate_shapes(lib, kind, n, v, d):
    # empty batches and zero-sized dimensions size to a finite workspace (the plans
    # divide by the number of row and column tiles, which is 0 here)
    assert lib.ns_workspace_bytes(kind, n, v, d) < 1 << 40
    assert lib.ns_lmhead_markov_bwd_workspace_bytes(n, v, d, 64) < 1 << 40


def test_forward_parts_and_row_copy_validation(lib):
    """The skip-masked-rows path's entry points reject bad arguments before device work."""
    p = ctypes.c_void_p

    def part(which, **over):
        a = dict(hidden=256, teacher=256, labels=256, weights=256, n=8, d=64, v=64, dl=512, row_stats=256,
                 ws=256, wsb=1 << 24)
        a.update(over)
        q = lambda x: None if x is None else p(x)
        return lib.ns_lmhead_ce_kl_fwd_part(which, q(a["hidden"]), 64, p(256), 64, None, 64, q(a["teacher"]), 0, 64,
                                            None, q(a["labels"]), q(a["weights"]), a["n"], a["d"], a["v"], 0.1, 0.9,
                                            1.0, q(a["dl"]), 64, q(a["row_stats"]), q(a["ws"]), a["wsb"], None)

    assert part(3) == -1 and "NS_PART" in lib.ns_last_error().decode()
    assert part(_lib.NS_PART_EMIT, row_stats=None) == -5 and "row_stats" in lib.ns_last_error().decode()
    assert part(_lib.NS_PART_STATS, d=96) == -1 and "hidden size" in lib.ns_last_error().decode()
    assert part(_lib.NS_PART_EMIT, wsb=16) == -4
    assert part(_lib.NS_PART_STATS, n=0, hidden=None, teacher=None, labels=None, weights=None, dl=None,
                row_stats=None, ws=None, wsb=0) == 0
    assert lib.ns_objective_metrics(p(256), p(256), p(256), 12, 8, 0.1, 0.9, p(256), None) == -1
    assert lib.ns_objective_metrics(p(256), None, p(256), 8, 8, 0.1, 0.9, p(256), None) == -5
    assert lib.ns_copy_rows(p(256), 64, 4, p(256), 4, 62, p(512), 64, None) == -1   # row_bytes % 4
    assert lib.ns_copy_rows(p(256), 32, 4, p(256), 4, 64, p(512), 64, None) == -1   # pitch below the row
    assert lib.ns_copy_rows(p(256), 64, 4, None, 4, 64, p(512), 64, None) == -5
    assert lib.ns_copy_rows(p(258), 64, 4, p(256), 4, 64, p(512), 64, None) == -3
    assert lib.ns_copy_rows(None, 64, 0, None, 0, 64, None, 64, None) == 0            # nothing to copy
