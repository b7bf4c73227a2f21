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
