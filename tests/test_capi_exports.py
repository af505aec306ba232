"""The C-ABI library loads without a GPU and exports every symbol include/*.h declares."""
import ctypes
from pathlib import Path

from torchpairwise_amd import _capi


def test_header_declares_entry_points():
    syms = _capi.header_symbols()
    for name in ("tpw_pack_bool_rows", "tpw_bool_pairwise_reduce", "tpw_jaccard_bool",
                 "tpw_pairwise_inner", "tpw_lp_distances", "tpw_directed_hausdorff"):
        assert name in syms


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_capi.LIB_PATH))
    headers = sorted(Path(_capi.HEADER).parent.glob("*.h"))
    missing = []
    for h in headers:
        for name in _capi.header_symbols(h):
            if not hasattr(lib, name):
                missing.append(f"{h.name}:{name}")
    assert not missing, f"declared but not exported: {missing}"


def test_binding_covers_header():
    assert set(_capi.header_symbols()) <= set(_capi._SIGNATURES), \
        set(_capi.header_symbols()) - set(_capi._SIGNATURES)


def test_pure_host_entry_points():
    l = _capi.lib()
    assert l.tpw_packed_words(1) == 4
    assert l.tpw_packed_words(128) == 4
    assert l.tpw_packed_words(129) == 8
    assert l.tpw_packed_words(1024) == 32
    assert l.tpw_runtime_version() > 0
    assert l.tpw_inner_backward_workspace_size(1, 10, 20, 8) >= 4 * 10 * 20
    assert l.tpw_hausdorff_workspace_size(1, 2, 10, 3, 20, 3) > 0


def test_argument_errors_are_reported_without_gpu():
    l = _capi.lib()
    # invalid sizes are rejected on the host before any launch
    rc = l.tpw_lp_distances(None, None, 1, 4, 4, 3, -1.0, None, None)
    assert rc == 1
    assert b"p must be non-negative" in l.tpw_last_error()
    rc = l.tpw_bool_pairwise_reduce(None, None, 1, 4, 4, 0, 0, 0, None, None)
    assert rc == 1
