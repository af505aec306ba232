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


def test_workspace_queries_accept_empty_sizes():
    # regression: split counts divided by the number of output tiles, 0 for an empty side;
    # run in a child so that a host fault fails this test instead of ending the session
    import subprocess
    import sys

    code = (
        "from torchpairwise_amd import _capi\n"
        "l = _capi.lib()\n"
        "for n, m, d in ((0, 37, 5), (41, 0, 5), (0, 0, 5), (5, 7, 0)):\n"
        "    for b in (0, 1):\n"
        "        [l.tpw_family_backward_workspace_size(k, b, n, m, d) for k in range(6)]\n"
        "        l.tpw_lp_backward_workspace_size(b, n, m, d)\n"
        "        l.tpw_inner_backward_workspace_size(b, n, m, d)\n"
        "        l.tpw_haversine_workspace_size(b, n, m)\n"
        "        l.tpw_hausdorff_workspace_size(b, 2, n, 3, m, d)\n"
        "print('ok')\n")
    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, "-c", code], cwd=root, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "ok", (r.returncode, r.stderr[-2000:])
