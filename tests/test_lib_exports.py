"""The kernel library loads without a GPU and exports every entry point the public header
declares; the ctypes binding covers exactly that list; bad arguments are rejected before any
launch."""
import os
import re
import subprocess

from openattention_amd import _build, lib

HDR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                   "openattention_amd.h")


def declared():
    text = open(HDR).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(oa_[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_exported():
    path = _build.lib_path()
    assert os.path.exists(path), "run __graft_entry__.build() first"
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (oa_[a-z0-9_]+)", out))
    names = declared()
    assert names, "no declarations parsed"
    missing = [n for n in names if n not in exported]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_matches_header():
    assert sorted(lib.SIGNATURES) == declared()


def test_library_loads_and_reports():
    L = lib.load()
    assert L.oa_abi_version() == lib.ABI_VERSION == 9
    assert b"invalid argument" in L.oa_error_string(-22)
    for name in lib.SIGNATURES:
        assert getattr(L, name) is not None


def test_argument_checks_reject_before_launch():
    """Shape checks fire on the host side of the C ABI (no device is touched)."""
    L = lib.load()
    # head_dim 64 is rejected by every entry point that takes it
    st = L.oa_flash_decode(None, 0, None, None, 0, 0, None, 0, 1, None, 0, 1, None, None, 0, 0, 0, 0,
                           None, 0, 0, None, 0, 0, 32, 8, 64, 0.1, 1, None, None, None, None)
    assert st == -22
    assert L.oa_waterfill(None, None, 4, 300, 10, None, None) == -22          # C > 256
    assert L.oa_topk_select(None, 0, None, 0, 4, 10, None, 5, None, 0, 0, 20, None) == -22   # k > tiles
    assert L.oa_qgs_prep(None, 0, None, None, 32, 8, 128, 16, None, None, None, None) == -22  # rank 16
    # top-q over heads: the scan's tile maxima without its tile minima (or the reverse)
    for tm, tmn in ((16, None), (None, 16)):
        assert L.oa_topq_heads(16, 64, 16, 64, 16, 4, 8, 64, 16, 8, 16, 16, 1, 16, 16, 16, 64, tm, tmn, 1, 0,
                               None) == -22
    # cluster sums over built lists: C above 256, rows not a multiple of G
    assert L.oa_cluster_sums(16, 16, 128 * 64, 128, 8, 4, 64, 300, 16, 16, 16, 16, 16, 64, 16, 16, None) == -22
    assert L.oa_cluster_sums(16, 16, 128 * 64, 128, 6, 4, 64, 8, 16, 16, 16, 16, 16, 64, 16, 16, None) == -22
    # query metric: more than 64 picked rows, rows not a multiple of G
    assert L.oa_query_metric(16, 1, 8192, 128, 8, 4, 16, 65, 16, 16, 1.0, 16, 32, 16, 16, None) == -22
    assert L.oa_query_metric(16, 1, 8192, 128, 6, 4, 16, 8, 16, 16, 1.0, 16, 32, 16, 16, None) == -22
    # eigensolver: n other than 128, k outside 1..64, a matrix stride below 128 * 128
    assert L.oa_sym_eig_top(16, 64 * 64, 1, 64, 16, 16, 16, None, None) == -22
    assert L.oa_sym_eig_top(16, 128 * 128, 1, 128, 65, 16, 16, None, None) == -22
    assert L.oa_sym_eig_top(16, 128 * 128, 1, 128, 0, 16, 16, None, None) == -22
    assert L.oa_sym_eig_top(16, 128 * 127, 1, 128, 32, 16, 16, None, None) == -22


def test_noalloc_flash_rejects_oversized_request_before_launch():
    """oa_flash_decode_noalloc refuses rows * n_split beyond its fixed device array (-28) before
    it resolves the array's address or launches anything."""
    L = lib.load()
    st = L.oa_flash_decode_noalloc(None, 0, None, None, 0, 0, None, 0, 1, None, 0, 1, None, None, 0,
                                   0, 0, 0, None, 0, 0, None, 0, 0, 1024, 256, 128, 0.1, 16, None)
    assert st == -28
    assert b"scratch" in L.oa_error_string(-28)
