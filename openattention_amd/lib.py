"""ctypes binding of the gfx950 kernel library (C ABI declared in include/openattention_amd.h).

torch is imported first on purpose: the library links the HIP runtime that ships inside torch,
and loading torch first makes both share that one runtime (device pointers and streams are
then interchangeable).  There is no CPU fallback: a missing or stale library raises.
"""
from __future__ import annotations

import ctypes as ct
import os

import torch  # noqa: F401  (must precede the kernel library: one HIP runtime per process)

from openattention_amd import _build

P = ct.c_void_p
L = ct.c_long
I = ct.c_int
F = ct.c_float
Dd = ct.c_double

# name -> argtypes, in the order of include/openattention_amd.h
SIGNATURES = {
    "oa_abi_version": [],
    "oa_error_string": [I],
    "oa_flash_decode": [P, L, P, P, L, L, P, L, I, P, L, I, P, P, L, L, I, I, P, L, I, P, L,
                        I, I, I, I, F, I, P, P, P, P],
    "oa_flash_decode_noalloc": [P, L, P, P, L, L, P, L, I, P, L, I, P, P, L, L, I, I, P, L, I, P,
                                L, I, I, I, I, F, I, P],
    "oa_index_update": [P, P, L, L, I, I, I, P, I, I, P, P, P, P, I, P, I, P, L, P, L, P, P, P, P, P,
                        P, I, P, P],
    "oa_index_downdate": [P, P, L, L, I, I, I, P, L, P, P, P, P, I, P, P],
    "oa_qgs_prep": [P, L, P, P, I, I, I, I, P, P, P, P],
    "oa_index_prep": [P, P, L, L, I, I, I, P, I, I, P, P, P, P, I, P, I, P, L, P, L, P, P, P, P, P,
                      P, I, P, P, L, P, P, P],
    "oa_qgs_scan": [P, I, I, I, P, P, P, L, P, L, P, I, I, P],
    "oa_qgs_scan_heads": [P, I, I, I, P, P, P, L, P, L, P, P, I, I, P],
    "oa_topk_select": [P, L, P, L, I, I, P, L, P, I, I, I, P],
    "oa_topk_select_heads": [P, L, P, L, I, I, P, L, P, I, I, I, P, I, I, P, P, P],
    "oa_errorgate": [P, L, P, L, L, I, I, I, P, L, P, L, I, P, P, P, I, F, F, P, P, P],
    "oa_gate_fill": [P, L, P, L, L, I, I, I, P, L, P, L, I, P, P, P, I, F, F, I, P, P, P, P, P],
    "oa_topk_gate_fill": [P, L, P, L, I, P, I, I, I, P, I, P, P, P, L, P, L, L, I, I, I, P, L, P, L,
                          P, P, P, I, F, F, I, P, P, P, P, P],
    "oa_qgs_scan_gate": [P, I, I, I, P, P, P, L, P, L, P, P, I, I, P, L, P, P, P, I, F, F, P, P, P, P],
    "oa_topk_fix_fill": [P, L, P, L, I, P, I, I, I, P, I, P, P, P, L, P, L, L, I, I, I, P, L, P, L,
                         P, P, P, I, F, F, I, P, P, P, P],
    "oa_waterfill": [P, P, I, I, I, P, P],
    "oa_topq": [P, L, P, L, P, I, I, I, P, I, P, P],
    "oa_topq_path": [P, L, P, L, P, I, I, I, P, I, P, I, P],
    "oa_topq_heads": [P, L, P, L, P, I, I, I, P, I, P, P, I, P, P, P, L, P, P, L, I, P],
    "oa_residual": [P, P, L, L, I, I, I, P, L, P, L, I, P, I, P, P, P, P, I, P, P, P, P],
    "oa_residual_flash": [P, L, P, P, L, L, I, I, I, P, L, P, L, I, P, I, P, P, P, P, I, F, P, L,
                          I, P, P],
    "oa_dense_decode": [P, L, P, P, L, L, I, I, I, I, P, F, I, P, P, P, P, L, P],
    "oa_qgs_codes": [P, L, L, I, I, P, P, L, P, P, P, P],
    "oa_qgc_project": [P, L, L, I, I, I, P, P, L, P, P, P, P],
    "oa_kmeans_assign": [P, P, L, I, I, P, I, P, L, P, L, P],
    "oa_kmeans_update": [P, P, L, I, I, P, L, I, P, P, P, P, L, P, P, P],
    "oa_cluster_build": [P, P, L, L, I, I, I, P, L, I, P, P, P, P, P, L, P, P, P],
    "oa_cluster_sums": [P, P, L, L, I, I, I, I, P, P, P, P, P, L, P, P, P],
    "oa_query_metric": [P, I, L, L, I, I, P, I, P, P, Dd, P, I, P, P, P],
    "oa_sym_eig_top": [P, L, I, I, I, P, P, P, P],
}

# must equal oa_abi_version() of the loaded library (OA_ABI_VERSION in the header): a library
# built from sources with other argument lists would be handed wrong pointers
ABI_VERSION = 9

_LIB = None


def load() -> ct.CDLL:
    """Load the kernel library; raises if it has not been built (run __graft_entry__.build()) or
    was built for another ABI version."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = _build.lib_path()
    if not os.path.exists(path):
        raise RuntimeError(f"kernel library not built: {path} (run __graft_entry__.build())")
    lib = ct.CDLL(path)
    lib.oa_abi_version.restype = ct.c_int
    have = lib.oa_abi_version()
    if have != ABI_VERSION:
        raise RuntimeError(f"kernel library {path} has ABI {have}, this binding expects {ABI_VERSION}: "
                           "rebuild it (__graft_entry__.build())")
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ct.c_char_p if name == "oa_error_string" else ct.c_int
    _LIB = lib
    return lib


def call(name: str, *args) -> None:
    """Call one C entry point; a nonzero status raises RuntimeError with the HIP error text."""
    lib = load()
    st = getattr(lib, name)(*args)
    if st != 0:
        msg = lib.oa_error_string(st).decode()
        sizes = [a for a in args if isinstance(a, (int, float)) and not isinstance(a, bool)]
        raise RuntimeError(f"{name} failed with status {st}: {msg} (numeric arguments {sizes})")
