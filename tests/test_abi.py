"""The C-ABI library loads on a CPU-only host and exports every entry point
that include/parakeet_hip.h declares (no compute calls without a GPU)."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    return sorted(set(re.findall(r"PK_API\s+[\w\s\*]+?\b(pk_\w+)\s*\(", text)))


def test_hip_library_exports_header_symbols(pkg):
    from parakeet_amd import pk
    names = declared("parakeet_hip.h")
    assert len(names) >= 9
    lib = ctypes.CDLL(pk.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(pk.EXPORTED) == names
