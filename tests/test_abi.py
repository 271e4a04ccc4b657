"""The C-ABI library loads on a CPU-only host and exports every entry point
that include/parakeet_hip.h declares (no compute calls without a GPU); the
Python mirror's constants match the header; the C++ API library defines the
device-frame handoff entry points."""
import ctypes
import os
import re
import shutil
import subprocess

import pytest

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


def header_enum(header, prefix):
    """PK_<prefix>_* = value pairs of the header's enums."""
    text = open(os.path.join(ROOT, "include", header)).read()
    return {m.group(1): int(m.group(2)) for m in re.finditer(rf"\bPK_({prefix}_\w+)\s*=\s*(\d+)", text)}


def test_python_mirror_constants_match_header(pkg):
    from parakeet_amd import pk
    for prefix in ("MEM", "KIND"):
        enum = header_enum("parakeet_hip.h", prefix)
        assert enum, prefix
        for name, value in enum.items():
            assert getattr(pk, name) == value, name


def test_decoder_library_exports_device_handoff(pkg):
    """The C++ API library defines the device-frame entry points the header declares."""
    lib = os.path.join(ROOT, "parakeet.cpp_amd", "libparakeet_decoder.so")
    nm = shutil.which("nm")
    if nm is None or not os.path.exists(lib):
        pytest.skip("nm or the built library is missing")
    syms = subprocess.run([nm, "-DC", "--defined-only", lib], capture_output=True, text=True, check=True).stdout
    for name in ("parakeet_hip::tdt_decode_batch_device(", "parakeet_hip::eou_decode_batch_device(",
                 "parakeet_hip::Engine::transcribe_device_batch("):
        assert name in syms, name


def test_python_mirror_checks_per_utterance_arrays(pkg):
    """pk_decode reads n_utts entries of every per-utterance array, so the
    Python mirror repeats a scalar (offsets, token bases, reset flags) and
    refuses an array of another length before any call."""
    import numpy as np
    from parakeet_amd import pk
    assert pk._per_utt(None, 3, np.float32, "blank_bias") is None
    assert pk._per_utt(2.0, 3, np.float32, "blank_bias").tolist() == [2.0, 2.0, 2.0]
    assert pk._per_utt([1, 2], 2, np.int32, "slots", scalar=False).dtype == np.int32
    for bad, scalar in (([1.0, 2.0], True), (5, False), ([[1], [2], [3]], True)):
        with pytest.raises(ValueError):
            pk._per_utt(bad, 3, np.float32, "x", scalar=scalar)
