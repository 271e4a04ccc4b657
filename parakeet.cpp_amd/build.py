"""Build recipe for the native libraries (gfx950 only, built in-tree).

  libparakeet_hip.so      HIP kernels + C ABI      (csrc/pk_decode.hip)
  libparakeet_decoder.so  C++ decoder API           (csrc/parakeet_decoder.cpp, csrc/gguf_reader.cpp)
  libpk_calib.so          copy kernel of known size (csrc/pk_calib.hip), used by bench.py to scale
                          hardware byte counters
  tests/cpp/decoder_api_main  test driver of the C++ API (tests/cpp/decoder_api_main.cpp)
  tests/cpp/dropin_main   test driver of the drop-in decoder headers (tests/cpp/dropin_main.cpp), built
                          only where parakeet.cpp's sources are present: it compiles against the
                          reference's own src/parakeet_ctc.h (headers only, no ggml)

  tests/cpp/oracle_asan, oracle_tsan, gguf_fuzz_asan
                          host-only sanitizer builds (g++/gcc, no device code): the oracle under
                          AddressSanitizer + UBSan and ThreadSanitizer, and the GGUF reader and
                          decoder loader under a mutation fuzzer with AddressSanitizer + UBSan

Called by __graft_entry__.build(); every call recompiles.
"""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INC = os.path.join(ROOT, "include")
REFERENCE_SRC = os.path.join(os.environ.get("PK_REFERENCE", "/root/reference"), "src")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wall", "-Wno-unused-result", f"-I{INC}"]


def _run(cmd):
    proc = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in proc.stderr.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")
    return err


def build_hip():
    out = os.path.join(HERE, "libparakeet_hip.so")
    # PK_TIMELINE=1 compiles the decode loop's per-wave checkpoint timeline (profiling builds only)
    extra = ["-DPK_TIMELINE"] if os.environ.get("PK_TIMELINE") else []
    _run([HIPCC, *HIP_FLAGS, *extra, "-shared", os.path.join(CSRC, "pk_decode.hip"), "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def build_calib():
    out = os.path.join(HERE, "libpk_calib.so")
    _run([HIPCC, *HIP_FLAGS, "-shared", os.path.join(CSRC, "pk_calib.hip"), "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def build_decoder():
    srcs = [os.path.join(CSRC, f) for f in ("parakeet_decoder.cpp", "decoder_core.cpp", "gguf_reader.cpp")]
    if not all(os.path.exists(s) for s in srcs):
        return None
    out = os.path.join(HERE, "libparakeet_decoder.so")
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", f"-I{INC}", f"-I{CSRC}", *srcs,
          f"-L{HERE}", "-lparakeet_hip", "-Wl,-rpath,$ORIGIN", "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def build_api_test(name="decoder_api_main", hip=False):
    """tests/cpp/<name>: drivers of the C++ API for the tests (not part of the library).
    hip: the driver calls the HIP runtime itself (device-resident frames), so hipcc builds it."""
    src = os.path.join(ROOT, "tests", "cpp", name + ".cpp")
    if not os.path.exists(src) or not os.path.exists(os.path.join(HERE, "libparakeet_decoder.so")):
        return None
    out = os.path.join(ROOT, "tests", "cpp", name)
    cc = [HIPCC, *HIP_FLAGS] if hip else ["g++", "-O2", "-std=c++17", "-Wall", f"-I{INC}"]
    _run([*cc, src, f"-L{HERE}", "-lparakeet_decoder", "-lparakeet_hip",
          "-Wl,-rpath,$ORIGIN/../../parakeet.cpp_amd", "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def build_dropin_test():
    """tests/cpp/dropin_main: include/dropin/ + csrc/dropin/parakeet_dropin.cpp compiled against
    parakeet.cpp's src/parakeet_ctc.h, the drop-in headers first on the include path (as in
    parakeet.cpp's build, where they replace src/parakeet_tdt.h and src/parakeet_eou.h)."""
    if not os.path.exists(os.path.join(REFERENCE_SRC, "parakeet_ctc.h")):
        return None
    src = os.path.join(ROOT, "tests", "cpp", "dropin_main.cpp")
    out = os.path.join(ROOT, "tests", "cpp", "dropin_main")
    srcs = [src, os.path.join(CSRC, "dropin", "parakeet_dropin.cpp"), os.path.join(CSRC, "decoder_core.cpp"),
            os.path.join(CSRC, "gguf_reader.cpp")]
    _run(["g++", "-O2", "-std=c++17", "-Wall", f"-I{os.path.join(INC, 'dropin')}", f"-I{INC}", f"-I{CSRC}",
          f"-I{os.path.join(CSRC, 'dropin')}", f"-I{REFERENCE_SRC}", *srcs, f"-L{HERE}", "-lparakeet_hip",
          "-Wl,-rpath,$ORIGIN/../../parakeet.cpp_amd", "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


SAN_FLAGS = ["-O1", "-g", "-fno-omit-frame-pointer", "-fno-sanitize-recover=all"]


def build_sanitizers():
    """Host code only, compiled by gcc / g++ (never hipcc): the oracle and its driver, and the
    GGUF reader + decoder loader with the fuzz driver."""
    oracle = os.path.join(ROOT, "oracle")
    cpp = os.path.join(ROOT, "tests", "cpp")
    outs = []
    o_src = [os.path.join(cpp, "oracle_sanitize_main.c"), os.path.join(oracle, "pk_oracle.c")]
    for name, san in (("oracle_asan", "-fsanitize=address,undefined"), ("oracle_tsan", "-fsanitize=thread")):
        out = os.path.join(cpp, name)
        _run(["gcc", "-std=c11", *SAN_FLAGS, san, f"-I{oracle}", *o_src, "-lm", "-lpthread", "-o", out + ".tmp"])
        os.replace(out + ".tmp", out)
        outs.append(out)
    if os.path.exists(os.path.join(HERE, "libparakeet_hip.so")):
        out = os.path.join(cpp, "gguf_fuzz_asan")
        srcs = [os.path.join(cpp, "gguf_fuzz_main.cpp")] + [os.path.join(CSRC, f) for f in
                                                           ("gguf_reader.cpp", "parakeet_decoder.cpp", "decoder_core.cpp")]
        _run(["g++", "-std=c++17", *SAN_FLAGS, "-fsanitize=address,undefined", f"-I{INC}", f"-I{CSRC}", *srcs,
              f"-L{HERE}", "-lparakeet_hip", "-Wl,-rpath,$ORIGIN/../../parakeet.cpp_amd", "-o", out + ".tmp"])
        os.replace(out + ".tmp", out)
        outs.append(out)
    return outs


def build_all():
    return [build_hip(), build_decoder(), build_calib(), build_api_test("decoder_api_main", hip=True),
            build_api_test("loader_main"), build_dropin_test(), *build_sanitizers()]


if __name__ == "__main__":
    print(build_all())
