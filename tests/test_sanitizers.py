"""Host code under the sanitizers (CPU only, no device call).

- The oracle (oracle/pk_oracle.c) built with AddressSanitizer + UBSan and with
  ThreadSanitizer, driven by tests/cpp/oracle_sanitize_main.c over every
  function: dequantisation of each block type, TDT and EOU windows of 0..40
  frames with state carried, the replay of each window's own trace (which must
  be exact), bounded-output overflow (rc 11), and the threaded batch driver
  against one-at-a-time windows.
- The GGUF reader and the decoder loader (csrc/gguf_reader.cpp,
  csrc/parakeet_decoder.cpp, csrc/decoder_core.cpp) built with AddressSanitizer
  + UBSan under a mutation fuzzer (tests/cpp/gguf_fuzz_main.cpp): truncations,
  byte flips, extreme values in header fields, inserted / removed bytes, on
  TDT and EOU seeds with q8_0 / q4_0 / f16 matrices.  A corrupt file must be
  rejected or accepted with every tensor inside the buffer, never crash.

The binaries are built by __graft_entry__.build() with gcc / g++ only."""
import json
import os
import subprocess

import pytest

from conftest import ROOT, small_eou, small_tdt

CPP = os.path.join(ROOT, "tests", "cpp")
SAN_ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", TSAN_OPTIONS="halt_on_error=1")


def _run(args, timeout=300):
    exe = args[0]
    assert os.path.exists(exe), f"{exe} missing: run __graft_entry__.build()"
    r = subprocess.run(args, capture_output=True, text=True, errors="replace", timeout=timeout, env=SAN_ENV)
    for marker in ("ERROR: AddressSanitizer", "ERROR: LeakSanitizer", "runtime error:", "WARNING: ThreadSanitizer"):
        assert marker not in r.stderr, r.stderr[-4000:]
    assert r.returncode == 0, (r.returncode, r.stderr[-4000:])
    return r.stdout


@pytest.mark.parametrize("name", ["oracle_asan", "oracle_tsan"])
def test_oracle_under_sanitizer(name):
    assert _run([os.path.join(CPP, name)]).strip() == "ok"


@pytest.mark.parametrize("model,quant", [("tdt", "q8_0"), ("tdt", "q4_0"), ("eou", "q5_0"), ("tdt", "f16")])
def test_gguf_reader_fuzz(tmp_path, model, quant):
    seed = str(tmp_path / "seed.gguf")
    (small_tdt if model == "tdt" else small_eou)(seed, quant=quant)
    for rng_seed in (1, 2):
        out = json.loads(_run([os.path.join(CPP, "gguf_fuzz_asan"), seed, "10000", str(rng_seed),
                               str(tmp_path / "scratch.gguf")]).strip().splitlines()[-1])
        assert out["iterations"] == 10000
        # both outcomes occur: the mutations reach past the header checks
        assert out["accepted"] > 500 and out["rejected"] > 500, out
        assert out["loaded"] > 0 and out["load_rejected"] > 0, out
