"""The reference-shaped C++ API (include/parakeet_decoder.h) driven the way
parakeet.cpp's callers drive it (tests/cpp/decoder_api_main.cpp), checked
against the C ABI path that the parity tests pin against the oracle.

- tdt_greedy_decode (src/parakeet_tdt.cpp:983-1005) and tdt_decode_batch give
  the C ABI's tokens; tdt_decode_window over 5-frame windows (longer than any
  duration, so no carry is dropped) gives the one-shot tokens
  (test/test_tdt_decoder_parity.cpp pins CPU == graph tokens the same way);
- a D_enc mismatch returns 1 (src/parakeet_tdt.cpp:877);
- result.text is detokenize(tokens) by src/sentencepiece_bpe.cpp:9-38;
- eou_greedy_decode / eou_decode_window give the C ABI's tokens and segment
  boundaries (test/test_eou_streaming.cpp:164-187);
- Engine::transcribe_features gives tdt_greedy_decode's result."""
import json
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT, small_eou, small_tdt

DRIVER = os.path.join(ROOT, "tests", "cpp", "decoder_api_main")


def _frames_file(path, encs):
    n, T, D = len(encs), encs[0].shape[0], encs[0].shape[1]
    with open(path, "wb") as f:
        np.array([n, T, D], np.int32).tofile(f)
        np.stack(encs).astype(np.float32).tofile(f)


def _detok(pieces, ids, skip):
    """src/sentencepiece_bpe.cpp:9-38: skipped ids, U+2581 -> ' ', leading spaces trimmed."""
    s = "".join(pieces[i] for i in ids if 0 <= i < len(pieces) and i not in skip).replace("▁", " ")
    return s.lstrip(" ")


def test_cpp_api_driver_built():
    """The driver links against both libraries; without arguments it prints
    its usage and exits 2 before any device call."""
    assert os.path.exists(DRIVER), "run __graft_entry__.build()"
    r = subprocess.run([DRIVER], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "usage" in r.stderr


@pytest.mark.gpu
def test_cpp_api_matches_c_abi(tmp_path):
    from parakeet_amd import pk, synth
    tdt_path, eou_path = str(tmp_path / "t.gguf"), str(tmp_path / "e.gguf")
    small_tdt(tdt_path)
    small_eou(eou_path)
    T, W = 40, 5
    encs_t = [synth.encoder_frames(700 + u, T, 128) for u in range(3)]
    encs_e = [synth.encoder_frames(800 + u, T, 64) for u in range(3)]
    _frames_file(tmp_path / "t.bin", encs_t)
    _frames_file(tmp_path / "e.bin", encs_e)
    print(f"cpp api: driver TDT/EOU B=3 T={T} window={W}", flush=True)
    r = subprocess.run([DRIVER, tdt_path, str(tmp_path / "t.bin"), eou_path, str(tmp_path / "e.bin"), str(W)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout)

    dt = pk.Decoder.from_gguf(tdt_path, n_slots=4)
    ref_t = dt.decode(encs_t)
    pieces_t = dt.info.pieces
    blank_t = dt.info.blank
    for u in range(3):
        want = ref_t[u]["tokens"].tolist()
        assert out["tdt"]["greedy"][u] == want, u
        assert out["tdt"]["batch"][u] == want, u
        assert out["tdt"]["chunked"][u] == want, u
        assert out["tdt"]["steps"][u] == ref_t[u]["steps"], u
        assert out["tdt"]["text"][u] == _detok(pieces_t, want, {blank_t}), u
    assert out["tdt"]["bad_dim_rc"] == 1
    assert out["engine"]["tokens"] == ref_t[0]["tokens"].tolist()
    assert out["engine"]["steps"] == ref_t[0]["steps"]
    dt.close()

    de = pk.Decoder.from_gguf(eou_path, n_slots=4)
    ref_e = de.decode(encs_e, max_symbols=5)
    for u in range(3):
        assert out["eou"]["greedy"][u] == ref_e[u]["tokens"].tolist(), u
        assert out["eou"]["segments"][u] == ref_e[u]["segments"].tolist(), u
        assert out["eou"]["chunked"][u] == ref_e[u]["tokens"].tolist(), u
        assert out["eou"]["chunked_segments"][u] == ref_e[u]["segments"].tolist(), u
    de.close()
    print("cpp api: tokens", [len(x) for x in out["tdt"]["greedy"]], [len(x) for x in out["eou"]["greedy"]],
          "eou segments", [len(x) for x in out["eou"]["segments"]])
