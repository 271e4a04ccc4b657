"""The drop-in decoder headers (include/dropin/parakeet_tdt.h, parakeet_eou.h)
in place of parakeet.cpp's src/parakeet_tdt.h and src/parakeet_eou.h.

CPU (skipped where parakeet.cpp's sources are absent, e.g. on a GPU host):
- parakeet.cpp's own translation units that call the decoder -- the Engine
  (src/parakeet_engine.cpp) and the decoder tests (test/test_tdt_decoder_parity.cpp,
  test/test_eou_streaming.cpp, test/test_decoder_determinism.cpp) -- compile
  unchanged with the drop-in headers shadowing the reference's two decoder
  headers, and so does the drop-in implementation against the reference's
  src/parakeet_ctc.h (its ParakeetCtcModel, TdtWeights, EouWeights, BpeVocab).

GPU: tests/cpp/dropin_main drives the drop-in through a reference
ParakeetCtcModel (built where the reference is present; the built driver needs
nothing of it at run time) and must give the C ABI's tokens, steps, text and
EOU boundaries, which the parity tests pin against the oracle; a copied state
continues the utterance exactly as the original, whichever runs first."""
import json
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT, small_eou, small_tdt
from parity import check_window

REF = os.environ.get("PK_REFERENCE", "/root/reference")
REF_SRC = os.path.join(REF, "src")
DROPIN = os.path.join(ROOT, "include", "dropin")
DRIVER = os.path.join(ROOT, "tests", "cpp", "dropin_main")
need_ref = pytest.mark.skipif(not os.path.exists(os.path.join(REF_SRC, "parakeet_ctc.h")),
                              reason="parakeet.cpp's sources are not present on this host")


def _shadow_tree(tmp_path):
    """The reference's src/ as symlinks, with parakeet_tdt.h / parakeet_eou.h
    pointing at the drop-in headers: quoted includes of reference files resolve
    their own directory first, so the headers are replaced there."""
    d = tmp_path / "src"
    d.mkdir()
    for name in os.listdir(REF_SRC):
        target = os.path.join(DROPIN, name) if name in ("parakeet_tdt.h", "parakeet_eou.h") else \
            os.path.join(REF_SRC, name)
        os.symlink(target, d / name)
    return str(d)


def _syntax(src, incs):
    cmd = ["g++", "-std=c++17", "-fsyntax-only", "-Wall", *[f"-I{i}" for i in incs], src]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, f"{' '.join(cmd)}\n{r.stderr[-4000:]}"


@need_ref
@pytest.mark.parametrize("unit", ["src/parakeet_engine.cpp", "test/test_tdt_decoder_parity.cpp",
                                  "test/test_eou_streaming.cpp", "test/test_decoder_determinism.cpp"])
def test_reference_callers_compile_against_dropin(tmp_path, unit):
    src_dir = _shadow_tree(tmp_path)
    path = os.path.join(REF, unit)
    if unit.startswith("src/"):
        path = os.path.join(src_dir, os.path.basename(unit))   # its own directory is the shadowed one
    _syntax(path, [src_dir, os.path.join(REF, "include"), os.path.join(ROOT, "include")])


@need_ref
def test_dropin_implementation_compiles_against_reference_model():
    csrc = os.path.join(ROOT, "parakeet.cpp_amd", "csrc")
    _syntax(os.path.join(csrc, "dropin", "parakeet_dropin.cpp"),
            [DROPIN, os.path.join(ROOT, "include"), csrc, os.path.join(csrc, "dropin"), REF_SRC])


def test_dropin_header_declarations_match_reference():
    """Every decoder function the reference declares is declared by the drop-in
    with the same parameter list (whitespace aside)."""
    import re

    def decls(text):
        text = re.sub(r"//[^\n]*", "", text)
        out = {}
        for m in re.finditer(r"\b(int|void)\s+((?:tdt|eou)_\w+)\s*\(([^;{]*)\)\s*;", text):
            out[m.group(2)] = re.sub(r"\s+", "", m.group(3))
        return out

    for h in ("parakeet_tdt.h", "parakeet_eou.h"):
        ref_h = os.path.join(REF_SRC, h)
        if not os.path.exists(ref_h):
            pytest.skip("parakeet.cpp's sources are not present on this host")
        ours = decls(open(os.path.join(DROPIN, h)).read())
        theirs = decls(open(ref_h).read())
        assert theirs, h
        for name, params in theirs.items():
            if name.endswith("_cpu") or name.endswith("_gpu"):
                continue
            assert name in ours, (h, name)
            # the drop-in runtime is the device decoder: W is taken the same way
            assert ours[name] == params, (h, name, ours[name], params)


def _frames_file(path, encs):
    n, T, D = len(encs), encs[0].shape[0], encs[0].shape[1]
    with open(path, "wb") as f:
        np.array([n, T, D], np.int32).tofile(f)
        np.stack(encs).astype(np.float32).tofile(f)


def _detok(pieces, ids, skip):
    """src/sentencepiece_bpe.cpp:9-38: skipped ids, U+2581 -> ' ', leading spaces trimmed."""
    s = "".join(pieces[i] for i in ids if 0 <= i < len(pieces) and i not in skip).replace("▁", " ")
    return s.lstrip(" ")


def test_dropin_driver_usage():
    if not os.path.exists(DRIVER):
        pytest.skip("the drop-in driver is built only where parakeet.cpp's sources are present")
    r = subprocess.run([DRIVER], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "usage" in r.stderr


@pytest.mark.gpu
def test_dropin_matches_c_abi(tmp_path):
    if not os.path.exists(DRIVER):
        pytest.skip("the drop-in driver is built only where parakeet.cpp's sources are present")
    import oracle
    from parakeet_amd import gguf as G, pk, synth
    tdt_path, eou_path = str(tmp_path / "t.gguf"), str(tmp_path / "e.gguf")
    small_tdt(tdt_path)
    w = small_eou(eou_path)
    bias = w["eou.joint.out.bias"].copy()
    bias[33] += 1.5   # <EOU> (id 33) raised so that segments end now and then
    small_eou(eou_path, overrides={"eou.joint.out.bias": bias})
    T, W = 40, 5
    encs_t = [synth.encoder_frames(900 + u, T, 128) for u in range(3)]
    encs_e = [synth.encoder_frames(950 + u, T, 64) for u in range(3)]
    _frames_file(tmp_path / "t.bin", encs_t)
    _frames_file(tmp_path / "e.bin", encs_e)
    print(f"dropin: driver TDT/EOU B=3 T={T} window={W}", flush=True)
    r = subprocess.run([DRIVER, tdt_path, str(tmp_path / "t.bin"), eou_path, str(tmp_path / "e.bin"), str(W), "20"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout)

    dt = pk.Decoder.from_gguf(tdt_path, n_slots=3)
    ref_t = dt.decode(encs_t, trace=True)
    pieces_t, blank_t = dt.info.pieces, dt.info.blank
    # the drop-in's tokens against the oracle: the same window replayed through it
    # (teacher-forced on the decisions, zero unexplained mismatches, final state within 1e-3)
    omt = oracle.OracleModel.from_gguf(tdt_path, G)
    for u in range(3):
        check_window(omt, dt, u, encs_t[u], ref_t[u], omt.new_state(), 10)
    dt.close()
    t = out["tdt"]
    for u in range(3):
        want = ref_t[u]["tokens"].tolist()
        assert t["greedy"][u] == want, u
        assert t["chunked"][u] == want, u
        assert t["batch"][u] == want, u
        assert t["steps"][u] == ref_t[u]["steps"], u
        assert t["text"][u] == _detok(pieces_t, want, {blank_t}), u
    # value semantics of a copied / assigned state
    assert t["slots_distinct"] == 1
    assert t["tail_a"] == t["tail_b"] == t["tail_c"]
    assert t["head"] + t["tail_a"] == ref_t[0]["tokens"].tolist()
    assert t["bad_dim_rc"] == 1
    assert t["call_steps"] == ref_t[0]["steps"] and t["call_us"] > 0

    de = pk.Decoder.from_gguf(eou_path, n_slots=3)
    ref_e = de.decode(encs_e, max_symbols=5)
    pieces_e, blank_e = de.info.pieces, de.info.blank
    de.close()
    om = oracle.OracleModel.from_gguf(eou_path, G)
    e = out["eou"]
    for u in range(3):
        want = ref_e[u]["tokens"].tolist()
        assert e["greedy"][u] == want, u
        assert e["batch"][u] == want, u
        assert e["chunked"][u] == want, u
        assert e["segments"][u] == ref_e[u]["segments"].tolist(), u
        assert e["batch_segments"][u] == ref_e[u]["segments"].tolist(), u
        # windows decoded into fresh vectors: boundaries count from each window's start
        st = om.new_state()
        om.init_state(st)
        segs = []
        for t0 in range(0, T, W):
            segs += om.decode_window(encs_e[u][t0:t0 + W], st, 5, tokens_before=0)["segments"].tolist()
        assert e["chunked_segments"][u] == segs, u
        # src/parakeet_eou.cpp:359-382: each segment detokenized and trimmed, non-empty ones joined by '\n'
        bounds = [0] + ref_e[u]["segments"].tolist() + [len(want)]
        parts = [_detok(pieces_e, want[a:b], {blank_e}).strip(" \t\r\n") for a, b in zip(bounds, bounds[1:])]
        assert e["text"][u] == "\n".join(p for p in parts if p), u
    assert sum(len(s) for s in e["segments"]) > 0   # the raised <EOU> bias does end segments
    print(f"dropin: tdt_greedy_decode B=1 T={T}: {t['call_us']:.1f} us per call, {t['call_steps']} steps "
          f"({t['call_us'] / max(1, t['call_steps']):.2f} us/step)", flush=True)


@pytest.mark.gpu
def test_dropin_window_past_the_stamp(tmp_path):
    """A window longer than one launch of the decode loop takes, through the
    drop-in: tdt_greedy_decode over 24,000 frames at the default symbol cap (past
    the 23,830 frames of one launch, so pk_decode chains launches) returns the
    same tokens and steps as the same utterance decoded by tdt_decode_window in
    three 8,000-frame windows on one state, and as the C ABI.  The reference's
    loop has no length limit (src/parakeet_tdt.cpp:917-967)."""
    if not os.path.exists(DRIVER):
        pytest.skip("the drop-in driver is built only where parakeet.cpp's sources are present")
    from parakeet_amd import pk, synth
    tdt_path, eou_path = str(tmp_path / "t.gguf"), str(tmp_path / "e.gguf")
    small_tdt(tdt_path)
    small_eou(eou_path)
    T, W = 24000, 8000
    _frames_file(tmp_path / "t.bin", [synth.encoder_frames(970, T, 128)])
    _frames_file(tmp_path / "e.bin", [synth.encoder_frames(971, 10, 64)])
    dt = pk.Decoder.from_gguf(tdt_path, n_slots=2)
    _, k = pk.window_split([T], 10, dt.info.J, 5)
    assert k[0] >= 2, k
    print(f"dropin: tdt_greedy_decode over T={T} ({k[0]} launches), windows of {W}", flush=True)
    r = subprocess.run([DRIVER, tdt_path, str(tmp_path / "t.bin"), eou_path, str(tmp_path / "e.bin"), str(W), "1"],
                       capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr[-2000:]
    t = json.loads(r.stdout)["tdt"]
    ref = dt.decode([synth.encoder_frames(970, T, 128)], slots=[0])[0]
    dt.close()
    assert t["greedy"][0] == t["chunked"][0] == ref["tokens"].tolist()
    assert t["steps"][0] == ref["steps"]
    print(f"  {len(t['greedy'][0])} tokens, {ref['steps']} steps", flush=True)


@pytest.mark.gpu
def test_dropin_static_runtime_exits_cleanly(tmp_path):
    """The reference CLI keeps each runtime in a function-local static
    (src/main.cpp:746, :761) that is destroyed after main returns: the process
    must exit 0 with both runtimes alive at exit, and decode as the C ABI does."""
    if not os.path.exists(DRIVER):
        pytest.skip("the drop-in driver is built only where parakeet.cpp's sources are present")
    from parakeet_amd import pk, synth
    tdt_path, eou_path = str(tmp_path / "t.gguf"), str(tmp_path / "e.gguf")
    small_tdt(tdt_path)
    small_eou(eou_path)
    encs_t = [synth.encoder_frames(970, 30, 128)]
    encs_e = [synth.encoder_frames(971, 30, 64)]
    _frames_file(tmp_path / "t.bin", encs_t)
    _frames_file(tmp_path / "e.bin", encs_e)
    print("dropin: --static-exit driver", flush=True)
    r = subprocess.run([DRIVER, "--static-exit", tdt_path, str(tmp_path / "t.bin"), eou_path,
                        str(tmp_path / "e.bin")], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (r.returncode, r.stderr)
    out = json.loads(r.stdout)["static_exit"]
    dt = pk.Decoder.from_gguf(tdt_path, n_slots=1)
    assert out[0] == dt.decode(encs_t)[0]["tokens"].tolist()
    dt.close()
    de = pk.Decoder.from_gguf(eou_path, n_slots=1)
    assert out[1] == de.decode(encs_e, max_symbols=de.info.max_symbols)[0]["tokens"].tolist()
    de.close()
