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
  boundaries (test/test_eou_streaming.cpp:164-187).  A boundary's token_index
  is the size of the caller's token vector and state.segment_start_token
  carries over (src/parakeet_eou.cpp:293-299), so windows decoded into fresh
  vectors (as the Engine's Mode 2/3 do) give the oracle's per-window
  boundaries, not the one-shot ones;
- Engine::transcribe_features gives tdt_greedy_decode's result;
- streaming over features (the decode half of Mode 2, src/parakeet_engine.cpp:389-489,
  and of Mode 3, :753-864): one segment per chunk whose tokens are that
  window's decode, whose text is the growth of detokenize(all tokens so far),
  timed by the encoder frame stride 1000 * hop * subsampling / sample_rate
  (:35-41); one EndOfTurn event (confidence 1) per EOU boundary of the chunk;
  sessions fed in one launch equal sessions fed one at a time;
- the encoder output resident in device memory (the handoff that replaces the
  host copy of src/parakeet_ctc.cpp:1660-1667): ragged windows decoded in place
  by tdt/eou_decode_batch_device and Engine::transcribe_device_batch equal the
  same windows decoded from host memory and through the C ABI; a window past
  the end of the output returns 3 and a d_model mismatch 1."""
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
    import oracle
    from parakeet_amd import gguf as G, pk, synth
    tdt_path, eou_path = str(tmp_path / "t.gguf"), str(tmp_path / "e.gguf")
    small_tdt(tdt_path)
    # EOU model with a 4x subsampling encoder (frame stride 1000 * 160 * 4 / 16000 = 40 ms)
    # whose <EOU> logit (id 33) is raised by 1.5, so that segments end now and then
    w = small_eou(eou_path)
    bias = w["eou.joint.out.bias"].copy()
    bias[33] += 1.5
    small_eou(eou_path, meta_u32={"parakeet.encoder.subsampling_factor": 4}, overrides={"eou.joint.out.bias": bias})
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

    dt = pk.Decoder.from_gguf(tdt_path, n_slots=6)
    ref_t = dt.decode(encs_t)
    lens = [max(1, T - (u % 4) * (T // 8)) for u in range(3)]   # the driver's ragged windows
    rag_t = dt.decode([encs_t[u][:lens[u]] for u in range(3)], slots=[3, 4, 5])   # fresh states
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

    de = pk.Decoder.from_gguf(eou_path, n_slots=6)
    ref_e = de.decode(encs_e, max_symbols=5)
    rag_e = de.decode([encs_e[u][:lens[u]] for u in range(3)], slots=[3, 4, 5], max_symbols=5)
    # the oracle, windows decoded into fresh token vectors with the state carried
    om = oracle.OracleModel.from_gguf(eou_path, G)
    chunks = [[] for _ in range(3)]
    for u in range(3):
        st = om.new_state()
        om.init_state(st)
        for t0 in range(0, T, W):
            r = om.decode_window(encs_e[u][t0:t0 + W], st, 5, tokens_before=0)
            chunks[u].append((r["tokens"].tolist(), r["segments"].tolist()))
    for u in range(3):
        assert out["eou"]["greedy"][u] == ref_e[u]["tokens"].tolist(), u
        assert out["eou"]["segments"][u] == ref_e[u]["segments"].tolist(), u
        assert out["eou"]["chunked"][u] == ref_e[u]["tokens"].tolist(), u
        assert out["eou"]["chunked_segments"][u] == sum((sg for _, sg in chunks[u]), []), u
    chunks = [[(tk, len(sg)) for tk, sg in c] for c in chunks]
    pieces_e = de.info.pieces
    blank_e = de.info.blank
    de.close()

    st = out["stream"]
    stride = 80.0   # TDT model: metadata defaults 1000 * 160 * 8 / 16000
    assert abs(st["stride_ms"] - stride) < 1e-9
    want = ref_t[0]["tokens"].tolist()
    assert st["tdt_tokens"] == want and st["tdt_steps"] == ref_t[0]["steps"]
    assert st["tdt_text"] == _detok(pieces_t, want, {blank_t})
    segs = st["tdt"]["segments"]
    assert [g["chunk"] for g in segs] == list(range((T + W - 1) // W))
    assert sum((g["tokens"] for g in segs), []) == want
    cum = []
    for k, g in enumerate(segs):
        before = _detok(pieces_t, cum, {blank_t})
        cum += g["tokens"]
        assert g["text"] == _detok(pieces_t, cum, {blank_t})[len(before):], k
        assert abs(g["start"] - k * W * stride / 1000) < 1e-6
        assert abs(g["end"] - min(T, (k + 1) * W) * stride / 1000) < 1e-6
        assert g["eou"] == 0 and g["final"] == 1
    assert st["tdt"]["events"] == []
    assert st["eou_batch"] == st["eou_single"]
    estride = 40.0
    n_events = 0
    for u in range(3):
        log = st["eou_batch"][u]
        assert len(log["segments"]) == len(chunks[u])
        cum = []
        want_events = []
        for k, (g, (toks, nb)) in enumerate(zip(log["segments"], chunks[u])):
            before = _detok(pieces_e, cum, {blank_e})
            cum += toks
            assert g["chunk"] == k and g["tokens"] == toks, (u, k)
            assert g["text"] == _detok(pieces_e, cum, {blank_e})[len(before):], (u, k)
            assert g["eou"] == (1 if nb > 0 else 0), (u, k)
            assert abs(g["end"] - min(T, (k + 1) * W) * estride / 1000) < 1e-6
            want_events += [k] * nb
        assert [e["chunk"] for e in log["events"]] == want_events, u
        for e in log["events"]:
            assert e["type"] == 2 and e["conf"] == 1.0
            assert abs(e["t"] - min(T, (e["chunk"] + 1) * W) * estride / 1000) < 1e-6
        assert cum == ref_e[u]["tokens"].tolist()
        n_events += len(log["events"])
    assert n_events == sum(len(s) for s in out["eou"]["chunked_segments"])
    assert n_events > 0        # the synthetic EOU model does fire <EOU> on these frames

    dv = out["device"]
    for u in range(3):
        want_t, want_e = rag_t[u]["tokens"].tolist(), rag_e[u]["tokens"].tolist()
        assert dv["tdt_host"][u] == want_t, ("tdt host frames", u)
        assert dv["tdt_dev"][u] == want_t, ("tdt device frames", u)
        assert dv["tdt_steps_host"][u] == dv["tdt_steps_dev"][u] == rag_t[u]["steps"], u
        assert dv["eou_host"][u] == want_e, ("eou host frames", u)
        assert dv["eou_dev"][u] == want_e, ("eou device frames", u)
        assert dv["eou_seg_host"][u] == dv["eou_seg_dev"][u] == rag_e[u]["segments"].tolist(), u
        assert dv["engine_host"][u] == want_t, ("engine host frames", u)
        assert dv["engine_dev"][u] == want_t, ("engine device frames", u)
    assert dv["engine_text_equal"] == 1
    assert dv["rc_range"] == 3 and dv["rc_dim"] == 1
    print("cpp api: tokens", [len(x) for x in out["tdt"]["greedy"]], [len(x) for x in out["eou"]["greedy"]],
          "eou segments", [len(x) for x in out["eou"]["segments"]], "EndOfTurn events", n_events)
