"""Streaming windows with carried device state (src/parakeet_engine.cpp:409-452,
808-838): every window is checked against the oracle carrying the same state,
and the chunked token stream must equal the one-shot stream
(test/test_eou_streaming.cpp:164-187 pins the same invariant for EOU)."""
import numpy as np
import pytest

from conftest import small_eou, small_tdt
from parity import check_window

pytestmark = pytest.mark.gpu


def _models(path, writer, **kw):
    from parakeet_amd import gguf, pk
    import oracle
    writer(path, **kw)
    return pk.Decoder.from_gguf(path, n_slots=8), oracle.OracleModel.from_gguf(path, gguf)


@pytest.mark.parametrize("chunk", [1, 2, 3, 5])
def test_tdt_chunked_windows(tmp_path, chunk):
    """Every window matches the oracle carrying the same state.  With windows of
    at least 3 frames (max duration 4 -> carry <= 3) the chunked stream equals
    the one-shot stream; shorter windows drop the part of carry_frames that
    exceeds the next window (src/parakeet_tdt.cpp:906-910 then :979), as the
    reference does, so only the per-window check applies there."""
    from parakeet_amd import synth
    dev, om = _models(str(tmp_path / "m.gguf"), small_tdt)
    enc = synth.encoder_frames(7, 33, 128)
    one = dev.decode([enc], slots=[1], trace=True)[0]
    dev.reset_state(0)
    ost = om.new_state()
    toks = []
    for s0 in range(0, len(enc), chunk):
        w = enc[s0:s0 + chunk]
        r = dev.decode([w], slots=[0], trace=True)[0]
        check_window(om, dev, 0, w, r, ost, 10)
        toks.extend(r["tokens"].tolist())
    if chunk >= 3:
        assert toks == one["tokens"].tolist()


def test_eou_chunked_sessions(tmp_path):
    """Config-4-like: several sessions, 2-frame chunks, h/c/last token carried;
    segment indices count from the caller's running token total."""
    from parakeet_amd import synth
    dev, om = _models(str(tmp_path / "e.gguf"), small_eou)
    B, n_chunks = 6, 12
    encs = [synth.encoder_frames(300 + u, 2 * n_chunks, 64) for u in range(B)]
    for u in range(B):
        dev.init_state(u)
    ost = [om.new_state() for _ in range(B)]
    for o in ost:
        om.init_state(o)
    total = np.zeros(B, np.int32)
    all_toks = [[] for _ in range(B)]
    all_segs = [[] for _ in range(B)]
    for c in range(n_chunks):
        ws = [e[2 * c:2 * c + 2] for e in encs]
        res = dev.decode(ws, slots=list(range(B)), trace=True, tokens_base=total, max_symbols=5)
        for u in range(B):
            check_window(om, dev, u, ws[u], res[u], ost[u], 5, tokens_before=int(total[u]))
            all_toks[u].extend(res[u]["tokens"].tolist())
            all_segs[u].extend(res[u]["segments"].tolist())
            total[u] += len(res[u]["tokens"])
    # one-shot device decode of the whole stream gives the same tokens and boundaries
    for u in range(2):
        dev.reset_state(7)
        r = dev.decode([encs[u]], slots=[7], max_symbols=5)[0]
        assert r["tokens"].tolist() == all_toks[u]
        assert r["segments"].tolist() == all_segs[u]


def test_slot_init_matches_oracle_init(tmp_path):
    dev, om = _models(str(tmp_path / "m.gguf"), small_tdt)
    dev.init_state(3)
    st = dev.read_state(3)
    o = om.new_state()
    om.init_state(o)
    from parity import rel
    assert rel(st["h"], o.h) < 1e-5 and rel(st["c"], o.c) < 1e-5
    assert st["ctrl"][0] == 1 and st["ctrl"][1] == 0 and st["ctrl"][2] == 0


def test_empty_tdt_window_leaves_state(tmp_path):
    """n_frames <= 0 returns before initialising (src/parakeet_tdt.cpp:879)."""
    dev, om = _models(str(tmp_path / "m.gguf"), small_tdt)
    dev.reset_state(2)
    r = dev.decode([np.zeros((0, 128), np.float32)], slots=[2])[0]
    assert r["steps"] == 0 and len(r["tokens"]) == 0
    assert dev.read_state(2)["ctrl"][0] == 0
