"""Runs of blanks over the joint tile's spare columns.

A blank decision keeps the prediction output, so while an utterance is in a
run of blanks the joint's spare columns (a 16-column tile holds fewer
utterances than columns) evaluate its next frames in the same iteration, and
the decision step walks the run there.  The steps are the same joint
evaluations the one-step-per-iteration loop makes, so:

- every decision replays through the oracle (teacher-forced, zero unexplained
  mismatches, final state within 1e-3), TDT and EOU, blank-heavy decodes;
- tokens, steps, traces, segments and final state equal the loop with the runs
  turned off (PK_SPEC=0), bit for bit, while the iteration count drops;
- windows carried across calls give the same stream as one call."""
import os

import numpy as np
import pytest

from conftest import small_eou, small_tdt
from parity import check_window

pytestmark = pytest.mark.gpu


def _both(dev, encs, n, **kw):
    """The same decode with the runs on and off (fresh slots each)."""
    os.environ["PK_SPEC"] = "0"
    try:
        off = dev.decode(encs, slots=list(range(n, 2 * n)), trace=True, **kw)
        it_off = dev.last_timing()["iterations"]
    finally:
        os.environ.pop("PK_SPEC", None)
    on = dev.decode(encs, slots=list(range(n)), trace=True, **kw)
    it_on = dev.last_timing()["iterations"]
    return on, off, it_on, it_off


@pytest.mark.parametrize("B", [1, 2, 4, 40])
def test_tdt_blank_runs_replay_and_equal(tmp_path, B):
    """B=1 and B=2 run the one-domain loop, whose argmax exchange switches between
    the per-workgroup key slots (at most 2 joint columns) and the sharded atomics
    (spare columns in use) from one iteration to the next."""
    from parakeet_amd import gguf, pk, synth
    import oracle
    path = str(tmp_path / "m.gguf")
    small_tdt(path)
    dev = pk.Decoder.from_gguf(path, n_slots=2 * B)
    om = oracle.OracleModel.from_gguf(path, gguf)
    encs = [synth.encoder_frames(1200 + u, 60 - (u % 5) * 7, 128) for u in range(B)]
    bb = np.full(B, 3.0, np.float32)
    print(f"blank runs: TDT B={B}, blank +3", flush=True)
    on, off, it_on, it_off = _both(dev, encs, B, blank_bias=bb, max_symbols=10)
    for u in range(B):
        assert np.array_equal(on[u]["tokens"], off[u]["tokens"]), u
        assert np.array_equal(on[u]["trace"], off[u]["trace"]), u
        assert on[u]["steps"] == off[u]["steps"], u
        a, b = dev.read_state(u), dev.read_state(B + u)
        assert np.array_equal(a["h"], b["h"]) and np.array_equal(a["c"], b["c"]), u
        assert np.array_equal(a["ctrl"], b["ctrl"]), u
        check_window(om, dev, u, encs[u], on[u], om.new_state(), 10, blank_bias=3.0)
    assert it_on < it_off, (it_on, it_off)
    print(f"  iterations {it_on} with runs, {it_off} without", flush=True)
    dev.close()


def test_eou_blank_runs_replay_and_equal(tmp_path):
    from parakeet_amd import gguf, pk, synth
    import oracle
    path = str(tmp_path / "e.gguf")
    w = small_eou(path)
    bias = w["eou.joint.out.bias"].copy()
    bias[33] += 1.0   # <EOU> now and then, so resets interrupt the runs
    small_eou(path, overrides={"eou.joint.out.bias": bias})
    dev = pk.Decoder.from_gguf(path, n_slots=6)
    om = oracle.OracleModel.from_gguf(path, gguf)
    encs = [synth.encoder_frames(1300 + u, 50, 64) for u in range(3)]
    bb = np.full(3, 2.0, np.float32)
    on, off, it_on, it_off = _both(dev, encs, 3, blank_bias=bb, max_symbols=5)
    for u in range(3):
        for k in ("tokens", "trace", "segments"):
            assert np.array_equal(on[u][k], off[u][k]), (u, k)
        check_window(om, dev, u, encs[u], on[u], om.new_state(), 5, blank_bias=2.0)
    assert it_on < it_off, (it_on, it_off)
    dev.close()


def test_tdt_blank_runs_across_windows(tmp_path):
    """Windows of 7 frames with the state carried give the one-call stream (a run of
    blanks that reaches a window's end stops there and resumes in the next call)."""
    from parakeet_amd import pk, synth
    path = str(tmp_path / "m.gguf")
    small_tdt(path)
    dev = pk.Decoder.from_gguf(path, n_slots=2)
    enc = synth.encoder_frames(1400, 70, 128)
    bb = np.full(1, 3.0, np.float32)
    whole = dev.decode([enc], slots=[0], blank_bias=bb)[0]
    toks = []
    for t0 in range(0, 70, 7):
        toks += dev.decode([enc[t0:t0 + 7]], slots=[1], blank_bias=bb)[0]["tokens"].tolist()
    assert toks == whole["tokens"].tolist()
    dev.close()


@pytest.mark.parametrize("B", [1, 2])
def test_argmax_slots_equal_sharded_atomics(tmp_path, B):
    """One-domain launches exchange the argmax keys through per-workgroup slots
    while at most 2 joint columns are live; PK_ARGMAX_SLOTS=0 runs the same decode
    with the sharded atomics and barrier.  Tokens, steps, traces and final state
    are bit-identical, with and without runs of blanks (which switch the exchange
    between the two forms from one iteration to the next)."""
    from parakeet_amd import pk, synth
    path = str(tmp_path / "m.gguf")
    small_tdt(path)
    dev = pk.Decoder.from_gguf(path, n_slots=8 * B)
    encs = [synth.encoder_frames(1500 + u, 45 + 9 * u, 128) for u in range(B)]
    for k, bias in enumerate((0.0, 3.0)):
        bb = np.full(B, bias, np.float32)
        base = 4 * B * k
        os.environ["PK_ARGMAX_SLOTS"] = "0"
        try:
            ref = dev.decode(encs, slots=list(range(base + B, base + 2 * B)), trace=True, blank_bias=bb, max_symbols=5)
        finally:
            os.environ.pop("PK_ARGMAX_SLOTS", None)
        got = dev.decode(encs, slots=list(range(base, base + B)), trace=True, blank_bias=bb, max_symbols=5)
        for u in range(B):
            assert np.array_equal(got[u]["tokens"], ref[u]["tokens"]), (bias, u)
            assert np.array_equal(got[u]["trace"], ref[u]["trace"]), (bias, u)
            assert got[u]["steps"] == ref[u]["steps"], (bias, u)
            a, b = dev.read_state(base + u), dev.read_state(base + B + u)
            assert np.array_equal(a["h"], b["h"]) and np.array_equal(a["c"], b["c"]), (bias, u)
    dev.close()


@pytest.mark.parametrize("B", [2, 4, 40])
def test_logit_tap_with_blank_runs(tmp_path, B):
    """The logit tap with the runs on: the joint logits of every step, including
    the steps a run takes from a spare column (possibly several frames ahead,
    after a duration skip), equal the oracle's logits of the same step within
    1e-3 (src/parakeet_tdt.cpp:154-177), and the bits equal the tap with the
    runs off."""
    from parakeet_amd import gguf, pk, synth
    import oracle
    from parity import rel
    path = str(tmp_path / "tdt06.gguf")
    synth.make_shape(path, "tdt-0.6b-v3")
    dev = pk.Decoder.from_gguf(path, n_slots=2 * B)
    om = oracle.OracleModel.from_gguf(path, gguf)
    encs = [synth.encoder_frames(1300 + u, 40 + 3 * (u % 4), 1024) for u in range(B)]
    bb = np.full(B, 4.0, np.float32)
    TAP = 64
    print(f"logit tap with blank runs: TDT-0.6b B={B}, blank +4, {TAP} steps", flush=True)
    on, off, it_on, it_off = _both(dev, encs, B, blank_bias=bb, max_symbols=10, logit_steps=TAP)
    assert it_on < it_off, (it_on, it_off)           # the runs were taken
    worst = 0.0
    for u in range(B):
        assert np.array_equal(on[u]["trace"], off[u]["trace"]), u
        n = min(TAP, on[u]["steps"])
        assert np.array_equal(on[u]["logits"][:n], off[u]["logits"][:n]), u
        rep = om.replay_window(encs[u], om.new_state(), 10, on[u]["trace"], blank_bias=4.0, n_tap=TAP)
        assert rep["stats"]["unexplained"] == 0, rep["stats"]
        for j in range(n):
            worst = max(worst, rel(on[u]["logits"][j], rep["logits"][j]))
    assert worst < 1e-3, worst
    print(f"  iterations {it_on} (runs on) vs {it_off}; worst logit rel {worst:.2e}", flush=True)
