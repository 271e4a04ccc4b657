"""Teacher-forced parity check of device decodes against the oracle.

The device returns, per utterance, the (token, duration index) it chose at
every joint evaluation.  The oracle replays the same window following those
decisions (so one legitimate near-tie cannot desynchronise the comparison)
and, at every step, checks that the device's choice is the oracle argmax or
lies within ``TIE_EPS`` of it.  The final LSTM state of the device slot is
compared with the replayed oracle state (L2-relative, bound ``STATE_RTOL``).
"""
import numpy as np

TIE_EPS = 1e-4        # top-2 margin below which a disagreement is a near-tie
STATE_RTOL = 1e-3     # L2-relative bound on h, c


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def check_window(om, dev, slot, enc, res, ostate, max_symbols, blank_bias=0.0, tokens_before=0,
                 compare_state=True):
    """Replay one device window on oracle state ``ostate`` (advanced in place).
    Returns the replay stats; asserts the parity bar."""
    rep = om.replay_window(enc, ostate, max_symbols, res["trace"], blank_bias=blank_bias,
                           tie_eps=TIE_EPS, tokens_before=tokens_before)
    s = rep["stats"]
    assert rep["rc"] == 0, rep
    assert s["structure_error"] == 0, s
    assert s["unexplained"] == 0, s
    assert len(res["trace"]) == res["steps"], (len(res["trace"]), res["steps"])
    assert np.array_equal(rep["tokens"], res["tokens"]), "emitted tokens differ from the replay"
    if "segments" in res and om.kind == 1:
        assert np.array_equal(rep["segments"], res["segments"]), (rep["segments"], res["segments"])
    if compare_state:
        st = dev.read_state(slot)
        assert rel(st["h"], ostate.h) < STATE_RTOL, rel(st["h"], ostate.h)
        assert rel(st["c"], ostate.c) < STATE_RTOL, rel(st["c"], ostate.c)
        ctrl = st["ctrl"]
        assert ctrl[0] == 1
        assert ctrl[1] == ostate.st.symbols_this_step, (ctrl[1], ostate.st.symbols_this_step)
        if om.kind == 0:
            assert ctrl[2] == ostate.st.carry_frames, (ctrl[2], ostate.st.carry_frames)
        else:
            assert ctrl[3] == ostate.st.last_token
            assert ctrl[4] == ostate.st.segment_start_token
    return s


def free_run_equal(om, enc, res, max_symbols, blank_bias=0.0):
    """Free-running oracle decode; equal to the device stream unless a
    near-tie was taken differently (then the replay check above holds)."""
    st = om.new_state()
    ref = om.decode_window(enc, st, max_symbols, blank_bias=blank_bias)
    return np.array_equal(ref["tokens"], res["tokens"]) and ref["steps"] == res["steps"]
