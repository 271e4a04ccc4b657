"""Full-size parity on the device, checked against the oracle.

  * TDT-0.6b-v3 q8_0, B=256 x 750 frames (the large-batch target workload):
    bitwise batch invariance for a sample, teacher-forced oracle replay of
    the sample, and the joint logits of the first steps within 1e-3.
  * TDT-1.1b f16, B=256 x 375 frames (full length): batch invariance and
    replay of a sample.
  * Exact ties on the device: all-equal logits (zero joint output) must pick
    index 0 of both heads; equal maxima far apart must pick the lower index,
    whichever workgroups and argmax shards hold them
    (src/parakeet_tdt.cpp:25-32, first index of the maximum).
  * Logit taps at B=64 for every utterance.
  * Encoder frames resident in device memory (the encoder-to-decoder
    handoff), replayed through the oracle.

Tolerances: tokens and durations exact except at near-ties (oracle top-2
margin < 1e-4, counted); h, c and logits within 1e-3 L2-relative."""
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from parity import STATE_RTOL, TIE_EPS, rel

pytestmark = pytest.mark.gpu

THREADS = max(1, min(16, os.cpu_count() or 1))
LOGIT_RTOL = 1e-3


def _replay(om, encs, res, max_symbols, n_tap=0, blank_bias=None):
    def one(i):
        st = om.new_state()
        bb = 0.0 if blank_bias is None else float(blank_bias[i])
        rep = om.replay_window(encs[i], st, max_symbols, res[i]["trace"], blank_bias=bb, tie_eps=TIE_EPS,
                               n_tap=n_tap)
        return rep, st
    with ThreadPoolExecutor(THREADS) as ex:
        return list(ex.map(one, range(len(encs))))


def _check(dev, slots, res, reps, n_tap=0):
    near = 0
    worst_state = worst_logit = 0.0
    for k, (r, (rep, st)) in enumerate(zip(res, reps)):
        s = rep["stats"]
        assert rep["rc"] == 0 and s["structure_error"] == 0, (k, s)
        assert s["unexplained"] == 0, (k, s)
        assert rep["tokens"].tolist() == r["tokens"].tolist(), k
        near += s["near_ties"]
        d = dev.read_state(slots[k])
        worst_state = max(worst_state, rel(d["h"], st.h), rel(d["c"], st.c))
        for j in range(min(n_tap, r["steps"])):
            worst_logit = max(worst_logit, rel(r["logits"][j], rep["logits"][j]))
    assert worst_state < STATE_RTOL, worst_state
    assert worst_logit < LOGIT_RTOL, worst_logit
    return near, worst_state, worst_logit


@pytest.fixture(scope="module")
def tdt06(tmp_path_factory):
    from parakeet_amd import gguf, synth
    import oracle
    path = str(tmp_path_factory.mktemp("m") / "tdt06.gguf")
    synth.make_shape(path, "tdt-0.6b-v3")
    return path, oracle.OracleModel.from_gguf(path, gguf)


def test_tdt06_q8_b256x750(tdt06):
    """B=256 utterances x 750 frames in one lockstep call (sixteen 16-utterance
    domains); logits of the first 4 steps tapped for every utterance."""
    from parakeet_amd import pk, synth
    path, om = tdt06
    B, T, TAP = 256, 750, 4
    dev = pk.Decoder.from_gguf(path, n_slots=B + 8)
    encs = [synth.encoder_frames(u, T, 1024) for u in range(B)]
    print(f"[tdt06 b256] decoding {B}x{T}", flush=True)
    res = dev.decode(encs, trace=True, logit_steps=TAP)
    sample = [0, 101, 200, 255]
    for k, u in enumerate(sample):
        alone = dev.decode([encs[u]], slots=[B + k], trace=True)[0]
        assert np.array_equal(alone["trace"], res[u]["trace"]), u
    reps = _replay(om, [encs[u] for u in sample], [res[u] for u in sample], 10, n_tap=TAP)
    near, ws, wl = _check(dev, sample, [res[u] for u in sample], reps, n_tap=TAP)
    steps = sum(r["steps"] for r in res)
    print(f"tdt06 b256x750: steps={steps} sample near_ties={near} state_rel={ws:.2e} logit_rel={wl:.2e}")
    dev.close()


def test_tdt11b_f16_b256x375_full_length(tmp_path):
    """TDT-1.1b shapes, f16 weights, B=256 x 375 frames (the full workload)."""
    from parakeet_amd import gguf, pk, synth
    import oracle
    path = str(tmp_path / "tdt11.gguf")
    synth.make_shape(path, "tdt-1.1b")
    B, T = 256, 375
    dev = pk.Decoder.from_gguf(path, n_slots=B + 4)
    om = oracle.OracleModel.from_gguf(path, gguf)
    encs = [synth.encoder_frames(u, T, 1024) for u in range(B)]
    print(f"[tdt11 b256] decoding {B}x{T}", flush=True)
    res = dev.decode(encs, trace=True, logit_steps=2)
    sample = [3, 64, 190, 254]
    for k, u in enumerate(sample):
        alone = dev.decode([encs[u]], slots=[B + k], trace=True)[0]
        assert np.array_equal(alone["trace"], res[u]["trace"]), u
    reps = _replay(om, [encs[u] for u in sample], [res[u] for u in sample], 10, n_tap=2)
    near, ws, wl = _check(dev, sample, [res[u] for u in sample], reps, n_tap=2)
    print(f"tdt11 b256x375: steps={sum(r['steps'] for r in res)} near_ties={near} state_rel={ws:.2e} "
          f"logit_rel={wl:.2e}")
    dev.close()


def test_b64_logit_taps_every_utterance(tdt06):
    """B=64 x 40 frames: the first 6 steps' logits of every utterance."""
    from parakeet_amd import pk, synth
    path, om = tdt06
    B, T, TAP = 64, 40, 6
    dev = pk.Decoder.from_gguf(path, n_slots=B)
    encs = [synth.encoder_frames(3000 + u, T, 1024) for u in range(B)]
    res = dev.decode(encs, trace=True, logit_steps=TAP)
    reps = _replay(om, encs, res, 10, n_tap=TAP)
    near, ws, wl = _check(dev, list(range(B)), res, reps, n_tap=TAP)
    print(f"b64 taps: near_ties={near} state_rel={ws:.2e} logit_rel={wl:.2e}")
    dev.close()


# ---------------------------------------------------------------- exact ties

def _tie_decoder(path, bias):
    from parakeet_amd import pk, synth
    Vo = 8198
    ov = {"tdt.joint.out.weight": np.zeros((Vo, 640), np.float32),
          "tdt.joint.out.bias": np.asarray(bias, np.float32)}
    synth.make_shape(path, "tdt-0.6b-v3", overrides=ov)
    return pk.Decoder.from_gguf(path, n_slots=260)


@pytest.mark.parametrize("B", [1, 64])
def test_all_equal_logits_pick_index_zero(tmp_path, B):
    """Zero joint output: every logit is exactly 0, so the token is 0 (not
    blank) and the duration index 0 (duration 0): max_symbols emissions of
    token 0 per frame.  Rows are spread over every workgroup of the domain."""
    from parakeet_amd import synth
    dev = _tie_decoder(str(tmp_path / "z.gguf"), np.zeros(8198, np.float32))
    T = 5
    res = dev.decode([synth.encoder_frames(u, T, 1024) for u in range(B)], trace=True)
    for r in res:
        assert r["tokens"].tolist() == [0] * (10 * T)
        assert r["steps"] == 10 * T
        assert np.all(r["trace"] == 0)
    dev.close()


@pytest.mark.parametrize("B", [1, 64, 256])
def test_equal_maxima_pick_lowest_index(tmp_path, B):
    """Equal maxima at tokens 300, 5000 and 8000 (different row tiles, so
    different workgroups and argmax shards) and at duration indices 1 and 3:
    token 300 and duration 1 win.  Blank (8192) sits just below."""
    from parakeet_amd import synth
    bias = np.zeros(8198, np.float32)
    bias[[300, 5000, 8000]] = 1.0
    bias[8192] = 0.999
    bias[8193 + 1] = bias[8193 + 3] = 1.0
    dev = _tie_decoder(str(tmp_path / "t.gguf"), bias)
    T = 6
    res = dev.decode([synth.encoder_frames(u, T, 1024) for u in range(B)], trace=True)
    for r in res:
        assert r["tokens"].tolist() == [300] * T     # duration 1: one emission per frame
        assert r["trace"][:, 1].tolist() == [1] * T
    dev.close()


# ---------------------------------------------------------------- device handoff

@pytest.mark.parametrize("kind", ["tdt", "eou"])
def test_device_frames_replay_through_oracle(tmp_path, kind):
    """Encoder frames left in device memory (ragged windows at scattered rows of
    one array, PK_MEM_DEVICE_FRAMES), decoded in place: every window replays
    through the oracle from the host copy of the same rows, logits tapped."""
    from parakeet_amd import gguf, hipmem, pk, synth
    import oracle
    from conftest import small_eou, small_tdt
    path = str(tmp_path / "m.gguf")
    (small_tdt if kind == "tdt" else small_eou)(path)
    dec = pk.Decoder.from_gguf(path, n_slots=8)
    om = oracle.OracleModel.from_gguf(path, gguf)
    D = dec.info.D
    Ts = [23, 7, 0, 31, 12] if kind == "eou" else [23, 7, 1, 31, 12]
    rows = np.array([50, 0, 48, 10, 90], np.int64)
    frames = np.full((110, D), np.nan, np.float32)
    for u, T in enumerate(Ts):
        frames[rows[u]:rows[u] + T] = synth.encoder_frames(700 + u, T, D)
    enc_d = hipmem.DeviceArray.from_numpy(frames)
    hipmem.synchronize()
    ms = dec.info.max_symbols
    got = dec.decode_device_frames(enc_d.ptr, rows, Ts, slots=list(range(5)), trace=True, logit_steps=3)
    encs = [frames[rows[u]:rows[u] + T] for u, T in enumerate(Ts)]
    reps = _replay(om, encs, got, ms, n_tap=3)
    near, ws, wl = _check(dec, list(range(5)), got, reps, n_tap=3)
    for u in range(5):
        if kind == "eou":
            assert reps[u][0]["segments"].tolist() == got[u]["segments"].tolist(), u
    enc_d.free()
    dec.close()
