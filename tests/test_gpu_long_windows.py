"""Windows longer than one launch of the decode loop takes (the argmax keys'
18-bit iteration stamp, the 32-bit enc_proj offsets): pk_decode decodes them in
several launches with the state carried (pk_window_split).  The reference's
loops have no length limit (src/parakeet_tdt.cpp:917-967,
src/parakeet_eou.cpp:266-334), so such windows must decode exactly as a single
one would: every step is replayed through the oracle, and the result equals the
same window decoded by the caller as consecutive shorter windows."""
import numpy as np
import pytest

from conftest import small_eou, small_tdt
from parity import check_window

pytestmark = pytest.mark.gpu


def _models(path, writer, **kw):
    from parakeet_amd import gguf, pk
    import oracle
    w = writer(path, **kw)
    return pk.Decoder.from_gguf(path, n_slots=8), oracle.OracleModel.from_gguf(path, gguf), w


def test_tdt_window_past_the_stamp(tmp_path):
    """max_symbols 100: one launch takes at most 2,595 frames, so 6,000 frames
    run as 3 launches; replayed step by step through the oracle."""
    from parakeet_amd import pk, synth
    dev, om, _ = _models(str(tmp_path / "t.gguf"), small_tdt)
    S, T = 100, 6000
    W, k = pk.window_split([T], S, dev.info.J, 5)
    assert k[0] == 3, (W, k)
    enc = synth.encoder_frames(61, T, 128)
    print(f"long TDT window: T={T} max_symbols={S} in {k[0]} launches", flush=True)
    r = dev.decode([enc], slots=[0], max_symbols=S, trace=True)[0]
    ost = om.new_state()
    s = check_window(om, dev, 0, enc, r, ost, S)
    print(f"  {r['steps']} steps replayed, near-ties {s['near_ties']}", flush=True)
    # the caller's own windows of 2,000 frames (one launch each) give the same stream
    toks, steps = [], 0
    for t0 in range(0, T, 2000):
        q = dev.decode([enc[t0:t0 + 2000]], slots=[1], max_symbols=S)[0]
        toks += q["tokens"].tolist()
        steps += q["steps"]
    assert toks == r["tokens"].tolist() and steps == r["steps"]
    a, b = dev.read_state(0), dev.read_state(1)
    assert np.array_equal(a["h"], b["h"]) and np.array_equal(a["c"], b["c"])
    assert a["ctrl"].tolist() == b["ctrl"].tolist()


def test_eou_window_past_the_stamp(tmp_path):
    """EOU with <EOU> raised so that segments end: boundaries and the carried
    segment start across the internal launches equal the oracle's."""
    from parakeet_amd import synth
    path = str(tmp_path / "e.gguf")
    w = small_eou(path)
    bias = w["eou.joint.out.bias"].copy()
    bias[33] += 1.5
    dev, om, _ = _models(path, small_eou, overrides={"eou.joint.out.bias": bias})
    S, T = 100, 5400
    enc = synth.encoder_frames(62, T, 64)
    print(f"long EOU window: T={T} max_symbols={S}", flush=True)
    dev.init_state(0)
    r = dev.decode([enc], slots=[0], max_symbols=S, trace=True, tokens_base=[7])[0]
    ost = om.new_state()
    om.init_state(ost)
    check_window(om, dev, 0, enc, r, ost, S, tokens_before=7)
    assert len(r["segments"]) > 0


def test_device_outputs_long_window(tmp_path):
    """Frames and outputs in device memory (PK_MEM_DEVICE) with a split window:
    the same tokens, steps and trace as host outputs."""
    from parakeet_amd import hipmem, synth
    dev, om, _ = _models(str(tmp_path / "t.gguf"), small_tdt)
    S, Ts = 100, np.array([5300, 40, 0, 2700], np.int32)
    encs = [synth.encoder_frames(70 + u, int(t), 128) if t else np.zeros((0, 128), np.float32)
            for u, t in enumerate(Ts)]
    want = dev.decode(encs, slots=[0, 1, 2, 3], max_symbols=S, trace=True)
    frames = np.concatenate([e for e in encs if len(e)])
    rows = np.concatenate([[0], np.cumsum(Ts)[:-1]]).astype(np.int64)
    n, cap, tcap = len(Ts), int(Ts.max()) * S + 1, int(Ts.max()) * (S + 1) + 1
    fd = hipmem.DeviceArray.from_numpy(frames)
    out = dict(tokens=hipmem.DeviceArray(4 * n * cap), n_tokens=hipmem.DeviceArray(4 * n),
               steps=hipmem.DeviceArray(4 * n))
    tr = hipmem.DeviceArray(8 * n * tcap)
    ptrs = {k: v.ptr for k, v in out.items()}
    ptrs["trace"] = tr.ptr
    print("long window, device outputs", flush=True)
    dev.decode_device(fd.ptr, rows, Ts, np.arange(4, 8, dtype=np.int32), S, ptrs, cap, trace_cap=tcap)
    hipmem.synchronize()
    ntok = out["n_tokens"].to_numpy(np.int32, n)
    steps = out["steps"].to_numpy(np.int32, n)
    toks = out["tokens"].to_numpy(np.int32, n * cap).reshape(n, cap)
    trace = tr.to_numpy(np.int32, n * tcap * 2).reshape(n, tcap, 2)
    for u in range(n):
        assert toks[u, :ntok[u]].tolist() == want[u]["tokens"].tolist(), u
        assert steps[u] == want[u]["steps"], u
        assert np.array_equal(trace[u, :steps[u]], want[u]["trace"]), u
    for a in (fd, tr, *out.values()):
        a.free()


def test_tdt06b_b1_30000_frames(tmp_path):
    """TDT-0.6b-v3 shapes, B=1, 30,000 frames (40 minutes at 80 ms) at the
    default symbol cap: past the 23,830 frames one launch takes.  Replayed
    through the oracle on the first 4,000 frames' decisions (the sample), and
    equal to the same window decoded as three 10,000-frame windows."""
    from parakeet_amd import pk, synth
    path = str(tmp_path / "tdt06.gguf")
    synth.make_shape(path, "tdt-0.6b-v3")
    import oracle
    from parakeet_amd import gguf
    dev = pk.Decoder.from_gguf(path, n_slots=4)
    T = 30000
    W, k = pk.window_split([T], 10, dev.info.J, 5)
    assert k[0] >= 2
    enc = synth.encoder_frames(63, T, dev.info.D)
    print(f"TDT-0.6b B=1 T={T}: {k[0]} launches of <= {W} frames", flush=True)
    r = dev.decode([enc], slots=[0], trace=True)[0]
    toks, steps = [], 0
    for t0 in range(0, T, 10000):
        q = dev.decode([enc[t0:t0 + 10000]], slots=[1])[0]
        toks += q["tokens"].tolist()
        steps += q["steps"]
    assert toks == r["tokens"].tolist() and steps == r["steps"]
    a, b = dev.read_state(0), dev.read_state(1)
    assert np.array_equal(a["h"], b["h"]) and np.array_equal(a["c"], b["c"])
    # sampled replay: the decisions of the first 4,000 frames against the oracle
    om = oracle.OracleModel.from_gguf(path, gguf)
    n0 = 4000
    q = dev.decode([enc[:n0]], slots=[2], trace=True)[0]
    assert q["tokens"].tolist() == r["tokens"][:len(q["tokens"])].tolist()
    ost = om.new_state()
    s = check_window(om, dev, 2, enc[:n0], q, ost, 10)
    print(f"  {r['steps']} steps; replayed the first {q['steps']}, near-ties {s['near_ties']}", flush=True)


def _alone_equal(dev, encs, res, base, **kw):
    for u, e in enumerate(encs):
        a = dev.decode([e], slots=[base + u], trace=True, **{k: (v[u:u + 1] if hasattr(v, "__len__") else v)
                                                             for k, v in kw.items()})[0]
        assert np.array_equal(a["trace"], res[u]["trace"]), u
        assert a["tokens"].tolist() == res[u]["tokens"].tolist(), u
        assert a["segments"].tolist() == res[u]["segments"].tolist(), u
        x, y = dev.read_state(u), dev.read_state(base + u)
        assert np.array_equal(x["h"], y["h"]) and np.array_equal(x["c"], y["c"]), u
        assert x["ctrl"].tolist() == y["ctrl"].tolist(), u


def test_ragged_batch_equals_alone(tmp_path):
    """A ragged batch (T ~ U{20..400}, per-utterance blank bias): every utterance
    equals its decode alone, bit for bit (decisions, tokens, final state and
    control words), and the longest and shortest replay through the oracle."""
    from parakeet_amd import gguf, pk, synth
    import oracle
    path = str(tmp_path / "t.gguf")
    small_tdt(path)
    B = 40
    dev = pk.Decoder.from_gguf(path, n_slots=2 * B)
    om = oracle.OracleModel.from_gguf(path, gguf)
    rng = np.random.default_rng(17)
    Ts = rng.integers(20, 401, size=B)
    encs = [synth.encoder_frames(80 + u, int(Ts[u]), 128) for u in range(B)]
    bb = np.array([0.0, 2.0, 4.0] * 14, np.float32)[:B]
    print(f"ragged batch: B={B}, T in [{Ts.min()}, {Ts.max()}]", flush=True)
    res = dev.decode(encs, slots=list(range(B)), trace=True, blank_bias=bb)
    _alone_equal(dev, encs, res, B, blank_bias=bb)
    for u in (int(np.argmax(Ts)), int(np.argmin(Ts))):
        check_window(om, dev, u, encs[u], res[u], om.new_state(), 10, blank_bias=float(bb[u]))


def test_ragged_eou_equals_alone(tmp_path):
    """EOU ragged batch with per-utterance token bases: segments, tokens, state and
    control words equal each utterance decoded alone."""
    from parakeet_amd import pk, synth
    path = str(tmp_path / "e.gguf")
    w = small_eou(path)
    bias = w["eou.joint.out.bias"].copy()
    bias[33] += 1.5
    small_eou(path, overrides={"eou.joint.out.bias": bias})
    B = 36
    dev = pk.Decoder.from_gguf(path, n_slots=2 * B)
    rng = np.random.default_rng(18)
    Ts = rng.integers(10, 300, size=B)
    encs = [synth.encoder_frames(120 + u, int(Ts[u]), 64) for u in range(B)]
    base = rng.integers(0, 50, size=B).astype(np.int32)
    print(f"ragged EOU batch: B={B}", flush=True)
    res = dev.decode(encs, slots=list(range(B)), trace=True, max_symbols=5, tokens_base=base)
    _alone_equal(dev, encs, res, B, max_symbols=5, tokens_base=base)
    assert sum(len(r["segments"]) for r in res) > 0
