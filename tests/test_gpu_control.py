"""Control flow on the device with scripted logits (weights zeroed, biases set
so the argmax is forced), where token/duration sequences have closed forms;
blank bias; determinism; error codes."""
import numpy as np
import pytest

from conftest import small_eou, small_tdt

pytestmark = pytest.mark.gpu


def _zero_out(path, writer, out_bias, **kw):
    """Decoder whose joint output is exactly out_bias (joint.out weight zero)."""
    from parakeet_amd import pk
    p = "tdt" if writer is small_tdt else "eou"
    J = kw.get("J", 96)
    Vo = len(out_bias)
    ov = {f"{p}.joint.out.weight": np.zeros((Vo, J), np.float32),
          f"{p}.joint.out.bias": np.asarray(out_bias, np.float32)}
    writer(path, overrides=ov, **kw)
    return pk.Decoder.from_gguf(path, n_slots=4)


def test_tdt_nonblank_dur0_hits_symbol_cap(tmp_path):
    """token 5 with duration index 0 (dur 0): max_symbols emissions per frame."""
    V1, Dn = 62, 5
    bias = np.zeros(V1 + Dn, np.float32)
    bias[5] = 3.0
    bias[V1 + 0] = 2.0
    dev = _zero_out(str(tmp_path / "a.gguf"), small_tdt, bias)
    from parakeet_amd import synth
    T = 9
    for ms in (1, 3, 10):
        dev.reset_state(0)
        r = dev.decode([synth.encoder_frames(0, T, 128)], slots=[0], max_symbols=ms)[0]
        assert r["tokens"].tolist() == [5] * (ms * T)
        assert r["steps"] == ms * T


def test_tdt_blank_dur0_advances_one(tmp_path):
    V1, Dn = 62, 5
    bias = np.zeros(V1 + Dn, np.float32)
    bias[61] = 1.0          # blank
    bias[V1 + 0] = 1.0      # duration 0 -> advance max(1, 0)
    dev = _zero_out(str(tmp_path / "b.gguf"), small_tdt, bias)
    from parakeet_amd import synth
    r = dev.decode([synth.encoder_frames(0, 11, 128)], max_symbols=10)[0]
    assert r["steps"] == 11 and len(r["tokens"]) == 0


def test_tdt_duration_carry_across_windows(tmp_path):
    """token with duration 4 over windows of 3 frames: carry_frames spills."""
    V1, Dn = 62, 5
    bias = np.zeros(V1 + Dn, np.float32)
    bias[7] = 1.0
    bias[V1 + 4] = 1.0
    dev = _zero_out(str(tmp_path / "c.gguf"), small_tdt, bias)
    from parakeet_amd import synth
    enc = synth.encoder_frames(0, 3, 128)
    expected_carry = []
    t_global, emitted = 0, []
    for w in range(5):
        r = dev.decode([enc], slots=[0], max_symbols=10)[0]
        emitted.append(len(r["tokens"]))
        expected_carry.append(dev.read_state(0)["ctrl"][2])
    # frames advance 4 per emission over a 15-frame stream split into 3-frame windows
    # emissions at frames 0, 4, 8, 12 -> windows [0..3) [3..6) [6..9) [9..12) [12..15);
    # after the third window t = 2 + 4 = 6 in a 3-frame window: carry 3, consumed whole by the fourth
    assert emitted == [1, 1, 1, 0, 1], emitted
    assert expected_carry == [1, 2, 3, 0, 1], expected_carry


def test_eou_reset_and_segments(tmp_path):
    """EOU token always wins: state reset each step, a boundary only when the
    segment has tokens (src/parakeet_eou.cpp:292-310)."""
    V1 = 36
    bias = np.zeros(V1, np.float32)
    bias[33] = 1.0          # eou
    dev = _zero_out(str(tmp_path / "e.gguf"), small_eou, bias)
    from parakeet_amd import synth
    r = dev.decode([synth.encoder_frames(0, 6, 64)], max_symbols=5, tokens_base=[3])[0]
    assert r["steps"] == 6 and len(r["tokens"]) == 0
    # 3 tokens before the call, segment start 0 -> one boundary at 3
    assert r["segments"].tolist() == [3]
    st = dev.read_state(0)
    assert st["ctrl"][3] == 35 and st["ctrl"][4] == 3      # last = blank, segment start


def test_eou_special_piece_skips(tmp_path):
    """token 0 is "<unk>": skipped, frame ends (src/parakeet_eou.cpp:315-320)."""
    V1 = 36
    bias = np.zeros(V1, np.float32)
    bias[0] = 1.0
    dev = _zero_out(str(tmp_path / "s.gguf"), small_eou, bias)
    from parakeet_amd import synth
    r = dev.decode([synth.encoder_frames(0, 4, 64)], max_symbols=5)[0]
    assert r["steps"] == 4 and len(r["tokens"]) == 0


def test_blank_bias_matches_oracle(tmp_path):
    from parakeet_amd import gguf, pk, synth
    import oracle
    from parity import check_window
    path = str(tmp_path / "m.gguf")
    small_tdt(path)
    dev = pk.Decoder.from_gguf(path, n_slots=3)
    om = oracle.OracleModel.from_gguf(path, gguf)
    encs = [synth.encoder_frames(u, 20, 128) for u in range(3)]
    bb = np.array([0.0, 2.0, 4.0], np.float32)
    res = dev.decode(encs, trace=True, blank_bias=bb)
    blanks = []
    for u in range(3):
        st = om.new_state()
        check_window(om, dev, u, encs[u], res[u], st, 10, blank_bias=float(bb[u]))
        blanks.append(int((res[u]["trace"][:, 0] == 61).sum()))
    assert blanks[0] <= blanks[1] <= blanks[2]


def test_deterministic(tmp_path):
    from parakeet_amd import synth
    path = str(tmp_path / "m.gguf")
    small_tdt(path)
    from parakeet_amd import pk
    dev = pk.Decoder.from_gguf(path, n_slots=6)
    encs = [synth.encoder_frames(u, 40, 128) for u in range(6)]
    a = dev.decode(encs, trace=True)
    for u in range(6):
        dev.reset_state(u)          # slots carry state: start the second run fresh too
    b = dev.decode(encs, trace=True)
    for x, y in zip(a, b):
        assert np.array_equal(x["trace"], y["trace"])
        assert np.array_equal(x["tokens"], y["tokens"])


def test_concurrent_decoders(tmp_path):
    """Two decoders, each on its own stream, driven from two threads at once:
    the loop launches are ordered on the device (a loop needs every CU), and
    each thread gets the results of a sequential run."""
    import threading
    from parakeet_amd import pk, synth
    small_tdt(str(tmp_path / "t.gguf"))
    small_eou(str(tmp_path / "e.gguf"))
    dt = pk.Decoder.from_gguf(str(tmp_path / "t.gguf"), n_slots=4)
    de = pk.Decoder.from_gguf(str(tmp_path / "e.gguf"), n_slots=4)
    et = [synth.encoder_frames(900 + u, 30, 128) for u in range(4)]
    ee = [synth.encoder_frames(950 + u, 30, 64) for u in range(4)]

    def run(dec, encs, out, rounds, start=None):
        if start is not None:
            start.wait()
        for _ in range(rounds):
            for u in range(len(encs)):
                dec.reset_state(u)
            out.append([r["tokens"].tolist() for r in dec.decode(encs)])

    want_t, want_e = [], []
    run(dt, et, want_t, 1)
    run(de, ee, want_e, 1)
    got_t, got_e = [], []
    start = threading.Barrier(2)
    th = [threading.Thread(target=run, args=(dt, et, got_t, 6, start)),
          threading.Thread(target=run, args=(de, ee, got_e, 6, start))]
    for t in th:
        t.start()
    for t in th:
        t.join(60)
    assert len(got_t) == 6 and len(got_e) == 6
    assert all(g == want_t[0] for g in got_t)
    assert all(g == want_e[0] for g in got_e)


def test_error_codes(tmp_path):
    from parakeet_amd import pk, synth
    path = str(tmp_path / "m.gguf")
    small_tdt(path)
    dev = pk.Decoder.from_gguf(path, n_slots=2)
    with pytest.raises(pk.PkError) as e:
        dev.decode([synth.encoder_frames(0, 5, 100)])
    assert e.value.rc == 1                        # encoder dim mismatch (reference rc 1)
    with pytest.raises(pk.PkError) as e:
        dev.decode([synth.encoder_frames(0, 40, 128)], token_cap=2)
    assert e.value.rc == 11
    with pytest.raises(pk.PkError) as e:
        dev.decode([synth.encoder_frames(0, 5, 128)] * 2, slots=[1, 1])
    assert e.value.rc == 3


@pytest.mark.parametrize("kind", ["tdt", "eou"])
def test_device_memory_batch_matches_host(tmp_path, kind):
    """Encoder frames already resident in HBM (PK_MEM_DEVICE): a ragged batch
    whose utterances sit at scattered row offsets of one device array, outputs
    written to device arrays, gives the host-memory batch's results."""
    from parakeet_amd import hipmem, pk, synth
    path = str(tmp_path / "m.gguf")
    (small_tdt if kind == "tdt" else small_eou)(path)
    dec = pk.Decoder.from_gguf(path, n_slots=12)
    D = dec.info.D
    Ts = [17, 0, 33, 5, 24] if kind == "eou" else [17, 1, 33, 5, 24]
    encs = [synth.encoder_frames(500 + u, T, D) for u, T in enumerate(Ts)]
    # rows: utterance u at offset rows[u], with unused rows between utterances
    rows = np.zeros(len(Ts), np.int64)
    at = 3
    for u, T in enumerate(Ts):
        rows[u] = at
        at += T + 2
    frames = np.full((at, D), np.nan, np.float32)     # gaps hold NaN: never read
    for u, T in enumerate(Ts):
        frames[rows[u]:rows[u] + T] = encs[u]
    bias = np.array([0.0, 2.0, 0.0, 4.0, 1.0], np.float32)
    ms = dec.info.max_symbols
    want = dec.decode(encs, slots=list(range(5)), blank_bias=bias)
    n = len(Ts)
    cap = max(Ts) * max(1, ms) + 1
    enc_d = hipmem.DeviceArray.from_numpy(frames)
    out = dict(tokens=hipmem.DeviceArray(4 * n * cap), n_tokens=hipmem.DeviceArray(4 * n),
               steps=hipmem.DeviceArray(4 * n), segments=hipmem.DeviceArray(4 * n * cap),
               n_segments=hipmem.DeviceArray(4 * n))
    ptrs = {k: v.ptr for k, v in out.items()}
    ptrs["seg_cap"] = cap
    dec.decode_device(enc_d.ptr, rows, Ts, np.arange(5, 10, dtype=np.int32), ms, ptrs, cap, blank_bias=bias)
    hipmem.synchronize()
    toks = out["tokens"].to_numpy(np.int32, n * cap).reshape(n, cap)
    ntok = out["n_tokens"].to_numpy(np.int32, n)
    steps = out["steps"].to_numpy(np.int32, n)
    segs = out["segments"].to_numpy(np.int32, n * cap).reshape(n, cap)
    nseg = out["n_segments"].to_numpy(np.int32, n)
    for u in range(n):
        assert toks[u, :ntok[u]].tolist() == want[u]["tokens"].tolist(), u
        assert steps[u] == want[u]["steps"], u
        if kind == "eou":
            assert segs[u, :nseg[u]].tolist() == want[u]["segments"].tolist(), u


def test_host_memory_scattered_rows(tmp_path):
    """Host buffers whose utterances are not packed in order (gaps, reversed
    order, a zero-frame EOU window): the uploads follow runs of consecutive
    rows and the results equal the packed batch's."""
    import ctypes as C
    from parakeet_amd import pk, synth
    path = str(tmp_path / "e.gguf")
    small_eou(path)
    dec = pk.Decoder.from_gguf(path, n_slots=12)
    D = dec.info.D
    Ts = [7, 0, 12, 3, 9, 4]
    encs = [synth.encoder_frames(600 + u, T, D) for u, T in enumerate(Ts)]
    want = dec.decode(encs, slots=list(range(6)), max_symbols=5)
    # rows: utterances 0 and 1 back to back, 2 after a gap, 3..5 in reverse order
    order_rows = {0: 0, 1: 7, 2: 10, 5: 30, 4: 34, 3: 43}
    frames = np.full((50, D), np.nan, np.float32)
    for u, r in order_rows.items():
        frames[r:r + Ts[u]] = encs[u]
    rows = np.array([order_rows[u] for u in range(6)], np.int64)
    T = np.array(Ts, np.int32)
    slots = np.arange(6, 12, dtype=np.int32)
    cap = max(Ts) * 5 + 1
    toks = np.zeros((6, cap), np.int32)
    ntok, steps, nseg = np.zeros(6, np.int32), np.zeros(6, np.int32), np.zeros(6, np.int32)
    segs = np.zeros((6, cap + 1), np.int32)
    b = pk.PkBatch()
    b.n_utts, b.mem, b.d_enc, b.max_symbols = 6, pk.MEM_HOST, D, 5
    b.enc, b.enc_row, b.n_frames, b.slot = pk._ptr(frames), pk._ptr(rows), pk._ptr(T), pk._ptr(slots)
    b.tokens, b.token_cap, b.n_tokens, b.steps = pk._ptr(toks), cap, pk._ptr(ntok), pk._ptr(steps)
    b.segments, b.seg_cap, b.n_segments = pk._ptr(segs), cap + 1, pk._ptr(nseg)
    pk.check(pk.lib().pk_decode(dec.h, C.byref(b)))
    for u in range(6):
        assert toks[u, :ntok[u]].tolist() == want[u]["tokens"].tolist(), u
        assert steps[u] == want[u]["steps"], u
        assert segs[u, :nseg[u]].tolist() == want[u]["segments"].tolist(), u


def test_device_frames_host_outputs(tmp_path):
    """PK_MEM_DEVICE_FRAMES (an encoder output left in HBM, outputs to host
    arrays): scattered device rows, reversed order and an empty TDT window
    (which returns before initialising, src/parakeet_tdt.cpp:879, so its
    outputs are zero) give the host-memory batch's results; a frame pointer
    that is not 16-byte aligned is refused before any launch."""
    import ctypes as C
    from parakeet_amd import hipmem, pk, synth
    path = str(tmp_path / "t.gguf")
    small_tdt(path)
    dec = pk.Decoder.from_gguf(path, n_slots=12)
    D = dec.info.D
    Ts = [9, 0, 14, 6]
    encs = [synth.encoder_frames(650 + u, T, D) for u, T in enumerate(Ts)]
    want = dec.decode(encs, slots=list(range(4)))
    order_rows = {0: 20, 1: 0, 2: 2, 3: 31}
    frames = np.full((40, D), np.nan, np.float32)     # rows between windows are never read
    for u, r in order_rows.items():
        frames[r:r + Ts[u]] = encs[u]
    enc_d = hipmem.DeviceArray.from_numpy(frames)
    rows = np.array([order_rows[u] for u in range(4)], np.int64)
    T = np.array(Ts, np.int32)
    slots = np.arange(4, 8, dtype=np.int32)
    cap = max(Ts) * dec.info.max_symbols + 1
    toks = np.zeros((4, cap), np.int32)
    ntok, steps = np.full(4, -1, np.int32), np.full(4, -1, np.int32)
    b = pk.PkBatch()
    b.n_utts, b.mem, b.d_enc, b.max_symbols = 4, pk.MEM_DEVICE_FRAMES, D, dec.info.max_symbols
    b.enc, b.enc_row, b.n_frames, b.slot = C.c_void_p(enc_d.ptr), pk._ptr(rows), pk._ptr(T), pk._ptr(slots)
    b.tokens, b.token_cap, b.n_tokens, b.steps = pk._ptr(toks), cap, pk._ptr(ntok), pk._ptr(steps)
    pk.check(pk.lib().pk_decode(dec.h, C.byref(b)))
    for u in range(4):
        assert toks[u, :ntok[u]].tolist() == want[u]["tokens"].tolist(), u
        assert steps[u] == want[u]["steps"], u
    assert ntok[1] == 0 and steps[1] == 0
    b.enc = C.c_void_p(enc_d.ptr + 4)
    b.slot = pk._ptr(np.arange(8, 12, dtype=np.int32))
    assert pk.lib().pk_decode(dec.h, C.byref(b)) == 3      # PK_ERR_ARG
    assert "aligned" in pk.lib().pk_last_error().decode()


@pytest.mark.parametrize("kind", ["tdt", "eou"])
def test_python_decode_device_frames(tmp_path, kind):
    """Decoder.decode_device_frames (the Python form of the device handoff):
    ragged windows of one device array, decoded in place, equal decode() of
    the same frames from host memory, traces and EOU segments included."""
    from parakeet_amd import hipmem, pk, synth
    path = str(tmp_path / "m.gguf")
    (small_tdt if kind == "tdt" else small_eou)(path)
    dec = pk.Decoder.from_gguf(path, n_slots=10)
    D = dec.info.D
    Ts = [11, 4, 0, 16] if kind == "eou" else [11, 4, 1, 16]
    encs = [synth.encoder_frames(680 + u, T, D) for u, T in enumerate(Ts)]
    want = dec.decode(encs, slots=[0, 1, 2, 3], trace=True)
    rows = np.array([40, 0, 20, 22], np.int64)
    frames = np.full((60, D), np.nan, np.float32)
    for u, T in enumerate(Ts):
        frames[rows[u]:rows[u] + T] = encs[u]
    enc_d = hipmem.DeviceArray.from_numpy(frames)
    hipmem.synchronize()
    got = dec.decode_device_frames(enc_d.ptr, rows, Ts, slots=[4, 5, 6, 7], trace=True)
    for u in range(len(Ts)):
        assert got[u]["tokens"].tolist() == want[u]["tokens"].tolist(), u
        assert got[u]["steps"] == want[u]["steps"], u
        assert np.array_equal(got[u]["trace"], want[u]["trace"]), u
        assert got[u]["segments"].tolist() == want[u]["segments"].tolist(), u


def test_timing_events_optional(tmp_path):
    """pk_decoder_set_timing(0): calls record no timing events, pk_last_timing
    gives -1 for the kernel times and still the lockstep iterations, and the
    decode is the same bit for bit; turned on again, the times come back."""
    from parakeet_amd import pk, synth
    path = str(tmp_path / "t.gguf")
    small_tdt(path)
    dev = pk.Decoder.from_gguf(path, n_slots=8)
    encs = [synth.encoder_frames(600 + u, 30 + 7 * u, 128) for u in range(3)]
    a = dev.decode(encs, slots=[0, 1, 2], trace=True)
    ta = dev.last_timing()
    assert ta["loop_ms"] > 0 and ta["enc_proj_ms"] > 0 and ta["iterations"] > 0
    dev.set_timing(False)
    b = dev.decode(encs, slots=[3, 4, 5], trace=True)
    tb = dev.last_timing()
    assert tb["loop_ms"] == -1 and tb["enc_proj_ms"] == -1 and tb["iterations"] == ta["iterations"]
    for u in range(3):
        assert np.array_equal(a[u]["trace"], b[u]["trace"]), u
    dev.set_timing(True)
    dev.decode(encs, slots=[6, 7, 0], reset=np.ones(3, np.uint8))
    assert dev.last_timing()["loop_ms"] > 0
