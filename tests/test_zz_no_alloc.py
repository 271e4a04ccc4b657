"""pk_decode_noalloc (no device allocation: every call buffer comes from the
fixed per-device scratch array) against pk_decode on the same device-resident
inputs: identical decisions, tokens, step counts and slot state, on two calls
in a row -- the second smaller, so it runs on what the first left in the
array -- and a clear refusal of a batch larger than the array."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _device_call(dec, hipmem, frames_d, rows, Ts, slots, noalloc):
    n = len(Ts)
    ms = dec.info.max_symbols
    cap = int(max(Ts)) * ms + 1
    tcap = int(max(Ts)) * (ms + 1) + 1
    out = dict(tokens=hipmem.DeviceArray(4 * n * cap), n_tokens=hipmem.DeviceArray(4 * n),
               steps=hipmem.DeviceArray(4 * n))
    tr = hipmem.DeviceArray(8 * n * tcap)
    ptrs = {k: v.ptr for k, v in out.items()}
    ptrs["trace"] = tr.ptr
    dec.decode_device(frames_d.ptr, rows, Ts, slots, ms, ptrs, cap, trace_cap=tcap, noalloc=noalloc)
    hipmem.synchronize()
    ntok = out["n_tokens"].to_numpy(np.int32, n)
    steps = out["steps"].to_numpy(np.int32, n)
    toks = out["tokens"].to_numpy(np.int32, n * cap).reshape(n, cap)
    trace = tr.to_numpy(np.int32, n * tcap * 2).reshape(n, tcap, 2)
    res = [dict(tokens=toks[u, :ntok[u]].copy(), steps=int(steps[u]), trace=trace[u, :steps[u]].copy())
           for u in range(n)]
    for a in (*out.values(), tr):
        a.free()
    return res


def test_noalloc_matches_pk_decode_two_calls(tmp_path):
    from parakeet_amd import hipmem, pk, synth
    path = str(tmp_path / "tdt06.gguf")
    synth.make_shape(path, "tdt-0.6b-v3")
    dec = pk.Decoder.from_gguf(path, n_slots=64)
    D = dec.info.D
    for call, (B, T) in enumerate(((16, 120), (5, 37))):          # the second call is smaller
        Ts = np.full(B, T, np.int32)
        Ts[::3] = max(1, T // 2)                                  # ragged lengths
        rows = np.concatenate([[0], np.cumsum(Ts)[:-1]]).astype(np.int64)
        frames = np.concatenate([synth.encoder_frames(40 * call + u, int(Ts[u]), D) for u in range(B)])
        frames_d = hipmem.DeviceArray.from_numpy(frames)
        print(f"[noalloc] call {call}: B={B} T={T}", flush=True)
        want = _device_call(dec, hipmem, frames_d, rows, Ts, np.arange(B, dtype=np.int32), noalloc=False)
        got = _device_call(dec, hipmem, frames_d, rows, Ts, np.arange(32, 32 + B, dtype=np.int32), noalloc=True)
        for u in range(B):
            assert got[u]["tokens"].tolist() == want[u]["tokens"].tolist(), (call, u)
            assert got[u]["steps"] == want[u]["steps"], (call, u)
            assert np.array_equal(got[u]["trace"], want[u]["trace"]), (call, u)
            a, b = dec.read_state(u), dec.read_state(32 + u)
            assert np.array_equal(a["h"], b["h"]) and np.array_equal(a["c"], b["c"]), (call, u)
            assert a["ctrl"].tolist() == b["ctrl"].tolist(), (call, u)
        frames_d.free()
    dec.close()


def test_noalloc_refuses_oversized_and_host_batches(tmp_path):
    """64 x 750 frames need about 123 MB of enc_proj rows: more than the
    32 MiB array, refused before any launch (PK_ERR_UNSUPPORTED); host-memory
    batches are refused too (PK_ERR_ARG)."""
    from parakeet_amd import hipmem, pk, synth
    path = str(tmp_path / "tdt06.gguf")
    synth.make_shape(path, "tdt-0.6b-v3")
    dec = pk.Decoder.from_gguf(path, n_slots=64)
    B, T = 64, 750
    frames_d = hipmem.DeviceArray(B * T * dec.info.D * 4)
    frames_d.zero()
    out = dict(tokens=hipmem.DeviceArray(4 * B * 16), n_tokens=hipmem.DeviceArray(4 * B),
               steps=hipmem.DeviceArray(4 * B))
    rows = np.arange(B, dtype=np.int64) * T
    with pytest.raises(pk.PkError) as e:
        dec.decode_device(frames_d.ptr, rows, np.full(B, T, np.int32), np.arange(B, dtype=np.int32), 10,
                          {k: v.ptr for k, v in out.items()}, 16, noalloc=True)
    assert e.value.rc == 5 and "fixed scratch" in str(e.value)
    # pk_decode_noalloc refuses a host-memory batch outright
    import ctypes as C
    b = pk.PkBatch()
    b.n_utts, b.mem, b.d_enc, b.max_symbols = 1, pk.MEM_HOST, dec.info.D, 10
    assert pk.lib().pk_decode_noalloc(dec.h, C.byref(b)) == 3
    for a in (frames_d, *out.values()):
        a.free()
    dec.close()
