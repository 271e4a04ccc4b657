"""The decode loop's launch: an ordinary dispatch whose workgroups first check
that the whole grid is resident, relaunched cooperatively when it is not.  The
barriers of the loop (the reference's per-step chain, src/parakeet_tdt.cpp:917-967,
run here by every workgroup in lockstep) need every workgroup resident; the
check turns a grid that is not into a clean relaunch instead of a 2 s barrier
time-out.  The relaunch path is forced from the host with an arrival limit of
one clock tick (PK_ARRIVE_US=0), so every kernel still exits normally, and the
results must equal the default launch bit for bit."""
import os

import numpy as np
import pytest

from conftest import small_eou, small_tdt

pytestmark = pytest.mark.gpu

NOTE = "decode loop grid not co-resident: relaunched cooperatively"


def _decode(dev, encs, slot0, **kw):
    return dev.decode(encs, slots=list(range(slot0, slot0 + len(encs))), trace=True, **kw)


def _same(dev, a, b, base_a, base_b):
    for u in range(len(a)):
        assert np.array_equal(a[u]["trace"], b[u]["trace"]), u
        assert a[u]["tokens"].tolist() == b[u]["tokens"].tolist(), u
        assert a[u]["segments"].tolist() == b[u]["segments"].tolist(), u
        x, y = dev.read_state(base_a + u), dev.read_state(base_b + u)
        assert np.array_equal(x["h"], y["h"]) and np.array_equal(x["c"], y["c"]), u
        assert x["ctrl"].tolist() == y["ctrl"].tolist(), u


@pytest.mark.parametrize("kind,B", [("tdt", 2), ("tdt", 40), ("eou", 24)])
def test_not_coresident_grid_is_relaunched(tmp_path, capfd, kind, B):
    from parakeet_amd import pk, synth
    path = str(tmp_path / "m.gguf")
    (small_tdt if kind == "tdt" else small_eou)(path)
    dev = pk.Decoder.from_gguf(path, n_slots=2 * B)
    rng = np.random.default_rng(40 + B)
    Ts = rng.integers(5, 60, size=B)
    encs = [synth.encoder_frames(500 + u, int(T), dev.info.D) for u, T in enumerate(Ts)]
    print(f"co-residency relaunch: {kind} B={B}", flush=True)
    want = _decode(dev, encs, 0)
    os.environ["PK_ARRIVE_US"] = "0"
    try:
        capfd.readouterr()
        got = _decode(dev, encs, B)
        err = capfd.readouterr().err
    finally:
        os.environ.pop("PK_ARRIVE_US")
    assert NOTE in err, err[-500:]
    _same(dev, want, got, 0, B)
    # the limit was a test setting: later launches are ordinary dispatches again (no relaunch),
    # with the same results (slots reset in the launch)
    again = _decode(dev, encs, 0, reset=np.ones(B, np.uint8))
    assert NOTE not in capfd.readouterr().err
    _same(dev, want, again, B, 0)
