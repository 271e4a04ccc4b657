"""A handle with more state slots than 32-bit byte offsets reach: 110,000 slots
of the TDT-0.6b-v3 decoder put the recurrent-product slot array (2 layers x
2560 floats per slot) past 2 GiB.  A window decoded on the last slot equals
the same window on slot 0 bit for bit (tokens, steps, state) and replays
through the oracle; copying the last slot to another slot and back keeps the
state.  The reference keeps one state per caller object (src/parakeet_tdt.h:170-183);
here each of the streaming sessions a GPU serves holds a slot."""
import numpy as np
import pytest

from parity import check_window

pytestmark = pytest.mark.gpu

N_SLOTS = 110_000


def test_last_of_110k_slots(tmp_path):
    from parakeet_amd import gguf, pk, synth
    import oracle
    path = str(tmp_path / "tdt06.gguf")
    synth.make_shape(path, "tdt-0.6b-v3")
    dev = pk.Decoder.from_gguf(path, n_slots=N_SLOTS)
    om = oracle.OracleModel.from_gguf(path, gguf)
    assert N_SLOTS * 2 * 4 * 640 * 4 > 2 ** 31
    last = N_SLOTS - 1
    encs = [synth.encoder_frames(77, 30, 1024), synth.encoder_frames(78, 30, 1024)]
    print(f"TDT-0.6b, {N_SLOTS} slots: slots 0 and {last}", flush=True)
    a = dev.decode(encs, slots=[0, last], trace=True)
    b = dev.decode(encs[::-1], slots=[1, 2], trace=True)
    st = om.new_state()
    check_window(om, dev, last, encs[1], a[1], st, 10)
    assert np.array_equal(a[1]["trace"], b[0]["trace"]) and a[1]["steps"] == b[0]["steps"]
    s_last, s_one = dev.read_state(last), dev.read_state(1)
    assert np.array_equal(s_last["h"], s_one["h"]) and np.array_equal(s_last["c"], s_one["c"])
    # the carried state keeps decoding the same way from the last slot and from a copy of it
    dev.copy_state(last, 3)
    nxt = synth.encoder_frames(79, 20, 1024)
    c1 = dev.decode([nxt], slots=[last], trace=True)[0]
    c2 = dev.decode([nxt], slots=[3], trace=True)[0]
    assert np.array_equal(c1["trace"], c2["trace"])
    check_window(om, dev, last, nxt, c1, st, 10)
    dev.close()
