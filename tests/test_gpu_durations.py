"""TDT duration tables other than {0, 1, 2, 3, 4}, and small symbol caps, on
the device, replayed through the oracle step by step.

The reference reads the number of duration logits (parakeet.tdt.num_durations,
default 5) apart from the value table (parakeet.tdt.durations, default
{0, 1, 2, 3, 4} when the key is absent; src/parakeet_ctc.cpp:428-439), and
takes the duration as the table's value at the argmax index, or the index
itself when the table is empty (src/parakeet_tdt.cpp:938-940).  The replay
applies the oracle's table to each index the device chose, so a device that
advanced by the index, or by another entry, lands on other frames and fails
the step-by-step comparison and the final carry check.  The oracle's table
handling is pinned by closed forms in tests/test_oracle.py."""
import json
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT, small_eou, small_tdt
from parity import check_window

pytestmark = pytest.mark.gpu

TABLES = {
    "0-2-3-5-8": dict(durations=[0, 2, 3, 5, 8]),
    "1-4-7": dict(durations=[1, 4, 7]),
    "empty-5": dict(durations=[], num_durations=5),
    "no-key-5": dict(durations=None, num_durations=5),
    "5-entries-3-logits": dict(durations=[0, 1, 2, 9, 9], num_durations=3),
    "8-durations": dict(durations=[0, 1, 2, 3, 4, 6, 8, 12]),
}


def _models(path, **kw):
    from parakeet_amd import gguf, pk
    import oracle
    small_tdt(path, **kw)
    return pk.Decoder.from_gguf(path, n_slots=8), oracle.OracleModel.from_gguf(path, gguf)


@pytest.mark.parametrize("name", list(TABLES))
def test_duration_tables_replay(tmp_path, name):
    from parakeet_amd import synth
    dev, om = _models(str(tmp_path / "m.gguf"), **TABLES[name])
    assert dev.info.Dn == om.Dn
    Ts = [1, 9, 40, 23, 64]
    encs = [synth.encoder_frames(300 + u, T, 128) for u, T in enumerate(Ts)]
    print(f"durations {name}: Dn={om.Dn} B={len(Ts)} T={Ts}", flush=True)
    res = dev.decode(encs, trace=True, max_symbols=10)
    used = set()
    for u, enc in enumerate(encs):
        check_window(om, dev, u, enc, res[u], om.new_state(), 10)
        used |= set(np.asarray(res[u]["trace"])[:, 1].tolist())
    assert used <= set(range(om.Dn)) and len(used) >= min(3, om.Dn), used
    # two utterances fed in 3-frame windows with the state carried: a carry of
    # up to 2 frames goes into the next window, a longer one ends with the
    # window (the reference's carry = max(0, t - n), src/parakeet_tdt.cpp:905-909, :980)
    slots, us = [5, 6], (2, 4)
    states = [om.new_state() for _ in slots]
    for t0 in range(0, 40, 3):
        ws = [encs[u][t0:t0 + 3] for u in us]
        r = dev.decode(ws, slots=slots, trace=True, max_symbols=10)
        for k in range(len(us)):
            check_window(om, dev, slots[k], ws[k], r[k], states[k], 10)
    dev.close()


@pytest.mark.parametrize("max_symbols", [1, 2])
def test_small_symbol_caps_replay(tmp_path, max_symbols):
    """max_symbols 1 and 2: the cap ends a frame after every one or two
    emissions (src/parakeet_tdt.cpp:958-963)."""
    from parakeet_amd import synth
    dev, om = _models(str(tmp_path / "m.gguf"))
    encs = [synth.encoder_frames(400 + u, T, 128) for u, T in enumerate([5, 31, 60])]
    print(f"max_symbols {max_symbols}: B=3", flush=True)
    res = dev.decode(encs, trace=True, max_symbols=max_symbols)
    for u, enc in enumerate(encs):
        check_window(om, dev, u, enc, res[u], om.new_state(), max_symbols)
    dev.close()


def test_cpp_loader_duration_table(tmp_path):
    """The C++ loader (parakeet.tdt.num_durations and the table as the
    reference reads them) through the reference-shaped API: tdt_greedy_decode,
    tdt_decode_batch and 9-frame tdt_decode_window chunks (longer than the
    table's largest duration, 8) give the C ABI decode, which the replay above
    ties to the oracle."""
    from parakeet_amd import synth
    driver = os.path.join(ROOT, "tests", "cpp", "decoder_api_main")
    tdt_path, eou_path = str(tmp_path / "t.gguf"), str(tmp_path / "e.gguf")
    dev, om = _models(tdt_path, durations=[0, 2, 3, 5, 8])
    small_eou(eou_path)
    T, W = 45, 9
    encs = [synth.encoder_frames(500 + u, T, 128) for u in range(3)]
    encs_e = [synth.encoder_frames(600 + u, T, 64) for u in range(3)]
    for name, e in (("t.bin", encs), ("e.bin", encs_e)):
        with open(tmp_path / name, "wb") as f:
            np.array([len(e), T, e[0].shape[1]], np.int32).tofile(f)
            np.stack(e).astype(np.float32).tofile(f)
    print(f"cpp loader durations: B=3 T={T} window={W}", flush=True)
    r = subprocess.run([driver, tdt_path, str(tmp_path / "t.bin"), eou_path, str(tmp_path / "e.bin"), str(W)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout)
    ref = dev.decode(encs, trace=True)
    for u in range(3):
        check_window(om, dev, u, encs[u], ref[u], om.new_state(), 10)
        want = ref[u]["tokens"].tolist()
        assert out["tdt"]["greedy"][u] == want, u
        assert out["tdt"]["batch"][u] == want, u
        assert out["tdt"]["chunked"][u] == want, u
        assert out["tdt"]["steps"][u] == ref[u]["steps"], u
    dev.close()
