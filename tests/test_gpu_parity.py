"""Device decode vs oracle: tokens/durations per step (teacher-forced replay,
zero unexplained mismatches), final LSTM state within 1e-3, across TDT and
EOU decoders, q8_0 / q5_0 / q4_0 / f16 / f32 weights, batches, streaming windows."""
import os

import numpy as np
import pytest

from conftest import small_eou, small_tdt
from parity import check_window, free_run_equal

pytestmark = pytest.mark.gpu


def _models(path, writer, **kw):
    from parakeet_amd import gguf, pk
    import oracle
    writer(path, **kw)
    return pk.Decoder.from_gguf(path, n_slots=8), oracle.OracleModel.from_gguf(path, gguf)


@pytest.mark.parametrize("quant", ["q8_0", "f16", "f32", "q5_0", "q4_0"])
def test_tdt_small_batch(tmp_path, quant):
    from parakeet_amd import synth
    dev, om = _models(str(tmp_path / "m.gguf"), small_tdt, quant=quant)
    Ts = [1, 7, 40, 3, 25]
    encs = [synth.encoder_frames(u, T, 128) for u, T in enumerate(Ts)]
    res = dev.decode(encs, trace=True, max_symbols=10)
    for u, enc in enumerate(encs):
        st = om.new_state()
        check_window(om, dev, u, enc, res[u], st, 10)
    dev.close()


def test_tdt_free_run_matches(tmp_path):
    from parakeet_amd import synth
    dev, om = _models(str(tmp_path / "m.gguf"), small_tdt)
    encs = [synth.encoder_frames(100 + u, 30, 128) for u in range(4)]
    res = dev.decode(encs, trace=True)
    n_equal = sum(free_run_equal(om, e, r, 10) for e, r in zip(encs, res))
    assert n_equal == len(encs)
    dev.close()


@pytest.mark.parametrize("quant", ["q8_0", "q5_0", "q4_0"])
def test_eou_small_batch(tmp_path, quant):
    from parakeet_amd import synth
    dev, om = _models(str(tmp_path / "e.gguf"), small_eou, quant=quant)
    encs = [synth.encoder_frames(200 + u, T, 64) for u, T in enumerate([5, 17, 2, 30])]
    res = dev.decode(encs, trace=True, max_symbols=5)
    for u, enc in enumerate(encs):
        st = om.new_state()
        check_window(om, dev, u, enc, res[u], st, 5)
    dev.close()


def test_tdt_06b_b1(tmp_path):
    """TDT-0.6b-v3 shapes, q8_0, B=1, T=125 frames."""
    from parakeet_amd import gguf, pk, synth
    import oracle
    path = str(tmp_path / "tdt06.gguf")
    synth.make_shape(path, "tdt-0.6b-v3")
    dev = pk.Decoder.from_gguf(path, n_slots=1)
    om = oracle.OracleModel.from_gguf(path, gguf)
    enc = synth.encoder_frames(0, 125, 1024)
    res = dev.decode([enc], trace=True, max_symbols=10)[0]
    st = om.new_state()
    stats = check_window(om, dev, 0, enc, res, st, 10)
    print("tdt-0.6b B=1:", res["steps"], "steps", stats)
    dev.close()


@pytest.mark.parametrize("quant", ["q5_0", "q4_0"])
def test_tdt_06b_block_quant(tmp_path, quant):
    """TDT-0.6b-v3 shapes with q5_0 / q4_0 matrices (the reference converter's --quant
    choices): B=4 x 60 frames, every utterance replayed through the oracle."""
    from parakeet_amd import gguf, pk, synth
    import oracle
    path = str(tmp_path / f"tdt06-{quant}.gguf")
    synth.make_shape(path, "tdt-0.6b-v3", quant=quant)
    dev = pk.Decoder.from_gguf(path, n_slots=4)
    om = oracle.OracleModel.from_gguf(path, gguf)
    encs = [synth.encoder_frames(300 + u, 60, 1024) for u in range(4)]
    print(f"tdt-0.6b {quant}: B=4 T=60", flush=True)
    res = dev.decode(encs, trace=True, max_symbols=10)
    for u, enc in enumerate(encs):
        check_window(om, dev, u, enc, res[u], om.new_state(), 10)
    dev.close()
