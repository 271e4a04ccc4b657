"""The benchmark configurations on the device, checked against the oracle.

Full-size runs are checked with size-independent properties (batch
invariance: an utterance decoded inside a lockstep batch gives exactly what
it gives alone; determinism) plus teacher-forced oracle replay of a sample of
utterances; reduced-size runs replay every utterance.  Oracle replays run on a
thread pool (the oracle is re-entrant and ctypes releases the GIL)."""
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from parity import TIE_EPS, rel

pytestmark = pytest.mark.gpu

THREADS = max(1, min(16, os.cpu_count() or 1))


def _replay_all(om, encs, res, max_symbols, blank_bias=None):
    def one(u):
        st = om.new_state()
        bb = 0.0 if blank_bias is None else float(blank_bias[u])
        rep = om.replay_window(encs[u], st, max_symbols, res[u]["trace"], blank_bias=bb, tie_eps=TIE_EPS)
        return u, rep, st
    with ThreadPoolExecutor(THREADS) as ex:
        return list(ex.map(one, range(len(encs))))


def _assert_replays(dev, replays, res, slots=None):
    near = 0
    worst_h = 0.0
    for u, rep, st in replays:
        s = rep["stats"]
        assert rep["rc"] == 0 and s["structure_error"] == 0, (u, s)
        assert s["unexplained"] == 0, (u, s)
        assert rep["tokens"].tolist() == res[u]["tokens"].tolist(), u
        near += s["near_ties"]
        d = dev.read_state(u if slots is None else slots[u])
        worst_h = max(worst_h, rel(d["h"], st.h), rel(d["c"], st.c))
    assert worst_h < 1e-3, worst_h
    return near, worst_h


@pytest.fixture(scope="module")
def tdt06(tmp_path_factory):
    from parakeet_amd import gguf, synth
    import oracle
    path = str(tmp_path_factory.mktemp("m") / "tdt06.gguf")
    synth.make_shape(path, "tdt-0.6b-v3")
    return path, oracle.OracleModel.from_gguf(path, gguf)


def test_cfg2_reduced_b64(tdt06):
    """TDT-0.6b q8_0, B=64 lockstep, T=60 frames each (every utterance replayed)."""
    from parakeet_amd import pk, synth
    path, om = tdt06
    dev = pk.Decoder.from_gguf(path, n_slots=64)
    encs = [synth.encoder_frames(u, 60, 1024) for u in range(64)]
    res = dev.decode(encs, trace=True)
    near, worst = _assert_replays(dev, _replay_all(om, encs, res, 10), res)
    print(f"cfg2-reduced: steps={sum(r['steps'] for r in res)} near_ties={near} worst_state_rel={worst:.2e}")
    dev.close()


def test_cfg2_full_batch_invariance(tdt06):
    """B=64, T=750: each utterance in the batch == the same utterance alone
    (bitwise); a sample of 4 utterances replayed through the oracle."""
    from parakeet_amd import pk, synth
    path, om = tdt06
    dev = pk.Decoder.from_gguf(path, n_slots=80)
    encs = [synth.encoder_frames(u, 750, 1024) for u in range(64)]
    res = dev.decode(encs, trace=True)
    for k, u in enumerate((0, 17, 42, 63)):
        alone = dev.decode([encs[u]], slots=[64 + k], trace=True)[0]
        assert np.array_equal(alone["trace"], res[u]["trace"]), u
    sample = [0, 17, 42, 63]
    reps = _replay_all(om, [encs[u] for u in sample], [res[u] for u in sample], 10)
    reps = [(sample[i], rep, st) for i, rep, st in reps]
    near, _ = _assert_replays(dev, reps, res)
    print(f"cfg2-full: steps={sum(r['steps'] for r in res)} sample near_ties={near}")
    dev.close()


def test_cfg3_tdt11b_f16(tmp_path):
    """TDT-1.1b shapes, f16 weights, B=256 lockstep, T=24 frames (all replayed)."""
    from parakeet_amd import gguf, pk, synth
    import oracle
    path = str(tmp_path / "tdt11.gguf")
    synth.make_shape(path, "tdt-1.1b")
    dev = pk.Decoder.from_gguf(path, n_slots=256)
    om = oracle.OracleModel.from_gguf(path, gguf)
    encs = [synth.encoder_frames(u, 24, 1024) for u in range(256)]
    res = dev.decode(encs, trace=True)
    near, worst = _assert_replays(dev, _replay_all(om, encs, res, 10), res)
    print(f"cfg3: steps={sum(r['steps'] for r in res)} near_ties={near} worst_state_rel={worst:.2e}")
    dev.close()


def test_cfg4_eou_streaming_sessions(tmp_path):
    """EOU-120m shapes, q8_0, B=128 sessions fed 2-frame chunks (all 40 chunks
    of the workload), state carried; every window replayed on the oracle
    carrying its own state."""
    from parakeet_amd import gguf, pk, synth
    import oracle
    path = str(tmp_path / "eou.gguf")
    synth.make_shape(path, "eou-120m")
    dev = pk.Decoder.from_gguf(path, n_slots=128)
    om = oracle.OracleModel.from_gguf(path, gguf)
    B, C = 128, 40
    encs = [synth.encoder_frames(u, 2 * C, 512) for u in range(B)]
    for u in range(B):
        dev.init_state(u)
    ost = []
    for _ in range(B):
        s = om.new_state()
        om.init_state(s)
        ost.append(s)
    total = np.zeros(B, np.int32)
    near = 0
    for c in range(C):
        ws = [e[2 * c:2 * c + 2] for e in encs]
        res = dev.decode(ws, trace=True, tokens_base=total, max_symbols=5)

        def one(u):
            rep = om.replay_window(ws[u], ost[u], 5, res[u]["trace"], tie_eps=TIE_EPS,
                                   tokens_before=int(total[u]))
            return u, rep
        with ThreadPoolExecutor(THREADS) as ex:
            reps = list(ex.map(one, range(B)))
        for u, rep in reps:
            s = rep["stats"]
            assert s["unexplained"] == 0 and s["structure_error"] == 0, (c, u, s)
            assert rep["tokens"].tolist() == res[u]["tokens"].tolist()
            assert rep["segments"].tolist() == res[u]["segments"].tolist()
            near += s["near_ties"]
        total += np.array([len(r["tokens"]) for r in res], np.int32)
    for u in (0, 77, 127):
        d = dev.read_state(u)
        assert rel(d["h"], ost[u].h) < 1e-3 and rel(d["c"], ost[u].c) < 1e-3
        assert d["ctrl"][3] == ost[u].st.last_token
    print(f"cfg4: tokens={int(total.sum())} near_ties={near}")
    dev.close()


def test_cfg5_ragged_blank_bias(tdt06):
    """B=512, T ~ U{50..1500}, blank offsets {0,+2,+4}: batch invariance for a
    sample (bitwise), oracle replay of the six shortest utterances and of one
    utterance of at least 1,000 frames per blank offset."""
    from parakeet_amd import pk, synth
    path, om = tdt06
    B = 512
    Ts = synth.ragged_lengths(B)
    bb = synth.blank_offsets(B)
    dev = pk.Decoder.from_gguf(path, n_slots=B + 8)
    encs = [synth.encoder_frames(u, int(Ts[u]), 1024) for u in range(B)]
    res = dev.decode(encs, trace=True, blank_bias=bb)
    order = np.argsort(Ts)
    sample = [int(order[0]), int(order[1]), int(order[B // 2]), int(order[-1])]
    for k, u in enumerate(sample):
        alone = dev.decode([encs[u]], slots=[B + k], trace=True, blank_bias=bb[u:u + 1])[0]
        assert np.array_equal(alone["trace"], res[u]["trace"]), u
    # replayed: the 6 shortest utterances, and one utterance of at least 1,000 frames per
    # blank offset (long blank-biased utterances chain runs of blanks over spare columns)
    short = [int(u) for u in order[:6]]
    longs = [int(next(u for u in order[::-1] if Ts[u] >= 1000 and bb[u] == b)) for b in (0.0, 2.0, 4.0)]
    picked = short + longs
    reps = _replay_all(om, [encs[u] for u in picked], [res[u] for u in picked], 10,
                       blank_bias=[bb[u] for u in picked])
    reps = [(picked[i], rep, st) for i, rep, st in reps]
    _assert_replays(dev, reps, res)
    print(f"cfg5: replayed long utterances {[(u, int(Ts[u]), float(bb[u])) for u in longs]}", flush=True)
    dens = [np.mean(res[u]["trace"][:, 0] == 8192) for u in range(B)]
    by_bias = {b: float(np.mean([d for d, x in zip(dens, bb) if x == b])) for b in (0.0, 2.0, 4.0)}
    assert by_bias[0.0] <= by_bias[2.0] <= by_bias[4.0], by_bias
    print(f"cfg5: steps={sum(r['steps'] for r in res)} blank fraction by bias {by_bias}")
    dev.close()


def test_eou_b200_sixteen_utterance_domains(tmp_path):
    """EOU-120m shapes, q8_0, 200 sessions in one call: the batch runs as
    sixteen-utterance domains of 16 workgroups (the plan for 129..256
    utterances).  A sample decoded alone gives the same decisions bit for bit,
    and the sample replays through the oracle."""
    from parakeet_amd import gguf, pk, synth
    import oracle
    path = str(tmp_path / "eou.gguf")
    synth.make_shape(path, "eou-120m")
    B, T = 200, 6
    dev = pk.Decoder.from_gguf(path, n_slots=B + 4)
    om = oracle.OracleModel.from_gguf(path, gguf)
    encs = [synth.encoder_frames(900 + u, T, 512) for u in range(B)]
    res = dev.decode(encs, trace=True, max_symbols=5)
    sample = [0, 77, 150, 199]
    for k, u in enumerate(sample):
        alone = dev.decode([encs[u]], slots=[B + k], trace=True, max_symbols=5)[0]
        assert np.array_equal(alone["trace"], res[u]["trace"]), u
        assert alone["segments"].tolist() == res[u]["segments"].tolist(), u
    reps = _replay_all(om, [encs[u] for u in sample], [res[u] for u in sample], 5)
    reps = [(sample[i], rep, st) for i, rep, st in reps]
    near, worst = _assert_replays(dev, reps, res)
    print(f"eou B=200: steps={sum(r['steps'] for r in res)} sample near_ties={near} worst_state_rel={worst:.2e}")
    dev.close()
