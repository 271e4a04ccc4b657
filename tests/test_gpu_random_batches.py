"""Randomised call sequences: batches of 1 .. 512 utterances on scattered
slots, ragged windows, per-utterance blank offsets, a symbol cap drawn per
call, some slots reset and the rest carrying their state from earlier calls
(TDT symbols and carry_frames; EOU last token and segment start, with the
segment indices counted from each session's running token total), and a tenth
of the windows empty (a TDT window of 0 frames returns before initialising,
src/parakeet_tdt.cpp:879, and leaves its slot as it was; an EOU one
initialises, src/parakeet_eou.cpp:246).  Every
window of every call is replayed through the oracle carrying the same state
per slot (teacher-forced, zero unexplained mismatches, final state within
1e-3), so batch composition, domain planning (one domain at B <= 16, 16 or 32
utterances per domain above) and state carry across calls are covered
together.  The reference decodes each window alone (src/parakeet_tdt.cpp:865-981,
src/parakeet_eou.cpp:232-336); the device must give the same per-utterance
result whatever else shares the launch."""
import numpy as np
import pytest

from conftest import small_eou, small_tdt
from parity import check_window

pytestmark = pytest.mark.gpu

N_SLOTS = 600
CALLS = 9


@pytest.mark.parametrize("kind", ["tdt", "eou"])
def test_random_call_sequence(tmp_path, kind):
    from parakeet_amd import gguf, pk, synth
    import oracle
    tdt = kind == "tdt"
    path = str(tmp_path / f"{kind}.gguf")
    (small_tdt if tdt else small_eou)(path)
    D = 128 if tdt else 64
    dev = pk.Decoder.from_gguf(path, n_slots=N_SLOTS)
    om = oracle.OracleModel.from_gguf(path, gguf)
    rng = np.random.default_rng(31 if tdt else 32)
    ost, tbase = {}, {}
    # batch sizes: both ends, the domain-plan boundaries, and random ones
    sizes = [1, 512, 17, 257, 16] + [int(v) for v in np.exp(rng.uniform(0, np.log(512), CALLS - 5)).round()]
    seed = 5000
    for call, B in enumerate(sizes):
        slots = rng.choice(N_SLOTS, size=B, replace=False).astype(np.int32)
        sl = slots.tolist()
        T = rng.integers(1, 41, size=B).astype(np.int32)
        T[rng.random(B) < 0.1] = 0   # empty windows: TDT returns before initialising, EOU initialises
        bias = rng.choice(np.array([0.0, 2.0, 4.0] if tdt else [0.0, 2.0], np.float32), size=B)
        ms = int(rng.choice([1, 2, 10] if tdt else [1, 3, 5]))
        reset = np.array([(s not in ost) or rng.random() < 0.2 for s in sl], np.uint8)
        for s, r, t in zip(sl, reset, T.tolist()):
            # an empty TDT window leaves its slot as it was, a requested reset included
            if (r and (not tdt or t > 0)) or s not in ost:
                ost[s] = om.new_state()
                tbase[s] = 0
        base = np.array([tbase[s] for s in sl], np.int32)
        encs = [synth.encoder_frames(seed + u, int(T[u]), D) for u in range(B)]
        seed += B
        print(f"{kind} call {call}: B={B}, T {T.min()}..{T.max()}, max_symbols {ms}, "
              f"{int(reset.sum())} reset", flush=True)
        res = dev.decode(encs, slots=slots, trace=True, max_symbols=ms, blank_bias=bias, tokens_base=base,
                         reset=reset)
        for u in range(B):
            s = sl[u]
            if tdt and T[u] == 0:
                assert res[u]["steps"] == 0 and len(res[u]["tokens"]) == 0, (call, u)
                continue
            check_window(om, dev, s, encs[u], res[u], ost[s], ms, blank_bias=float(bias[u]),
                         tokens_before=int(base[u]))
            tbase[s] += len(res[u]["tokens"])
    dev.close()
