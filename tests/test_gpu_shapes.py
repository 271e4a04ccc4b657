"""Decoder shapes away from the published checkpoints: every dimension the
loader accepts (pred_rnn_layers 1..8, pred_hidden / joint_hidden / d_enc any
multiple of 32, any vocabulary, up to 16 durations) decodes with the oracle's
decisions.  The reference reads these from GGUF metadata
(src/parakeet_ctc.cpp:418-458) and its loops take any of them
(src/parakeet_tdt.cpp:106-142, 865-981; src/parakeet_eou.cpp:78-116, 232-336).

Each shape decodes a batch in one domain (B=5) and in several (B=40), every
utterance replayed through the oracle (teacher-forced, zero unexplained
mismatches, final state within 1e-3), and the batched streams equal the same
utterances decoded one at a time, bit for bit (batch invariance)."""
import numpy as np
import pytest

from parity import check_window

pytestmark = pytest.mark.gpu

# (name, writer arguments).  Chosen to move every layout boundary: one and
# several layers, 16-row tiles of the gate and joint rows that do not fill a
# workgroup's share evenly, output rows that fill whole tiles exactly (vocab 42:
# 43 + 5 = 48 rows) or leave 1 or 15 past the last tile, duration tables of 1 and 16.
SHAPES = [
    ("tdt_L1_h32", dict(kind="tdt", H=32, L=1, J=32, D=32, vocab=15, durations=[0, 1, 2, 3, 4], quant="q8_0")),
    ("tdt_L3_h96", dict(kind="tdt", H=96, L=3, J=160, D=96, vocab=95, durations=[0, 1, 2, 3, 4], quant="q8_0")),
    ("tdt_L4_dur16_f16", dict(kind="tdt", H=64, L=4, J=64, D=64, vocab=90, durations=list(range(16)),
                              quant="f16")),
    ("tdt_whole_tiles", dict(kind="tdt", H=128, L=2, J=96, D=160, vocab=42, durations=[0, 1, 2, 3, 4],
                             quant="q8_0")),
    ("tdt_dur1_tail15", dict(kind="tdt", H=64, L=2, J=64, D=64, vocab=253, durations=[1], quant="q4_0")),
    ("eou_L2", dict(kind="eou", H=64, L=2, J=64, D=96, vocab=43, eou_id=41, eob_id=42, max_symbols=5,
                    quant="q8_0")),
    ("eou_L3_f32", dict(kind="eou", H=32, L=3, J=128, D=32, vocab=30, eou_id=28, eob_id=29, max_symbols=3,
                        quant="f32")),
    ("tdt_L8_h32", dict(kind="tdt", H=32, L=8, J=32, D=64, vocab=20, durations=[0, 1, 2], quant="q5_0")),
    ("tdt_h1024", dict(kind="tdt", H=1024, L=2, J=1024, D=512, vocab=500, durations=[0, 1, 2, 3, 4],
                       quant="q8_0")),
    # near the LDS bound: one activation block of 16 rows x 2048 (hi + lo) takes 128.5 KB
    ("tdt_j2048", dict(kind="tdt", H=64, L=2, J=2048, D=64, vocab=50, durations=[0, 1, 2, 3, 4], quant="q8_0")),
]


@pytest.mark.parametrize("name,cfg", SHAPES, ids=[s[0] for s in SHAPES])
def test_shape_replay_and_batch_invariance(tmp_path, name, cfg):
    from parakeet_amd import gguf, pk, synth
    import oracle
    path = str(tmp_path / f"{name}.gguf")
    synth.make_decoder_gguf(path, **cfg)
    tdt = cfg["kind"] == "tdt"
    ms = 10 if tdt else cfg["max_symbols"]
    D = cfg["D"]
    om = oracle.OracleModel.from_gguf(path, gguf)
    B = 40
    dev = pk.Decoder.from_gguf(path, n_slots=B + 5 + 1)
    Ts = [3 + (7 * u) % 29 for u in range(B)]
    encs = [synth.encoder_frames(4000 + u, T, D) for u, T in enumerate(Ts)]
    print(f"{name}: B=5 and B={B}, T {min(Ts)}..{max(Ts)}", flush=True)
    small = dev.decode(encs[:5], slots=list(range(B, B + 5)), trace=True, max_symbols=ms)
    for u in range(5):
        check_window(om, dev, B + u, encs[u], small[u], om.new_state(), ms)
    big = dev.decode(encs, slots=list(range(B)), trace=True, max_symbols=ms)
    for u in range(B):
        check_window(om, dev, u, encs[u], big[u], om.new_state(), ms)
    # bit-equal to the same utterances alone (one-domain launches, B=1)
    for u in (0, 17, B - 1):
        one = dev.decode([encs[u]], slots=[B + 5], trace=True, max_symbols=ms, reset=[1])[0]
        assert np.array_equal(one["trace"], big[u]["trace"]), (name, u)
        assert np.array_equal(one["tokens"], big[u]["tokens"]), (name, u)
        a, b = dev.read_state(B + 5), dev.read_state(u)
        assert np.array_equal(a["h"], b["h"]) and np.array_equal(a["c"], b["c"]), (name, u)
    for u in range(5):
        assert np.array_equal(small[u]["trace"], big[u]["trace"]), (name, u)
    print(f"  steps {sum(r['steps'] for r in big)}", flush=True)
    dev.close()


def test_hidden_past_the_lds_is_refused(tmp_path):
    """A joint_hidden whose activation block (16 rows x J, f16 hi + lo) does not fit
    the LDS beside the loop's other buffers is refused at creation with
    PK_ERR_UNSUPPORTED and a message, not decoded wrongly."""
    from parakeet_amd import pk, synth
    path = str(tmp_path / "j4096.gguf")
    synth.make_decoder_gguf(path, kind="tdt", H=64, L=2, J=4096, D=64, vocab=50, durations=[0, 1, 2, 3, 4])
    with pytest.raises(pk.PkError) as ei:
        pk.Decoder.from_gguf(path, n_slots=1)
    assert ei.value.rc == 5 and "LDS" in str(ei.value), ei.value
