"""Blank ids other than vocab_size on the device.  The reference takes the
blank from parakeet.{tdt,eou}.blank_id (src/parakeet_ctc.cpp:430): the
predictor is primed with embed[blank] (src/parakeet_tdt.cpp:813-830,
src/parakeet_eou.cpp:217-230), a blank ends the frame's symbols, and EOU's
<EOU> resets the predictor to the blank (src/parakeet_eou.cpp:288-310).

- replays through the oracle step by step: TDT with blank 0 (with and without
  a blank-logit offset, which must move logit 0), EOU with blank 5 fed in
  2-frame chunks with the state and segment starts carried;
- relabelling: a decoder whose blank and one ordinary id are swapped (rows of
  the embedding and the joint output, and blank_id) decodes bit for bit the
  same on the device once the two ids are swapped back.  The oracle's blank
  handling is pinned the same way, and by closed forms, in tests/test_oracle.py."""
import numpy as np
import pytest

from conftest import small_eou, small_tdt
from parity import check_window
from test_oracle import swap_blank

pytestmark = pytest.mark.gpu


def _models(path, writer, **kw):
    from parakeet_amd import gguf, pk
    import oracle
    writer(path, **kw)
    return pk.Decoder.from_gguf(path, n_slots=8), oracle.OracleModel.from_gguf(path, gguf)


@pytest.mark.parametrize("blank_bias", [0.0, 2.0])
def test_tdt_blank_zero_replay(tmp_path, blank_bias):
    from parakeet_amd import synth
    path = str(tmp_path / "m.gguf")
    bias = small_tdt(path)["tdt.joint.out.bias"].copy()
    bias[0] += 1.5           # the blank is taken now and then even without the offset
    dev, om = _models(path, small_tdt, blank_id=0, overrides={"tdt.joint.out.bias": bias})
    assert dev.info.blank == 0 and om.blank == 0
    encs = [synth.encoder_frames(900 + u, T, 128) for u, T in enumerate([3, 30, 57, 12])]
    print(f"TDT blank 0, blank_bias {blank_bias}: B=4", flush=True)
    res = dev.decode(encs, trace=True, max_symbols=10, blank_bias=blank_bias)
    n_blank = 0
    for u, enc in enumerate(encs):
        check_window(om, dev, u, enc, res[u], om.new_state(), 10, blank_bias=blank_bias)
        n_blank += int((np.asarray(res[u]["trace"])[:, 0] == 0).sum())
        assert 0 not in res[u]["tokens"].tolist()
    assert n_blank > 0
    dev.close()


def test_eou_blank_five_chunked(tmp_path):
    from parakeet_amd import synth
    path = str(tmp_path / "e.gguf")
    w = small_eou(path)
    bias = w["eou.joint.out.bias"].copy()
    bias[33] += 1.5          # <EOU> now and then, so segments end and the predictor resets
    dev, om = _models(path, small_eou, blank_id=5, overrides={"eou.joint.out.bias": bias})
    assert dev.info.blank == 5
    B, n_chunks = 4, 10
    encs = [synth.encoder_frames(950 + u, 2 * n_chunks, 64) for u in range(B)]
    for u in range(B):
        dev.init_state(u)
    ost = [om.new_state() for _ in range(B)]
    for o in ost:
        om.init_state(o)
    total = np.zeros(B, np.int32)
    n_seg = 0
    print(f"EOU blank 5: B={B} chunks={n_chunks}", flush=True)
    for c in range(n_chunks):
        ws = [e[2 * c:2 * c + 2] for e in encs]
        res = dev.decode(ws, slots=list(range(B)), trace=True, tokens_base=total, max_symbols=5)
        for u in range(B):
            check_window(om, dev, u, ws[u], res[u], ost[u], 5, tokens_before=int(total[u]))
            assert 5 not in res[u]["tokens"].tolist()
            total[u] += len(res[u]["tokens"])
            n_seg += len(res[u]["segments"])
    assert n_seg > 0 and total.sum() > 0
    dev.close()


@pytest.mark.parametrize("kind", ["tdt", "eou"])
def test_blank_id_relabelling_on_device(tmp_path, kind):
    from parakeet_amd import pk, synth
    writer, vocab, D, b = (small_tdt, 61, 128, 0) if kind == "tdt" else (small_eou, 35, 64, 5)
    w = writer(str(tmp_path / "a.gguf"))
    bias = w[f"{kind}.joint.out.bias"].copy()
    bias[b] += 1.0
    bias[vocab] += 2.0
    w = writer(str(tmp_path / "a.gguf"), overrides={f"{kind}.joint.out.bias": bias})
    shaped = dict(w)
    shaped[f"{kind}.predict.embed.weight"] = w[f"{kind}.predict.embed.weight"].reshape(-1, 64)
    shaped[f"{kind}.joint.out.weight"] = w[f"{kind}.joint.out.weight"].reshape(-1, 96)
    writer(str(tmp_path / "b.gguf"), blank_id=b, overrides=swap_blank(shaped, kind, vocab, b))
    da = pk.Decoder.from_gguf(str(tmp_path / "a.gguf"), n_slots=4)
    db = pk.Decoder.from_gguf(str(tmp_path / "b.gguf"), n_slots=4)
    ms = 10 if kind == "tdt" else 5
    encs = [synth.encoder_frames(990 + u, T, D) for u, T in enumerate([25, 40, 9])]
    print(f"relabelling {kind}: blank {vocab} <-> {b}", flush=True)
    ra = da.decode(encs, trace=True, max_symbols=ms)
    rb = db.decode(encs, trace=True, max_symbols=ms)
    for u in range(len(encs)):
        tb = np.array(rb[u]["trace"])
        tb[:, 0] = np.where(tb[:, 0] == b, vocab, np.where(tb[:, 0] == vocab, b, tb[:, 0]))
        assert np.array_equal(np.asarray(ra[u]["trace"]), tb), u
        assert ra[u]["steps"] == rb[u]["steps"]
        if kind == "eou":
            assert np.array_equal(ra[u]["segments"], rb[u]["segments"])
        sa, sb = da.read_state(u), db.read_state(u)
        assert np.array_equal(sa["h"], sb["h"]) and np.array_equal(sa["c"], sb["c"]), u
    da.close()
    db.close()
