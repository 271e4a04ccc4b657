"""The C++ GGUF loader and detokenize (host only, no GPU): tests/cpp/loader_main
prints what load_from_gguf read.

- metadata dispatch and defaults follow src/parakeet_ctc.cpp:418-458
  (parakeet.model.type -> tdt / eou / sortformer, anything else ctc; TDT
  vocab 8192, blank = vocab, durations {0,1,2,3,4}; EOU vocab 1026, eou_id /
  eob_id -1 when absent) and :470-473 / :385 for the frame stride;
- status codes: 1 cannot open, 2 wrong architecture or a missing decoder
  tensor (encoder tensors are not required);
- detokenize (src/sentencepiece_bpe.cpp:9-38): ids out of range and the
  blank / bos / eos / pad ids are skipped, U+2581 becomes a space, leading
  spaces are trimmed and nothing else."""
import json
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT, small_eou, small_tdt

DRIVER = os.path.join(ROOT, "tests", "cpp", "loader_main")


def _load(path, *ids):
    assert os.path.exists(DRIVER), "run __graft_entry__.build()"
    r = subprocess.run([DRIVER, path, *[str(i) for i in ids]], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout)


def _gguf(path, meta, tensors=(), pieces=None, special=None):
    """A GGUF with the given metadata and tiny f32 tensors of the given names
    (the loader checks presence; shapes are checked when a runtime is made)."""
    from parakeet_amd import gguf as G
    w = G.GGUFWriter()
    w.add_str("general.architecture", meta.pop("general.architecture", "parakeet-ctc"))
    for k, v in meta.items():
        if isinstance(v, str):
            w.add_str(k, v)
        elif isinstance(v, list):
            w.add_arr(k, G.T_I32, v)
        elif k.endswith("_id") and v < 0:
            w.add_i32(k, v)
        else:
            w.add_u32(k, v)
    if pieces is not None:
        w.add_arr("tokenizer.ggml.tokens", G.T_STR, pieces)
    for k, v in (special or {}).items():
        w.add_u32(k, v)
    for name in tensors:
        w.add_tensor(name, np.zeros(4, np.float32).tobytes(), (4,), G.GGML_F32)
    w.write(path)


def _decoder_tensors(p, L):
    names = [f"{p}.predict.embed.weight", f"{p}.joint.enc.weight", f"{p}.joint.enc.bias",
             f"{p}.joint.pred.weight", f"{p}.joint.pred.bias", f"{p}.joint.out.weight", f"{p}.joint.out.bias"]
    for l in range(L):
        names += [f"{p}.predict.lstm.{l}.{n}" for n in ("w_ih", "w_hh", "b_ih", "b_hh")]
    return names


def test_synthetic_tdt_and_eou(tmp_path):
    small_tdt(str(tmp_path / "t.gguf"))
    m = _load(str(tmp_path / "t.gguf"))
    assert m["rc"] == 0 and m["type"] == "tdt" and m["d_model"] == 128
    assert m["vocab"] == 61 and m["blank"] == 61 and m["tdt"] == [64, 2, 96, 5]
    assert m["durations"] == [0, 1, 2, 3, 4] and m["n_pieces"] == 61
    assert m["stride_ms"] == 80.0 and m["special"] == [-1, -1, -1, -1]
    small_eou(str(tmp_path / "e.gguf"), meta_u32={"parakeet.preproc.hop_length": 320,
                                                   "parakeet.encoder.subsampling_factor": 4,
                                                   "parakeet.preproc.sample_rate": 8000})
    m = _load(str(tmp_path / "e.gguf"))
    assert m["type"] == "eou" and m["vocab"] == 35 and m["blank"] == 35 and m["eou"] == 33 and m["eob"] == 34
    assert m["eou_cfg"] == [64, 1, 96, 5]
    assert m["stride_ms"] == 1000.0 * 320 * 4 / 8000


def test_defaults_when_keys_are_absent(tmp_path):
    p = str(tmp_path / "d.gguf")
    _gguf(p, {"parakeet.model.type": "tdt"}, _decoder_tensors("tdt", 2))
    m = _load(p)
    assert m["rc"] == 0 and m["type"] == "tdt" and m["d_model"] == 1024
    assert m["vocab"] == 8192 and m["blank"] == 8192 and m["durations"] == [0, 1, 2, 3, 4]
    assert m["tdt"] == [640, 2, 640, 5]
    _gguf(p, {"parakeet.model.type": "eou"}, _decoder_tensors("eou", 1))
    m = _load(p)
    assert m["type"] == "eou" and m["vocab"] == 1026 and m["blank"] == 1026
    assert m["eou"] == -1 and m["eob"] == -1 and m["eou_cfg"] == [640, 1, 640, 5]
    _gguf(p, {"parakeet.model.type": "tdt", "parakeet.tdt.vocab_size": 100, "parakeet.tdt.durations": [0, 2, 4]},
          _decoder_tensors("tdt", 2))
    m = _load(p)
    assert m["vocab"] == 100 and m["blank"] == 100 and m["durations"] == [0, 2, 4]


def test_model_type_dispatch(tmp_path):
    p = str(tmp_path / "c.gguf")
    for t, want in [("ctc", "ctc"), ("sortformer", "sortformer"), ("rnnt-unknown", "ctc")]:
        _gguf(p, {"parakeet.model.type": t}, ["encoder.pre_encode.conv.0.weight"])
        assert _load(p)["type"] == want, t
    _gguf(p, {}, [])                           # no type key: ctc
    assert _load(p)["type"] == "ctc"


def test_status_codes(tmp_path):
    assert _load(str(tmp_path / "missing.gguf"))["rc"] == 1
    p = str(tmp_path / "x.gguf")
    _gguf(p, {"general.architecture": "llama", "parakeet.model.type": "tdt"}, _decoder_tensors("tdt", 2))
    assert _load(p)["rc"] == 2
    names = _decoder_tensors("tdt", 2)
    for drop in ("tdt.joint.out.bias", "tdt.predict.lstm.1.w_hh"):
        _gguf(p, {"parakeet.model.type": "tdt"}, [n for n in names if n != drop])
        assert _load(p)["rc"] == 2, drop
    # a full checkpoint carries encoder tensors too; they are not read
    _gguf(p, {"parakeet.model.type": "tdt"}, names + ["encoder.layers.0.ff1.linear1.weight"])
    assert _load(p)["rc"] == 0
    with open(p, "r+b") as f:                   # not a GGUF file
        f.write(b"NOPE")
    assert _load(p)["rc"] == 1


def test_detokenize(tmp_path):
    p = str(tmp_path / "v.gguf")
    pieces = ["<unk>", "▁he", "llo", "▁wor", "ld", "<s>", "</s>", "<pad>", "▁▁x", "y▁", "\xe9", "▁"]
    _gguf(p, {"parakeet.model.type": "tdt", "parakeet.tdt.vocab_size": len(pieces)}, _decoder_tensors("tdt", 2),
          pieces=pieces, special={"tokenizer.ggml.bos_token_id": 5, "tokenizer.ggml.eos_token_id": 6,
                                  "tokenizer.ggml.pad_token_id": 7})
    assert _load(p)["special"] == [-1, 5, 6, 7]
    assert _load(p, 1, 2, 3, 4)["detok"] == "hello world"
    assert _load(p, 5, 1, 2, 6, 7, 3, 4, 6)["detok"] == "hello world"     # bos / eos / pad skipped
    assert _load(p, -1, 12, 99, 1, 2)["detok"] == "hello"                  # out of range (12 = blank) skipped
    assert _load(p, 0, 1)["detok"] == "<unk> he"                           # unk is not skipped
    assert _load(p, 8)["detok"] == "x" and _load(p, 9)["detok"] == "y "    # leading trimmed, trailing kept
    assert _load(p, 11, 11, 10)["detok"] == "\xe9"
    assert _load(p)["detok"] == ""


@pytest.mark.parametrize("quant", ["q4_0", "q5_0", "q8_0"])
def test_block_quantized_files_load(tmp_path, quant):
    """Decoder GGUFs with q4_0 / q5_0 / q8_0 matrices (18 / 22 / 34 bytes per 32 weights):
    the reader sizes every tensor from its type, so the whole file loads; the same file cut
    by one byte does not (its last tensor runs past the end)."""
    path = str(tmp_path / "m.gguf")
    small_tdt(path, quant=quant)
    assert _load(path)["rc"] == 0
    raw = open(path, "rb").read()
    cut = str(tmp_path / "cut.gguf")
    open(cut, "wb").write(raw[:-1])
    assert _load(cut)["rc"] == 1


@pytest.mark.parametrize("key,value", [("parakeet.tdt.pred_rnn_layers", 0x7FFFFFFF), ("parakeet.tdt.pred_rnn_layers", 9),
                                       ("parakeet.tdt.pred_hidden", 0), ("parakeet.tdt.vocab_size", 1 << 24),
                                       ("parakeet.tdt.num_durations", 17), ("parakeet.encoder.d_model", 0)])
def test_decoder_sizes_out_of_range(tmp_path, key, value):
    """Sizes the decoder cannot hold are refused with rc 2 before anything is sized from them
    (a corrupt layer count once made the loader build billions of tensor names)."""
    meta = {"parakeet.model.type": "tdt", key: value}
    path = str(tmp_path / "m.gguf")
    _gguf(path, meta, _decoder_tensors("tdt", 2))
    assert _load(path)["rc"] == 2
