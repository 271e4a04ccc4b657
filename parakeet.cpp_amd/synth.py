"""Seeded synthetic decoder checkpoints and encoder frames.

Writes decoder-only GGUFs in the reference converter's layout
(scripts/convert-nemo-to-gguf.py:293-352 metadata, :506-525 EOU tensors,
:563-582 TDT tensors) with random weights N(0, 1/sqrt(fan_in)), fan_in being
the ``in`` dimension of each matrix (the embedding uses its row length H).
Biases are drawn the same way and stored f32.  Matrices are q8_0 / q5_0 /
q4_0 when ``in % 32 == 0`` (otherwise f16), or f16 / f32 for those
quantisation modes, as in the converter's ``add_2d``.

The files carry only the prediction/joint network: the encoder is not part of
the decode path and its tensors are absent (readers run in decoder-only mode).
"""
from __future__ import annotations

import numpy as np

from . import gguf as G

WEIGHT_SEED = 0xC0FFEE

# Decoder shapes of the published checkpoints (dims from their NeMo configs).
SHAPES = {
    "tdt-0.6b-v3": dict(kind="tdt", H=640, L=2, J=640, D=1024, vocab=8192,
                        durations=[0, 1, 2, 3, 4], quant="q8_0"),
    "tdt-1.1b": dict(kind="tdt", H=640, L=2, J=640, D=1024, vocab=1024,
                     durations=[0, 1, 2, 3, 4], quant="f16"),
    "eou-120m": dict(kind="eou", H=640, L=1, J=640, D=512, vocab=1027,
                     eou_id=1025, eob_id=1026, max_symbols=5, quant="q8_0"),
}


def _matrix(w: G.GGUFWriter, name: str, arr: np.ndarray, quant: str):
    out_dim, in_dim = arr.shape
    if quant in G.QUANT_TYPES and in_dim % 32 == 0:
        t = G.QUANT_TYPES[quant]
        w.add_tensor(name, G.QUANTIZE[t](arr), (in_dim, out_dim), t)
    elif quant == "f32":
        w.add_tensor(name, arr.astype(np.float32).tobytes(), (in_dim, out_dim), G.GGML_F32)
    else:
        w.add_tensor(name, arr.astype(np.float16).tobytes(), (in_dim, out_dim), G.GGML_F16)


def _vec(w: G.GGUFWriter, name: str, arr: np.ndarray):
    w.add_tensor(name, arr.astype(np.float32).tobytes(), (arr.shape[0],), G.GGML_F32)


def vocab_pieces(kind: str, vocab: int, eou_id: int = -1, eob_id: int = -1) -> list[str]:
    """Synthetic SentencePiece table: ``<unk>`` at 0, ``<EOU>``/``<EOB>`` for EOU
    models, word pieces elsewhere.  Only ``<...>`` pieces are special."""
    pieces = ["▁t%d" % i for i in range(vocab)]
    pieces[0] = "<unk>"
    if kind == "eou":
        pieces[eou_id] = "<EOU>"
        pieces[eob_id] = "<EOB>"
    return pieces


def make_decoder_gguf(path: str, kind: str, H: int, L: int, J: int, D: int, vocab: int,
                      durations=None, eou_id: int = -1, eob_id: int = -1, max_symbols: int = 5,
                      quant: str = "q8_0", seed: int = WEIGHT_SEED, scale: float = 1.0,
                      overrides: dict | None = None, meta_u32: dict | None = None,
                      num_durations: int | None = None, blank_id: int | None = None) -> dict:
    """Write a decoder GGUF and return its float32 weights (dequantised from
    the stored bytes) keyed by tensor name.  ``overrides`` replaces named
    tensors (PyTorch layout) before quantisation -- used by scripted models;
    ``meta_u32`` adds u32 metadata keys (e.g. parakeet.preproc.hop_length).

    TDT durations: ``num_durations`` (the duration logits, default the table's
    length, or 5 without a table) is written apart from the table, as the
    reference reads them (src/parakeet_ctc.cpp:428-439).  ``durations=None``
    leaves the table key out (readers then use {0, 1, 2, 3, 4}); an empty list
    writes an empty table (the duration is then the logit index).  ``blank_id``
    defaults to ``vocab`` (the converter's choice; readers take any id)."""
    rng = np.random.default_rng(seed)
    p = "tdt" if kind == "tdt" else "eou"
    V1 = vocab + 1
    if kind == "tdt":
        n_dur = num_durations if num_durations is not None else (5 if durations is None else len(durations))
    else:
        n_dur = 0
    Vo = V1 + n_dur
    G4 = 4 * H

    def normal(shape, fan_in):
        return (rng.standard_normal(shape, dtype=np.float32) * (scale / np.sqrt(fan_in))).astype(np.float32)

    tensors = {}
    tensors[f"{p}.predict.embed.weight"] = normal((V1, H), H)
    for l in range(L):
        tensors[f"{p}.predict.lstm.{l}.w_ih"] = normal((G4, H), H)
        tensors[f"{p}.predict.lstm.{l}.w_hh"] = normal((G4, H), H)
        tensors[f"{p}.predict.lstm.{l}.b_ih"] = normal((G4,), H)
        tensors[f"{p}.predict.lstm.{l}.b_hh"] = normal((G4,), H)
    tensors[f"{p}.joint.enc.weight"] = normal((J, D), D)
    tensors[f"{p}.joint.enc.bias"] = normal((J,), D)
    tensors[f"{p}.joint.pred.weight"] = normal((J, H), H)
    tensors[f"{p}.joint.pred.bias"] = normal((J,), H)
    tensors[f"{p}.joint.out.weight"] = normal((Vo, J), J)
    tensors[f"{p}.joint.out.bias"] = normal((Vo,), J)
    for k, v in (overrides or {}).items():
        assert tensors[k].shape == v.shape, (k, tensors[k].shape, v.shape)
        tensors[k] = np.asarray(v, dtype=np.float32)

    w = G.GGUFWriter()
    w.add_str("general.architecture", "parakeet-ctc")
    w.add_str("general.name", f"parakeet-{kind}-synthetic-decoder")
    w.add_str("parakeet.model.type", kind)
    w.add_u32("parakeet.encoder.d_model", D)
    if kind == "tdt":
        w.add_u32("parakeet.tdt.vocab_size", vocab)
        w.add_u32("parakeet.tdt.blank_id", vocab if blank_id is None else blank_id)
        w.add_u32("parakeet.tdt.pred_hidden", H)
        w.add_u32("parakeet.tdt.pred_rnn_layers", L)
        w.add_u32("parakeet.tdt.joint_hidden", J)
        w.add_u32("parakeet.tdt.num_durations", n_dur)
        if durations is not None:
            w.add_arr("parakeet.tdt.durations", G.T_I32, list(durations))
    else:
        w.add_u32("parakeet.eou.vocab_size", vocab)
        w.add_u32("parakeet.eou.blank_id", vocab if blank_id is None else blank_id)
        w.add_i32("parakeet.eou.eou_id", eou_id)
        w.add_i32("parakeet.eou.eob_id", eob_id)
        w.add_u32("parakeet.eou.pred_hidden", H)
        w.add_u32("parakeet.eou.pred_rnn_layers", L)
        w.add_u32("parakeet.eou.joint_hidden", J)
        w.add_u32("parakeet.eou.max_symbols_per_step", max_symbols)
    w.add_arr("tokenizer.ggml.tokens", G.T_STR, vocab_pieces(kind, vocab, eou_id, eob_id))
    w.add_bool("parakeet.decoder_only", True)
    for k, v in (meta_u32 or {}).items():
        w.add_u32(k, int(v))

    for name, arr in tensors.items():
        if arr.ndim == 2:
            _matrix(w, name, arr, quant)
        else:
            _vec(w, name, arr)
    w.write(path)
    rd = G.GGUFReader(path)
    return {name: rd.f32(name) for name in tensors}


def make_shape(path: str, shape: str, seed: int = WEIGHT_SEED, quant: str | None = None, **kw) -> dict:
    cfg = dict(SHAPES[shape])
    if quant is not None:
        cfg["quant"] = quant
    cfg.update(kw)
    return make_decoder_gguf(path, seed=seed, **cfg)


def encoder_frames(u: int, T: int, D: int, base_seed: int = 1000) -> np.ndarray:
    """fp32 N(0,1) frames [T, D] for utterance u (seed base_seed + u)."""
    return np.random.default_rng(base_seed + u).standard_normal((T, D), dtype=np.float32)


def ragged_lengths(n: int, lo: int = 50, hi: int = 1500, seed: int = 7) -> np.ndarray:
    return np.random.default_rng(seed).integers(lo, hi + 1, size=n).astype(np.int32)


def blank_offsets(n: int, seed: int = 11) -> np.ndarray:
    return np.random.default_rng(seed).choice(np.array([0.0, 2.0, 4.0], dtype=np.float32), size=n)
