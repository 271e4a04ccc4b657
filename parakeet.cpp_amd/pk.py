"""ctypes binding of the C ABI in include/parakeet_hip.h (libparakeet_hip.so).

``Decoder`` mirrors the reference decoder runtime for one GGUF:
``Decoder.from_gguf`` ~ load_from_gguf + tdt_prepare_runtime / eou_prepare_runtime
(src/parakeet_ctc.cpp:297-682, src/parakeet_tdt.cpp:585, src/parakeet_eou.cpp:172),
``init_state`` ~ tdt_init_state / eou_init_state, ``decode_window`` ~
tdt_decode_window / eou_decode_window batched over utterances.  The library
must be built (``python -m`` build via __graft_entry__.build()); loading fails
loudly otherwise -- there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

from . import gguf as G

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libparakeet_hip.so")

PK_MAX_LAYERS = 8
PK_MAX_DURATIONS = 16
PK_MAX_BATCH = 512
KIND_TDT, KIND_EOU = 0, 1
MEM_HOST, MEM_DEVICE, MEM_DEVICE_FRAMES = 0, 1, 2   # pk_batch.mem (parakeet_hip.h)
PK_CTRL_N = 8
CTRL_INIT, CTRL_SYM, CTRL_CARRY, CTRL_LAST, CTRL_SEGSTART, CTRL_CUR = range(6)

RC_NAMES = {0: "ok", 1: "encoder dim mismatch", 2: "tensor", 3: "argument", 4: "no memory",
            5: "unsupported", 6: "device", 7: "timeout", 11: "overflow"}


class PkError(RuntimeError):
    def __init__(self, rc, msg):
        super().__init__(f"pk rc={rc} ({RC_NAMES.get(rc, '?')}): {msg}")
        self.rc = rc


class PkTensor(C.Structure):
    _fields_ = [("data", C.c_void_p), ("type", C.c_int32), ("ne0", C.c_int64), ("ne1", C.c_int64)]


class PkDecoderDesc(C.Structure):
    _fields_ = [("kind", C.c_int32), ("pred_hidden", C.c_int32), ("pred_rnn_layers", C.c_int32),
                ("joint_hidden", C.c_int32), ("d_enc", C.c_int32), ("vocab_size", C.c_int32),
                ("blank_id", C.c_int32), ("num_durations", C.c_int32),
                ("n_duration_values", C.c_int32), ("durations", C.c_int32 * PK_MAX_DURATIONS),
                ("eou_id", C.c_int32), ("eob_id", C.c_int32), ("special", C.POINTER(C.c_uint8)),
                ("n_special", C.c_int32), ("embed", PkTensor),
                ("w_ih", PkTensor * PK_MAX_LAYERS), ("w_hh", PkTensor * PK_MAX_LAYERS),
                ("b_ih", PkTensor * PK_MAX_LAYERS), ("b_hh", PkTensor * PK_MAX_LAYERS),
                ("joint_enc_w", PkTensor), ("joint_enc_b", PkTensor),
                ("joint_pred_w", PkTensor), ("joint_pred_b", PkTensor),
                ("joint_out_w", PkTensor), ("joint_out_b", PkTensor)]


class PkBatch(C.Structure):
    _fields_ = [("n_utts", C.c_int32), ("mem", C.c_int32), ("d_enc", C.c_int32),
                ("max_symbols", C.c_int32), ("enc", C.c_void_p), ("enc_row", C.c_void_p),
                ("n_frames", C.c_void_p), ("slot", C.c_void_p), ("blank_bias", C.c_void_p),
                ("tokens_base", C.c_void_p), ("tokens", C.c_void_p), ("token_cap", C.c_int32),
                ("n_tokens", C.c_void_p), ("steps", C.c_void_p), ("segments", C.c_void_p),
                ("seg_cap", C.c_int32), ("n_segments", C.c_void_p), ("trace", C.c_void_p),
                ("trace_cap", C.c_int32), ("logits", C.c_void_p), ("logit_steps", C.c_int32),
                ("reset", C.c_void_p), ("ctrl_out", C.c_void_p)]


EXPORTED = ["pk_decoder_create", "pk_decoder_destroy", "pk_slot_init", "pk_slot_reset",
            "pk_slot_read", "pk_slot_copy", "pk_decode", "pk_decode_noalloc", "pk_last_timing", "pk_last_error",
            "pk_device_info", "pk_window_split", "pk_decoder_set_timing"]

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        L.pk_decoder_create.argtypes = [C.POINTER(PkDecoderDesc), C.c_int32, C.POINTER(C.c_void_p)]
        L.pk_decoder_destroy.argtypes = [C.c_void_p]
        L.pk_slot_init.argtypes = [C.c_void_p, C.c_int32]
        L.pk_slot_reset.argtypes = [C.c_void_p, C.c_int32]
        L.pk_slot_read.argtypes = [C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        L.pk_slot_copy.argtypes = [C.c_void_p, C.c_int32, C.c_int32]
        L.pk_decode.argtypes = [C.c_void_p, C.POINTER(PkBatch)]
        L.pk_decode_noalloc.argtypes = [C.c_void_p, C.POINTER(PkBatch)]
        L.pk_last_timing.argtypes = [C.c_void_p, C.POINTER(C.c_float), C.POINTER(C.c_float),
                                     C.POINTER(C.c_int32)]
        L.pk_last_error.restype = C.c_char_p
        L.pk_decoder_set_timing.argtypes = [C.c_void_p, C.c_int32]
        L.pk_device_info.argtypes = [C.POINTER(C.c_int32)] * 3
        L.pk_window_split.argtypes = [C.c_int32, C.c_void_p, C.c_int32, C.c_int32, C.c_int32,
                                      C.POINTER(C.c_int32), C.c_void_p]
        _lib = L
    return _lib


def check(rc):
    if rc != 0:
        raise PkError(rc, lib().pk_last_error().decode(errors="replace"))


def _ptr(a: np.ndarray | None):
    return None if a is None else C.c_void_p(a.ctypes.data)


def _per_utt(v, n: int, dtype, name: str, scalar: bool = True):
    """A per-utterance descriptor array of exactly n entries (the C ABI reads n
    of them); a scalar is repeated for every utterance where ``scalar``."""
    if v is None:
        return None
    a = np.asarray(v, dtype)
    if a.ndim == 0 and scalar:
        a = np.full(n, a, dtype)
    if a.shape != (n,):
        raise ValueError(f"{name}: shape {a.shape} for {n} utterances")
    return np.ascontiguousarray(a)


class DecoderInfo:
    """Decoder metadata as the reference loader reads it (src/parakeet_ctc.cpp:418-458)."""

    def __init__(self, rd: G.GGUFReader):
        kv = rd.kv
        if kv.get("general.architecture") != "parakeet-ctc":
            raise PkError(2, "expected general.architecture = parakeet-ctc")
        self.kind_str = kv.get("parakeet.model.type", "ctc")
        if self.kind_str not in ("tdt", "eou"):
            raise PkError(5, f"model type {self.kind_str!r} has no transducer decoder")
        self.kind = KIND_TDT if self.kind_str == "tdt" else KIND_EOU
        p = f"parakeet.{self.kind_str}."
        self.D = int(kv.get("parakeet.encoder.d_model", 1024))
        if self.kind == KIND_TDT:
            self.H = int(kv.get(p + "pred_hidden", 640))
            self.L = int(kv.get(p + "pred_rnn_layers", 2))
            self.J = int(kv.get(p + "joint_hidden", 640))
            self.Dn = int(kv.get(p + "num_durations", 5))
            self.vocab = int(kv.get(p + "vocab_size", 8192))
            self.blank = int(kv.get(p + "blank_id", self.vocab))
            d = kv.get(p + "durations")
            self.durations = [0, 1, 2, 3, 4] if d is None else [int(x) for x in d]
            self.eou_id = self.eob_id = -1
            self.max_symbols = 10          # TdtDecodeOptions default (src/parakeet_tdt.h:165)
        else:
            self.H = int(kv.get(p + "pred_hidden", 640))
            self.L = int(kv.get(p + "pred_rnn_layers", 1))
            self.J = int(kv.get(p + "joint_hidden", 640))
            self.Dn = 0
            self.vocab = int(kv.get(p + "vocab_size", 1026))
            self.blank = int(kv.get(p + "blank_id", self.vocab))
            self.durations = []
            self.eou_id = int(kv.get(p + "eou_id", -1))
            self.eob_id = int(kv.get(p + "eob_id", -1))
            self.max_symbols = int(kv.get(p + "max_symbols_per_step", 5))
        pieces = kv.get("tokenizer.ggml.tokens", [])
        self.pieces = list(pieces)
        self.special = np.array([1 if (len(s) > 0 and s[0] == "<" and s[-1] == ">") else 0
                                 for s in pieces], np.uint8)
        self.V1 = self.vocab + 1
        self.Vo = self.V1 + self.Dn


class Decoder:
    """One uploaded decoder with ``n_slots`` device state slots."""

    def __init__(self, rd: G.GGUFReader, n_slots: int = 1):
        self.info = info = DecoderInfo(rd)
        self.n_slots = n_slots
        pfx = info.kind_str
        desc = PkDecoderDesc()
        desc.kind, desc.pred_hidden, desc.pred_rnn_layers = info.kind, info.H, info.L
        desc.joint_hidden, desc.d_enc, desc.vocab_size = info.J, info.D, info.vocab
        desc.blank_id, desc.num_durations = info.blank, info.Dn
        desc.n_duration_values = len(info.durations)
        for i, v in enumerate(info.durations):
            desc.durations[i] = v
        desc.eou_id, desc.eob_id = info.eou_id, info.eob_id
        keep = []

        def tensor(name):
            t = PkTensor()
            if name not in rd.tensors:
                return t
            ti = rd.tensors[name]
            raw = np.frombuffer(rd.raw(name), np.uint8).copy()
            keep.append(raw)
            t.data = raw.ctypes.data
            t.type = ti.ggml_type
            t.ne0 = ti.ne[0]
            t.ne1 = ti.ne[1] if len(ti.ne) > 1 else 1
            return t

        if len(info.special):
            sp = np.ascontiguousarray(info.special)
            keep.append(sp)
            desc.special = sp.ctypes.data_as(C.POINTER(C.c_uint8))
            desc.n_special = len(sp)
        desc.embed = tensor(f"{pfx}.predict.embed.weight")
        for l in range(info.L):
            desc.w_ih[l] = tensor(f"{pfx}.predict.lstm.{l}.w_ih")
            desc.w_hh[l] = tensor(f"{pfx}.predict.lstm.{l}.w_hh")
            desc.b_ih[l] = tensor(f"{pfx}.predict.lstm.{l}.b_ih")
            desc.b_hh[l] = tensor(f"{pfx}.predict.lstm.{l}.b_hh")
        desc.joint_enc_w = tensor(f"{pfx}.joint.enc.weight")
        desc.joint_enc_b = tensor(f"{pfx}.joint.enc.bias")
        desc.joint_pred_w = tensor(f"{pfx}.joint.pred.weight")
        desc.joint_pred_b = tensor(f"{pfx}.joint.pred.bias")
        desc.joint_out_w = tensor(f"{pfx}.joint.out.weight")
        desc.joint_out_b = tensor(f"{pfx}.joint.out.bias")
        h = C.c_void_p()
        check(lib().pk_decoder_create(C.byref(desc), n_slots, C.byref(h)))
        self.h = h
        del keep

    @classmethod
    def from_gguf(cls, path: str, n_slots: int = 1):
        return cls(G.GGUFReader(path), n_slots)

    def close(self):
        if getattr(self, "h", None):
            lib().pk_decoder_destroy(self.h)
            self.h = None

    def __del__(self):
        if sys.is_finalizing():   # no HIP call during interpreter shutdown (see hipmem.DeviceArray)
            return
        try:
            self.close()
        except Exception:
            pass

    # ---- state ----
    def init_state(self, slot: int):
        check(lib().pk_slot_init(self.h, slot))

    def reset_state(self, slot: int):
        check(lib().pk_slot_reset(self.h, slot))

    def copy_state(self, src: int, dst: int):
        check(lib().pk_slot_copy(self.h, src, dst))

    def read_state(self, slot: int):
        i = self.info
        h = np.zeros(i.L * i.H, np.float32)
        c = np.zeros(i.L * i.H, np.float32)
        pred = np.zeros(i.H, np.float32)
        ctrl = np.zeros(PK_CTRL_N, np.int32)
        check(lib().pk_slot_read(self.h, slot, _ptr(h), _ptr(c), _ptr(pred), _ptr(ctrl)))
        return dict(h=h, c=c, pred=pred, ctrl=ctrl)

    # ---- decode ----
    def decode(self, encs: list, slots=None, max_symbols: int | None = None, blank_bias=None,
               tokens_base=None, trace: bool = False, token_cap: int | None = None, logit_steps: int = 0,
               reset=None):
        """Host-memory batch: encs[u] is [T_u, D] f32.  Returns a list of dicts
        (``logits``: [logit_steps, Vo] joint logits of the first steps when
        logit_steps > 0; rows past the utterance's steps are NaN)."""
        n = len(encs)
        T = np.array([e.shape[0] if e.ndim == 2 else 0 for e in encs], np.int32)
        rows = np.concatenate([[0], np.cumsum(T)[:-1]]).astype(np.int64) if n else np.zeros(0, np.int64)
        d_enc = encs[0].shape[1] if n and encs[0].ndim == 2 else self.info.D
        if n and T.sum() > 0:
            live = [e for e in encs if e.ndim == 2 and e.shape[0] > 0]
            enc = (np.concatenate(live) if all(e.dtype == np.float32 for e in live)
                   else np.concatenate([np.asarray(e, np.float32) for e in live]))
        else:
            enc = np.zeros((1, d_enc), np.float32)
        return self._decode(MEM_HOST, _ptr(enc), rows, T, d_enc, slots, max_symbols, blank_bias, tokens_base,
                            trace, token_cap, logit_steps, reset)

    def decode_device_frames(self, enc_ptr: int, enc_row, n_frames, slots=None, max_symbols: int | None = None,
                             blank_bias=None, tokens_base=None, trace: bool = False, token_cap: int | None = None,
                             logit_steps: int = 0):
        """Frames already in device memory (e.g. an encoder output tensor's data
        pointer), read in place: utterance u decodes rows enc_row[u] ..
        enc_row[u] + n_frames[u] of the [rows, D] f32 array at enc_ptr.  The
        producer's stream must be synchronised first.  Returns what decode does."""
        T = np.ascontiguousarray(n_frames, np.int32).reshape(-1)
        rows = _per_utt(enc_row, len(T), np.int64, "enc_row", scalar=False)
        return self._decode(MEM_DEVICE_FRAMES, C.c_void_p(enc_ptr), rows, T, self.info.D, slots, max_symbols,
                            blank_bias, tokens_base, trace, token_cap, logit_steps)

    def _decode(self, mem, enc, rows, T, d_enc, slots, max_symbols, blank_bias, tokens_base, trace, token_cap,
                logit_steps=0, reset=None):
        """One pk_decode call with host outputs; per-utterance result dicts."""
        info = self.info
        n = len(T)
        max_symbols = info.max_symbols if max_symbols is None else max_symbols
        slots = np.arange(n, dtype=np.int32) if slots is None else _per_utt(slots, n, np.int32, "slots", False)
        maxT = int(T.max()) if n else 0
        cap = token_cap if token_cap is not None else maxT * max(1, max_symbols) + 1
        toks = np.zeros((n, cap), np.int32)
        ntok = np.zeros(n, np.int32)
        steps = np.zeros(n, np.int32)
        segs = np.zeros((n, cap + 1), np.int32)
        nseg = np.zeros(n, np.int32)
        tcap = maxT * (max(1, max_symbols) + 1) + 1 if trace else 0
        tr = np.zeros((n, max(tcap, 1), 2), np.int32)
        bb = _per_utt(blank_bias, n, np.float32, "blank_bias")
        tb = _per_utt(tokens_base, n, np.int32, "tokens_base")
        b = PkBatch()
        b.n_utts, b.mem, b.d_enc, b.max_symbols = n, mem, d_enc, max_symbols
        b.enc, b.enc_row, b.n_frames, b.slot = enc, _ptr(rows), _ptr(T), _ptr(slots)
        b.blank_bias, b.tokens_base = _ptr(bb), _ptr(tb)
        b.tokens, b.token_cap, b.n_tokens, b.steps = _ptr(toks), cap, _ptr(ntok), _ptr(steps)
        b.segments, b.seg_cap, b.n_segments = _ptr(segs), cap + 1, _ptr(nseg)
        b.trace, b.trace_cap = (_ptr(tr) if trace else None), tcap
        rs = _per_utt(reset, n, np.uint8, "reset")
        ctrl = np.zeros((n, PK_CTRL_N), np.int32)
        b.reset, b.ctrl_out = _ptr(rs), _ptr(ctrl)
        lg = None
        if logit_steps > 0:
            lg = np.full((n, logit_steps, info.Vo), np.nan, np.float32)
            b.logits, b.logit_steps = _ptr(lg), logit_steps
        check(lib().pk_decode(self.h, C.byref(b)))
        # per-utterance views of this call's output arrays
        nt, st, ns = ntok.tolist(), steps.tolist(), nseg.tolist()
        out = [dict(tokens=toks[u, :nt[u]], steps=st[u], segments=segs[u, :ns[u]], ctrl=ctrl[u]) for u in range(n)]
        if trace:
            for u in range(n):
                out[u]["trace"] = tr[u, :min(st[u], tcap)]
        if lg is not None:
            for u in range(n):
                out[u]["logits"] = lg[u]
        return out

    def decode_device(self, enc_ptr: int, enc_row, n_frames, slots, max_symbols: int,
                      out_ptrs: dict, token_cap: int, blank_bias=None, trace_cap: int = 0,
                      tokens_base=None, noalloc: bool = False):
        """Device-memory batch (inputs resident in HBM): pointers are device
        addresses; the descriptor arrays (enc_row, n_frames, slots, blank_bias,
        tokens_base) are host arrays.  noalloc: pk_decode_noalloc (no device
        allocation; call scratch from the fixed per-device array)."""
        T = np.ascontiguousarray(n_frames, np.int32).reshape(-1)
        n = len(T)
        rows = _per_utt(enc_row, n, np.int64, "enc_row", scalar=False)
        sl = _per_utt(slots, n, np.int32, "slots", scalar=False)
        bb = _per_utt(blank_bias, n, np.float32, "blank_bias")
        b = PkBatch()
        b.n_utts, b.mem, b.d_enc, b.max_symbols = n, MEM_DEVICE, self.info.D, max_symbols
        b.enc, b.enc_row, b.n_frames, b.slot = C.c_void_p(enc_ptr), _ptr(rows), _ptr(T), _ptr(sl)
        tb = _per_utt(tokens_base, n, np.int32, "tokens_base")
        b.blank_bias, b.tokens_base = _ptr(bb), _ptr(tb)
        b.tokens, b.token_cap = C.c_void_p(out_ptrs["tokens"]), token_cap
        b.n_tokens, b.steps = C.c_void_p(out_ptrs["n_tokens"]), C.c_void_p(out_ptrs["steps"])
        b.segments = C.c_void_p(out_ptrs["segments"]) if out_ptrs.get("segments") else None
        b.seg_cap = out_ptrs.get("seg_cap", 0)
        b.n_segments = C.c_void_p(out_ptrs["n_segments"]) if out_ptrs.get("n_segments") else None
        b.trace = C.c_void_p(out_ptrs["trace"]) if trace_cap else None
        b.trace_cap = trace_cap
        check((lib().pk_decode_noalloc if noalloc else lib().pk_decode)(self.h, C.byref(b)))

    def last_timing(self):
        """Kernel times of the last call (ms; -1 when timing was off for it) and its
        lockstep iterations."""
        a, b, it = C.c_float(), C.c_float(), C.c_int32()
        check(lib().pk_last_timing(self.h, C.byref(a), C.byref(b), C.byref(it)))
        return dict(enc_proj_ms=a.value, loop_ms=b.value, iterations=it.value)

    def set_timing(self, on: bool):
        """Record the timing events of last_timing in each call (the default) or not."""
        check(lib().pk_decoder_set_timing(self.h, 1 if on else 0))


def window_split(n_frames, max_symbols: int, joint_hidden: int, max_duration: int):
    """pk_window_split: (piece_frames, launches[u]) -- how pk_decode splits windows that
    one launch cannot take (host arithmetic, no device needed)."""
    T = np.ascontiguousarray(n_frames, np.int32)
    k = np.zeros(len(T), np.int32)
    w = C.c_int32()
    check(lib().pk_window_split(len(T), _ptr(T), max_symbols, joint_hidden, max_duration, C.byref(w), _ptr(k)))
    return w.value, k


def device_info():
    a, b, c = C.c_int32(), C.c_int32(), C.c_int32()
    check(lib().pk_device_info(C.byref(a), C.byref(b), C.byref(c)))
    return dict(n_cu=a.value, lds_per_block=b.value, wave_size=c.value)
