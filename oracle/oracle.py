"""ctypes binding of the oracle library (liboracle.so, built by oracle/Makefile).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product path.

``OracleModel`` wraps a decoder given as float32 arrays keyed by GGUF tensor
name (the dequantised stored bytes, i.e. what the reference's
``*_prepare_runtime`` builds with ``dequantize_to_f32``), plus the metadata
the reference reads in src/parakeet_ctc.cpp:418-458.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

ORA_MAX_L = 8
ORA_MAX_DUR = 16
TDT, EOU = 0, 1

_fp = C.POINTER(C.c_float)
_ip = C.POINTER(C.c_int32)


class OraModel(C.Structure):
    _fields_ = [("kind", C.c_int), ("H", C.c_int), ("L", C.c_int), ("J", C.c_int), ("D", C.c_int),
                ("V1", C.c_int), ("Dn", C.c_int), ("Vo", C.c_int), ("blank", C.c_int),
                ("eou", C.c_int), ("eob", C.c_int), ("n_dur", C.c_int),
                ("durations", C.c_int * ORA_MAX_DUR), ("embed", _fp),
                ("w_ih", _fp * ORA_MAX_L), ("w_hh", _fp * ORA_MAX_L),
                ("b_ih", _fp * ORA_MAX_L), ("b_hh", _fp * ORA_MAX_L),
                ("enc_w", _fp), ("enc_b", _fp), ("pred_w", _fp), ("pred_b", _fp),
                ("out_w", _fp), ("out_b", _fp), ("special", C.POINTER(C.c_uint8)),
                ("n_special", C.c_int)]


class OraState(C.Structure):
    _fields_ = [("h", _fp), ("c", _fp), ("pred", _fp), ("symbols_this_step", C.c_int),
                ("initialized", C.c_int), ("carry_frames", C.c_int), ("last_token", C.c_int),
                ("segment_start_token", C.c_int)]


class OraReplayStats(C.Structure):
    _fields_ = [("steps", C.c_int), ("tok_mismatch", C.c_int), ("dur_mismatch", C.c_int),
                ("near_ties", C.c_int), ("unexplained", C.c_int), ("structure_error", C.c_int),
                ("first_unexplained", C.c_int), ("worst_margin", C.c_float),
                ("min_top2", C.c_float)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.ora_argmax.argtypes = [_fp, C.c_int]
        L.ora_argmax.restype = C.c_int
        L.ora_gemv.argtypes = [_fp, _fp, _fp, _fp, C.c_int, C.c_int]
        L.ora_gemv_add.argtypes = [_fp, _fp, _fp, C.c_int, C.c_int]
        L.ora_f16_to_f32.argtypes = [C.c_uint16]
        L.ora_f16_to_f32.restype = C.c_float
        L.ora_dequant.argtypes = [C.c_void_p, C.c_int, C.c_int64, _fp]
        L.ora_lstm_step.argtypes = [C.POINTER(OraModel), _fp, _fp, _fp, _fp, _fp]
        L.ora_joint_step.argtypes = [C.POINTER(OraModel), _fp, _fp, _fp, _fp, _fp]
        L.ora_init_state.argtypes = [C.POINTER(OraModel), C.POINTER(OraState)]
        L.ora_tdt_decode_window.argtypes = [C.POINTER(OraModel), _fp, C.c_int, C.c_int, C.c_int,
                                            C.c_float, C.POINTER(OraState), _ip, C.c_int,
                                            C.POINTER(C.c_int), C.POINTER(C.c_int), _ip, C.c_int]
        L.ora_eou_decode_window.argtypes = [C.POINTER(OraModel), _fp, C.c_int, C.c_int, C.c_int,
                                            C.c_float, C.POINTER(OraState), _ip, C.c_int,
                                            C.POINTER(C.c_int), _ip, C.c_int, C.POINTER(C.c_int),
                                            C.POINTER(C.c_int), _ip, C.c_int]
        L.ora_replay_window.argtypes = [C.POINTER(OraModel), _fp, C.c_int, C.c_int, C.c_int,
                                        C.c_float, C.POINTER(OraState), _ip, C.c_int, C.c_float,
                                        _ip, C.c_int, C.POINTER(C.c_int), _ip, C.c_int,
                                        C.POINTER(C.c_int), _fp, C.c_int,
                                        C.POINTER(OraReplayStats)]
        L.ora_decode_batch.argtypes = [C.POINTER(OraModel), C.c_int, C.POINTER(_fp), _ip, _fp,
                                       C.c_int, C.c_int, _ip, C.c_int, _ip, _ip]
        _lib = L
    return _lib


def fptr(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_fp)


def iptr(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(_ip)


class State:
    """Host decoder state (the reference's TdtDecodeState / EouDecodeState)."""

    def __init__(self, m: "OracleModel"):
        self.h = np.zeros(m.L * m.H, np.float32)
        self.c = np.zeros(m.L * m.H, np.float32)
        self.pred = np.zeros(m.H, np.float32)
        self.st = OraState(fptr(self.h), fptr(self.c), fptr(self.pred), 0, 0, 0, -1, 0)

    def copy(self, m):
        s = State(m)
        s.h[:] = self.h
        s.c[:] = self.c
        s.pred[:] = self.pred
        for k in ("symbols_this_step", "initialized", "carry_frames", "last_token",
                  "segment_start_token"):
            setattr(s.st, k, getattr(self.st, k))
        return s


class OracleModel:
    def __init__(self, weights: dict, kind: str, H: int, L: int, J: int, D: int, vocab: int,
                 blank: int | None = None, durations=None, eou_id: int = -1, eob_id: int = -1,
                 special=None, num_durations: int | None = None):
        p = "tdt" if kind == "tdt" else "eou"
        self.kind = TDT if kind == "tdt" else EOU
        self.H, self.L, self.J, self.D = H, L, J, D
        self.V1 = vocab + 1
        # duration logits: num_durations (src/parakeet_tdt.cpp:592, from
        # parakeet.tdt.num_durations), apart from the value table, which may be
        # empty (duration = logit index, src/parakeet_tdt.cpp:938-940) or longer
        if kind != "tdt":
            self.Dn = 0
        elif num_durations is not None:
            self.Dn = int(num_durations)
        else:
            self.Dn = len(durations) if durations is not None else 0
        self.Vo = self.V1 + self.Dn
        self.blank = vocab if blank is None else blank
        self._keep = []

        def arr(name):
            a = np.ascontiguousarray(weights[f"{p}.{name}"], dtype=np.float32).reshape(-1)
            self._keep.append(a)
            return fptr(a)

        m = OraModel()
        m.kind, m.H, m.L, m.J, m.D = self.kind, H, L, J, D
        m.V1, m.Dn, m.Vo, m.blank = self.V1, self.Dn, self.Vo, self.blank
        m.eou = eou_id if eou_id >= 0 else vocab - 2
        m.eob = eob_id if eob_id >= 0 else vocab - 1
        self.eou, self.eob = m.eou, m.eob
        durs = list(durations or [])
        if len(durs) > ORA_MAX_DUR or self.Dn > ORA_MAX_DUR:
            raise ValueError(f"at most {ORA_MAX_DUR} durations")
        if kind == "tdt" and 0 < len(durs) < self.Dn:
            # the reference would index past its table; the device refuses it too
            raise ValueError(f"durations table ({len(durs)}) shorter than num_durations ({self.Dn})")
        m.n_dur = len(durs) if kind == "tdt" else 0
        for i, d in enumerate(durs):
            m.durations[i] = int(d)
        m.embed = arr("predict.embed.weight")
        for l in range(L):
            m.w_ih[l] = arr(f"predict.lstm.{l}.w_ih")
            m.w_hh[l] = arr(f"predict.lstm.{l}.w_hh")
            m.b_ih[l] = arr(f"predict.lstm.{l}.b_ih")
            m.b_hh[l] = arr(f"predict.lstm.{l}.b_hh")
        m.enc_w, m.enc_b = arr("joint.enc.weight"), arr("joint.enc.bias")
        m.pred_w, m.pred_b = arr("joint.pred.weight"), arr("joint.pred.bias")
        m.out_w, m.out_b = arr("joint.out.weight"), arr("joint.out.bias")
        if special is not None:
            sp = np.ascontiguousarray(special, dtype=np.uint8)
            self._keep.append(sp)
            m.special = sp.ctypes.data_as(C.POINTER(C.c_uint8))
            m.n_special = len(sp)
        self.m = m

    @classmethod
    def from_gguf(cls, path: str, gguf_mod):
        rd = gguf_mod.GGUFReader(path)
        kv = rd.kv
        kind = kv.get("parakeet.model.type", "ctc")
        weights = {name: rd.f32(name) for name in rd.tensors}
        D = int(kv.get("parakeet.encoder.d_model", 1024))
        pieces = kv.get("tokenizer.ggml.tokens", [])
        special = np.array([1 if (len(s) > 0 and s[0] == "<" and s[-1] == ">") else 0
                            for s in pieces], np.uint8)
        if kind == "tdt":
            vocab = int(kv.get("parakeet.tdt.vocab_size", 8192))
            # src/parakeet_ctc.cpp:428-439: the count defaults to 5, an absent
            # table to {0, 1, 2, 3, 4}
            durs = kv.get("parakeet.tdt.durations")
            durs = [0, 1, 2, 3, 4] if durs is None else [int(x) for x in durs]
            return cls(weights, "tdt", int(kv.get("parakeet.tdt.pred_hidden", 640)),
                       int(kv.get("parakeet.tdt.pred_rnn_layers", 2)),
                       int(kv.get("parakeet.tdt.joint_hidden", 640)), D, vocab,
                       blank=int(kv.get("parakeet.tdt.blank_id", vocab)), durations=durs,
                       special=special, num_durations=int(kv.get("parakeet.tdt.num_durations", 5)))
        vocab = int(kv.get("parakeet.eou.vocab_size", 1026))
        return cls(weights, "eou", int(kv.get("parakeet.eou.pred_hidden", 640)),
                   int(kv.get("parakeet.eou.pred_rnn_layers", 1)),
                   int(kv.get("parakeet.eou.joint_hidden", 640)), D, vocab,
                   blank=int(kv.get("parakeet.eou.blank_id", vocab)),
                   eou_id=int(kv.get("parakeet.eou.eou_id", -1)),
                   eob_id=int(kv.get("parakeet.eou.eob_id", -1)), special=special)

    # ---- primitives ----
    def new_state(self) -> State:
        return State(self)

    def init_state(self, s: State):
        lib().ora_init_state(C.byref(self.m), C.byref(s.st))

    def lstm_step(self, x: np.ndarray, s: State):
        g = np.zeros(4 * self.H, np.float32)
        hh = np.zeros(self.H, np.float32)
        lib().ora_lstm_step(C.byref(self.m), fptr(np.ascontiguousarray(x, np.float32)),
                            s.st.h, s.st.c, fptr(g), fptr(hh))

    def joint(self, enc: np.ndarray, pred: np.ndarray) -> np.ndarray:
        hidden = np.zeros(self.J, np.float32)
        tmp = np.zeros(self.J, np.float32)
        logits = np.zeros(self.Vo, np.float32)
        lib().ora_joint_step(C.byref(self.m), fptr(np.ascontiguousarray(enc, np.float32)),
                             fptr(np.ascontiguousarray(pred, np.float32)), fptr(hidden),
                             fptr(logits), fptr(tmp))
        return logits

    # ---- decode ----
    def decode_window(self, enc: np.ndarray, s: State, max_symbols: int, blank_bias: float = 0.0,
                      token_cap: int | None = None, tokens_before: int = 0, trace: bool = False):
        """One ``*_decode_window`` call.  Returns dict(rc, tokens, steps, segments, trace)."""
        enc = np.ascontiguousarray(enc, np.float32)
        T = enc.shape[0] if enc.ndim == 2 else 0
        D = enc.shape[1] if enc.ndim == 2 else self.D
        cap = token_cap if token_cap is not None else T * max(1, max_symbols) + 1
        out = np.zeros(tokens_before + cap, np.int32)
        n_out = C.c_int(tokens_before)
        steps = C.c_int(0)
        tcap = T * (max(1, max_symbols) + 1) + 1 if trace else 0
        tr = np.zeros(2 * max(tcap, 1), np.int32)
        if self.kind == TDT:
            rc = lib().ora_tdt_decode_window(C.byref(self.m), fptr(enc), T, D, max_symbols,
                                             blank_bias, C.byref(s.st), iptr(out), len(out),
                                             C.byref(n_out), C.byref(steps),
                                             iptr(tr) if trace else None, tcap)
            segs = np.zeros(0, np.int32)
        else:
            seg = np.zeros(cap + 1, np.int32)
            n_seg = C.c_int(0)
            rc = lib().ora_eou_decode_window(C.byref(self.m), fptr(enc), T, D, max_symbols,
                                             blank_bias, C.byref(s.st), iptr(out), len(out),
                                             C.byref(n_out), iptr(seg), len(seg), C.byref(n_seg),
                                             C.byref(steps), iptr(tr) if trace else None, tcap)
            segs = seg[:n_seg.value].copy()
        res = dict(rc=rc, tokens=out[tokens_before:n_out.value].copy(), steps=steps.value,
                   segments=segs)
        if trace:
            res["trace"] = tr[:2 * min(steps.value, tcap)].reshape(-1, 2).copy()
        return res

    def replay_window(self, enc: np.ndarray, s: State, max_symbols: int, trace: np.ndarray,
                      blank_bias: float = 0.0, tie_eps: float = 1e-4, tokens_before: int = 0,
                      n_tap: int = 0):
        enc = np.ascontiguousarray(enc, np.float32)
        T = enc.shape[0]
        cap = T * max(1, max_symbols) + 1
        out = np.zeros(tokens_before + cap, np.int32)
        seg = np.zeros(cap + 1, np.int32)
        n_out, n_seg = C.c_int(tokens_before), C.c_int(0)
        tr = np.ascontiguousarray(trace, np.int32).reshape(-1)
        tap = np.zeros(max(n_tap, 1) * self.Vo, np.float32)
        stats = OraReplayStats()
        rc = lib().ora_replay_window(C.byref(self.m), fptr(enc), T, enc.shape[1], max_symbols,
                                     blank_bias, C.byref(s.st), iptr(tr), len(tr) // 2, tie_eps,
                                     iptr(out), len(out), C.byref(n_out), iptr(seg), len(seg),
                                     C.byref(n_seg), fptr(tap) if n_tap else None, n_tap,
                                     C.byref(stats))
        return dict(rc=rc, tokens=out[tokens_before:n_out.value].copy(),
                    segments=seg[:n_seg.value].copy(), stats=stats.as_dict(),
                    logits=tap[:n_tap * self.Vo].reshape(n_tap, self.Vo) if n_tap else None)

    def decode_batch(self, encs: list, max_symbols: int, blank_bias=None, n_threads: int = 1):
        n = len(encs)
        encs = [np.ascontiguousarray(e, np.float32) for e in encs]
        T = np.array([e.shape[0] for e in encs], np.int32)
        cap = int(T.max()) * max(1, max_symbols) + 1 if n else 1
        ptrs = (_fp * n)(*[fptr(e) for e in encs])
        toks = np.zeros(n * cap, np.int32)
        ntok = np.zeros(n, np.int32)
        steps = np.zeros(n, np.int32)
        bb = np.ascontiguousarray(blank_bias, np.float32) if blank_bias is not None else None
        rc = lib().ora_decode_batch(C.byref(self.m), n, ptrs, iptr(T),
                                    fptr(bb) if bb is not None else None, max_symbols, n_threads,
                                    iptr(toks), cap, iptr(ntok), iptr(steps))
        toks = toks.reshape(n, cap)
        return dict(rc=rc, tokens=[toks[u, :ntok[u]].copy() for u in range(n)], steps=steps)
