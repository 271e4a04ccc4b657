"""Algorithmic bytes and flops of the greedy-decode loop, per lockstep iteration.

Unit of work: one decode step = one joint evaluation for one utterance (the
reference's out_steps counter, src/parakeet_tdt.cpp:936).  In lockstep
iteration i, A_j utterances evaluate the joint and A_l run the prediction
LSTM (after a non-blank emission, an EOU reset, or at initialisation):

  bytes_i = [A_j>0] (W(joint.pred) + W(joint.out) + biases)
          + [A_l>0] (W(LSTM, all layers) + biases)
          + A_l * row(embed) + A_j * 4 J            (enc_proj row, f32)
          + A_l * 2 L H * 4 * 2                     (h, c read + write, f32)
  flops_i = A_j * 2 J (H + Vo) + A_l * 2 L 4H (H + H)

and once per utterance the encoder-side projection:
  bytes = W(joint.enc) + 4 T D + 4 T J,   flops = 2 T D J.

W(.) is the stored size: q8_0 34 bytes per 32 weights, f16 2, f32 4.
"""
from __future__ import annotations

import numpy as np

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s
FP32_PEAK_TFLOPS = 157.3       # MI355X fp32 (vector and matrix), TFLOP/s


BLOCK_BYTES = {8: 34, 6: 22, 2: 18}   # q8_0, q5_0, q4_0: bytes per 32 stored weights


def wbytes(rows: int, cols: int, ggml_type: int) -> int:
    """Stored bytes of a matrix: the algorithmic weight bytes (q8_0 34, q5_0 22, q4_0 18
    bytes per 32 weights).  The device reads q5_0 / q4_0 matrices as their exact q8_0
    repacking, 34 bytes per 32 weights, so its weight reads for those types exceed these."""
    if ggml_type in BLOCK_BYTES:
        return rows * (cols // 32) * BLOCK_BYTES[ggml_type]
    return rows * cols * (2 if ggml_type == 1 else 4)


class DecoderCost:
    def __init__(self, info, types: dict):
        """info: pk.DecoderInfo; types: ggml type per matrix role
        ('embed', 'lstm', 'pred', 'out', 'enc')."""
        H, L, J, Vo, D = info.H, info.L, info.J, info.Vo, info.D
        self.info = info
        self.joint_w = wbytes(J, H, types["pred"]) + wbytes(Vo, J, types["out"]) + 4 * (J + Vo)
        self.lstm_w = L * (2 * wbytes(4 * H, H, types["lstm"]) + 2 * 4 * 4 * H)
        self.embed_row = wbytes(1, H, types["embed"])
        self.enc_w = wbytes(J, D, types["enc"]) + 4 * J
        self.H, self.L, self.J, self.Vo, self.D = H, L, J, Vo, D

    def iteration(self, A_j: np.ndarray, A_l: np.ndarray):
        A_j = np.asarray(A_j, np.float64)
        A_l = np.asarray(A_l, np.float64)
        b = ((A_j > 0) * self.joint_w + (A_l > 0) * self.lstm_w + A_l * self.embed_row
             + A_j * 4 * self.J + A_l * 2 * self.L * self.H * 4 * 2)
        f = A_j * 2 * self.J * (self.H + self.Vo) + A_l * 2 * self.L * 4 * self.H * (2 * self.H)
        return b, f

    def enc_proj(self, total_frames: int):
        return (self.enc_w + 4 * total_frames * (self.D + self.J),
                2.0 * total_frames * self.D * self.J)


def lockstep_counts(traces: list, kind: int, blank: int, eou: int = -1, eob: int = -1,
                    special=None, fresh: bool = True):
    """Per-iteration (A_j, A_l) of one batched launch, reconstructed from the
    per-step decisions: step s of an utterance runs in iteration s+1, and a
    step that emits (or resets the EOU state) puts an LSTM update in the next
    iteration.  Fresh slots run the initial LSTM in iteration 1."""
    n_it = max((len(t) for t in traces), default=0) + 2
    A_j = np.zeros(n_it + 1, np.int64)
    A_l = np.zeros(n_it + 1, np.int64)
    for tr in traces:
        if fresh:
            A_l[1] += 1
        s = len(tr)
        A_j[1:s + 1] += 1
        toks = np.asarray(tr)[:, 0] if s else np.zeros(0, np.int64)
        if kind == 0:
            emit = toks != blank
        else:
            sp = np.zeros(len(toks), bool)
            if special is not None and len(special):
                inr = (toks >= 0) & (toks < len(special))
                sp[inr] = np.asarray(special)[toks[inr]] != 0
            emit = (toks != blank) & (toks != eob) & ~sp        # emit or EOU reset
        idx = np.nonzero(emit)[0] + 2
        np.add.at(A_l, idx, 1)
    last = int(max(np.max(np.nonzero(A_j)[0], initial=0), np.max(np.nonzero(A_l)[0], initial=0)))
    return A_j[1:last + 1], A_l[1:last + 1]


def _pmc_rows(path: str, counter: str):
    import csv
    with open(path, newline="") as f:
        return [r for r in csv.DictReader(f) if r.get("Counter_Name") == counter]


def pmc_traffic(fetch_csv: str, write_csv: str, kernel: str = "decode_loop_kernel",
                probe: str = "calib_copy_kernel", probe_bytes: int = 256 << 20):
    """HBM bytes per launch of `kernel` from two rocprofv3 --pmc runs
    (FETCH_SIZE, then WRITE_SIZE; counter_collection.csv, values in KiB per
    dispatch), each scaled so that the copy kernel of the same run reads
    `probe_bytes` read and `probe_bytes` written.  Returns a dict."""
    out = {}
    for name, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        rows = _pmc_rows(path, name)
        cal = [float(r["Counter_Value"]) for r in rows if probe in r["Kernel_Name"]]
        vals = [float(r["Counter_Value"]) for r in rows if kernel in r["Kernel_Name"]]
        if not cal or not vals:
            raise ValueError(f"{path}: no {probe} or {kernel} dispatch with {name}")
        factor = probe_bytes / (cal[0] * 1024.0)
        out[name] = {"kib_per_dispatch": float(np.mean(vals)), "copy_kib": cal[0], "factor": factor,
                     "bytes_per_launch": float(np.mean(vals)) * 1024.0 * factor}
    out["bytes_per_launch"] = out["FETCH_SIZE"]["bytes_per_launch"] + out["WRITE_SIZE"]["bytes_per_launch"]
    return out
