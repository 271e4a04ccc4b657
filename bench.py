#!/usr/bin/env python3
"""Benchmark: TDT greedy decode steps/s on one MI355X.

Workload (one bench step = one batched decode call, inputs resident in HBM):
TDT-0.6b-v3-shaped decoder, q8_0 weights (seeded random, GGUF decoder
layout), B=64 independent utterances of T=750 encoder frames each (fp32
N(0,1), 1024-d, seed 1000+u), max_symbols_per_step 10, every utterance
decoded in lockstep with on-device compaction.  A decode step is one joint
evaluation for one utterance (the reference's out_steps counter).

Prints one JSON line.  Extra fields: the roofline of the dominant kernel (the
decode loop), the CPU baseline (the oracle, a C restatement of the
reference's scalar decoder, timed on this host on a bounded sample), and the
other workload shapes (--no-extras skips them):
  b1                 B=1, T=125 on the same decoder: latency per step
  b1_cpp             the same utterance through the drop-in tdt_greedy_decode (the reference
                     CLI's call), wall time per call and per step, host overhead included
  eou_stream_cpp     the EOU streaming workload below through the C++ API
                     (eou_decode_batch_device over device frames, states carried), wall
                     time per chunk call
  b1_blank4          the same with the blank logit raised by 4 (blank-dominated decoding, as a
                     trained model's is): latency per step with runs of blanks walked over
                     the joint tile's spare columns, and without them (PK_SPEC=0)
  b256               B=256, T=750 on the same decoder
  ragged_b512        B=512, T ~ U{50..1500}, blank-logit offsets {0, +2, +4}
  tdt11b_f16_b256    TDT-1.1b shapes (vocab 1024), f16 weights, B=256, T=375
  eou_stream_b128    EOU-120m shapes, q8_0, 128 sessions x 40 chunks of 2 frames,
                     state carried between chunk calls
Each carries its own roofline ratio (roofline time of its lockstep
iterations over the measured loop time).

roofline.traffic (HBM bytes per launch of the decode loop) comes from two
rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) that the default run makes in
child processes before it touches the GPU, each one step of the same workload
with a 256 MiB copy for calibration (--no-traffic skips them).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)


EXTRAS = ("b1", "b1_blank4", "b256", "ragged_b512", "tdt11b_f16_b256", "eou_stream_b128")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--frames", type=int, default=750)
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", choices=EXTRAS, default=None,
                    help="run one of the other workload shapes alone and print its result (for per-workload "
                         "kernel traces); the metric line is not produced")
    ap.add_argument("--cpu-utts", type=int, default=64)
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="first run a plain device copy of MIB MiB (calibrates hardware byte counters)")
    ap.add_argument("--traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="counter_collection.csv of two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) of "
                         "this bench with --copy-probe 256: fills roofline.traffic")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 --pmc passes the default run makes for roofline.traffic")
    return ap.parse_args()


def traffic_passes(args) -> tuple[list[str] | None, str | None]:
    """HBM traffic of the decode loop at this workload: two rocprofv3 --pmc
    passes (FETCH_SIZE, then WRITE_SIZE), each a child process running this
    bench for one step with the copy calibration (--copy-probe 256), started
    before this process touches the GPU.  Returns the two counter CSVs, or
    None and the reason they are missing (no rocprofv3, already under a
    profiler, or a failed pass)."""
    import glob
    import shutil
    import subprocess
    exe = shutil.which("rocprofv3")
    if exe is None:
        return None, "rocprofv3 not found"
    if any(k.startswith("ROCPROF") for k in os.environ) or "rocprof" in os.environ.get("LD_PRELOAD", ""):
        return None, "already running under a profiler"
    out = tempfile.mkdtemp(prefix="pk_traffic_", dir="/tmp")
    # (under the profiler the library launches the loop as an ordinary dispatch by itself)
    env = dict(os.environ, TMPDIR="/tmp")
    csvs = []
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        d = os.path.join(out, ctr)
        cmd = ["timeout", "-s", "KILL", "180", exe, "--pmc", ctr, "--output-format", "csv", "-d", d, "-o", "c",
               "--", sys.executable, os.path.abspath(__file__), "--batch", str(args.batch), "--frames",
               str(args.frames), "--steps", "1", "--warmup", "0", "--no-extras", "--no-cpu", "--no-traffic",
               "--copy-probe", "256"]
        print(f"[bench] traffic pass {ctr}", file=sys.stderr, flush=True)
        r = subprocess.run(cmd, cwd="/tmp", env=env, stdout=subprocess.DEVNULL, stderr=subprocess.PIPE,
                           text=True, errors="replace")
        found = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
        if r.returncode != 0 or not found:
            return None, f"{ctr} pass failed (status {r.returncode}): {r.stderr[-300:]}"
        csvs.append(found[0])
    return csvs, None


def cpp_b1(frames=125, reps=30):
    """B=1 latency through the reference's own decoder interface: the drop-in
    tdt_greedy_decode (include/dropin/parakeet_tdt.h, the call the reference CLI
    makes, src/main.cpp:745-761) on the TDT-0.6b-v3 q8_0 decoder, one 125-frame
    utterance, timed by tests/cpp/dropin_main --bench in a child process started
    before this process touches the GPU.  Wall time per call includes the frame
    upload, enc_proj, the decode loop and the output copies."""
    import subprocess
    exe = os.path.join(ROOT, "tests", "cpp", "dropin_main")
    if not os.path.exists(exe):
        return {"missing": "tests/cpp/dropin_main is built only where parakeet.cpp's sources are present"}
    import __graft_entry__ as graft
    graft.load_package()
    from parakeet_amd import synth
    tmp = tempfile.mkdtemp(prefix="pk_cpp_")
    path = os.path.join(tmp, "tdt-0.6b-v3-q8_0.gguf")
    synth.make_shape(path, "tdt-0.6b-v3")
    fpath = os.path.join(tmp, "frames.bin")
    enc = synth.encoder_frames(0, frames, 1024)
    with open(fpath, "wb") as f:
        np.array([1, frames, 1024], np.int32).tofile(f)
        enc.astype(np.float32).tofile(f)
    print("[bench] b1_cpp: drop-in tdt_greedy_decode", file=sys.stderr, flush=True)
    r = subprocess.run(["timeout", "-k", "10", "120", exe, "--bench", path, fpath, str(reps)], capture_output=True,
                       text=True, errors="replace")
    if r.returncode != 0:
        return {"missing": f"dropin_main --bench failed (status {r.returncode}): {r.stderr[-300:]}"}
    d = json.loads(r.stdout.strip().splitlines()[-1])
    steps = max(1, d["steps"])
    return {"api": "drop-in tdt_greedy_decode (host frames, host outputs)", "frames": frames, "steps": d["steps"],
            "us_per_call": d["call_us"], "us_per_call_min": d["call_us_min"],
            "us_per_step_wall": round(d["call_us"] / steps, 3),
            "kernel_us_per_call": d["kernel_us"],
            "host_us_per_call": round(d["call_us_timed"] - d["kernel_us"], 3),
            "note": "wall with the handle's timing events off, as the drop-in runs; kernel and host "
                    "shares from a second pass with them on",
            "reps": d["reps"]}


def cpp_eou_stream(B=128, chunks=40, F=2):
    """The EOU streaming workload of eou_stream_extra (EOU-120m shapes, q8_0, B
    sessions x `chunks` chunks of F frames, the same frames) through the C++ API:
    tests/cpp/decoder_api_main --bench-eou-stream, one eou_decode_batch_device call
    per chunk over the encoder output in device memory, with the session states
    carried, in a child process started before this process touches the GPU."""
    import subprocess
    exe = os.path.join(ROOT, "tests", "cpp", "decoder_api_main")
    if not os.path.exists(exe):
        return {"missing": "tests/cpp/decoder_api_main is not built"}
    import __graft_entry__ as graft
    graft.load_package()
    from parakeet_amd import synth
    tmp = tempfile.mkdtemp(prefix="pk_cpp_")
    path = os.path.join(tmp, "eou-120m-q8_0.gguf")
    synth.make_shape(path, "eou-120m")
    D = 512
    fpath = os.path.join(tmp, "frames.bin")
    with open(fpath, "wb") as f:
        np.array([B, chunks * F, D], np.int32).tofile(f)
        for u in range(B):
            synth.encoder_frames(u, chunks * F, D).astype(np.float32).tofile(f)
    print("[bench] eou_stream_cpp: eou_decode_batch_device", file=sys.stderr, flush=True)
    r = subprocess.run(["timeout", "-k", "10", "120", exe, "--bench-eou-stream", path, fpath, str(F)],
                       capture_output=True, text=True, errors="replace")
    if r.returncode != 0:
        return {"missing": f"decoder_api_main --bench-eou-stream failed (status {r.returncode}): {r.stderr[-300:]}"}
    d = json.loads(r.stdout.strip().splitlines()[-1])
    return {"api": "C++ eou_decode_batch_device (device frames, host outputs, states carried)",
            "sessions": d["sessions"], "chunks": d["chunks"], "frames_per_chunk": d["frames_per_chunk"],
            "decode_steps": d["steps"], "tokens": d["tokens"], "us_per_chunk_call": d["call_us"],
            "us_per_chunk_call_min": d["call_us_min"]}


class Workload:
    """Utterances of Ts[u] frames resident on the device (packed rows), with
    output buffers and fresh state slots for every call."""

    def __init__(self, pk, hipmem, dec, Ts, D, max_sym, n_calls, slot_base, first_seed=1000,
                 blank_bias=None):
        from parakeet_amd import synth
        self.pk, self.hm, self.dec = pk, hipmem, dec
        self.Ts = np.ascontiguousarray(Ts, np.int32)
        self.B, self.max_sym = len(self.Ts), max_sym
        self.rows = np.concatenate([[0], np.cumsum(self.Ts, dtype=np.int64)[:-1]]).astype(np.int64)
        frames = np.empty((int(self.Ts.sum()), D), np.float32)
        for u in range(self.B):
            r, t = int(self.rows[u]), int(self.Ts[u])
            frames[r:r + t] = synth.encoder_frames(u, t, D, base_seed=first_seed)
        self.enc = hipmem.DeviceArray.from_numpy(frames)
        del frames
        T = int(self.Ts.max())
        self.cap = T * max(1, max_sym) + 1
        self.tcap = T * (max(1, max_sym) + 1) + 1
        self.out = dict(tokens=hipmem.DeviceArray(4 * self.B * self.cap), n_tokens=hipmem.DeviceArray(4 * self.B),
                        steps=hipmem.DeviceArray(4 * self.B))
        self.trace = hipmem.DeviceArray(8 * self.B * self.tcap)
        self.blank_bias = blank_bias
        self.calls = 0
        self.n_calls = n_calls
        self.slot_base = slot_base
        assert slot_base + self.B * n_calls <= dec.n_slots

    def run(self, trace=False):
        assert self.calls < self.n_calls, "every call decodes fresh slots"
        slots = np.arange(self.B, dtype=np.int32) + self.slot_base + self.calls * self.B
        self.calls += 1
        if trace:
            self.traced_slots = slots
        ptrs = {k: v.ptr for k, v in self.out.items()}
        if trace:
            ptrs["trace"] = self.trace.ptr
        self.dec.decode_device(self.enc.ptr, self.rows, self.Ts, slots, self.max_sym, ptrs, self.cap,
                               blank_bias=self.blank_bias, trace_cap=self.tcap if trace else 0)

    def steps(self):
        return self.out["steps"].to_numpy(np.int32, self.B)

    def traces(self):
        st = self.steps()
        tr = self.trace.to_numpy(np.int32, self.B * self.tcap * 2).reshape(self.B, self.tcap, 2)
        return [tr[u, :st[u]] for u in range(self.B)]

    def free(self):
        for a in (self.enc, self.trace, *self.out.values()):
            a.free()


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def sampled_parity(om, wl, traces, encs_of, sample, max_symbols):
    """Teacher-forced oracle replay of a sample of the workload's utterances
    (decisions from the traced call): unexplained mismatches, near-ties, and
    the worst L2-relative error of the final h and c against the oracle."""
    from concurrent.futures import ThreadPoolExecutor
    sample = [u for u in sample if u < wl.B]

    def one(u):
        st = om.new_state()
        rep = om.replay_window(encs_of(u), st, max_symbols, traces[u], tie_eps=1e-4)
        return u, rep, st
    with ThreadPoolExecutor(len(sample)) as ex:
        reps = list(ex.map(one, sample))
    unexplained = near = 0
    worst = 0.0
    for u, rep, st in reps:
        unexplained += rep["stats"]["unexplained"] + rep["stats"]["structure_error"]
        near += rep["stats"]["near_ties"]
        d = wl.dec.read_state(int(wl.traced_slots[u]))
        for a, b in ((d["h"], st.h), (d["c"], st.c)):
            worst = max(worst, float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)))
    return {"utterances": list(sample), "steps": int(sum(len(traces[u]) for u in sample)),
            "unexplained_mismatches": int(unexplained), "near_ties": int(near),
            "tie_eps": 1e-4, "max_state_rel_err": float(f"{worst:.3e}")}


def untimed_wall(wl, warmup, steps):
    """Wall seconds of `steps` calls with the decoder's timing events off, as a
    latency-bound caller runs it (the events add a few microseconds per call)."""
    wl.dec.set_timing(False)
    try:
        for _ in range(warmup):
            wl.run()
        wl.hm.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            wl.run()
        wl.hm.synchronize()
        return time.perf_counter() - t0
    finally:
        wl.dec.set_timing(True)


def timed(wl, warmup, steps):
    for _ in range(warmup):
        wl.run()
    wl.hm.synchronize()
    loop_ms, enc_ms, iters = [], [], []
    t0 = time.perf_counter()
    for _ in range(steps):
        wl.run()
        t = wl.dec.last_timing()
        loop_ms.append(t["loop_ms"])
        enc_ms.append(t["enc_proj_ms"])
        iters.append(t["iterations"])
    wl.hm.synchronize()
    wall = time.perf_counter() - t0
    return wall, float(np.mean(loop_ms)), float(np.mean(enc_ms)), int(np.max(iters))


def matrix_types(rd, pfx):
    t = rd.tensors
    return dict(embed=t[f"{pfx}.predict.embed.weight"].ggml_type, lstm=t[f"{pfx}.predict.lstm.0.w_ih"].ggml_type,
                pred=t[f"{pfx}.joint.pred.weight"].ggml_type, out=t[f"{pfx}.joint.out.weight"].ggml_type,
                enc=t[f"{pfx}.joint.enc.weight"].ggml_type)


def roof_time(roofline, cost, A_j, A_l):
    """Roofline time of the given lockstep iterations: (seconds, binding resource)."""
    b, f = cost.iteration(A_j, A_l)
    tb, tf = b / (roofline.HBM_PEAK_GBS * 1e9), f / (roofline.BF16_PEAK_TFLOPS * 1e12)
    return float(np.maximum(tb, tf).sum()), ("hbm" if tb.sum() >= tf.sum() else "mfma")


def lockstep_extra(pk, hipmem, roofline, dec, cost, Ts, D, MS, slot_base, blank_bias=None, timed_calls=2):
    """One traced call (decisions for the cost model), one warm-up call, then
    `timed_calls` timed calls of the same batch on fresh slots."""
    wl = Workload(pk, hipmem, dec, Ts, D, MS, timed_calls + 2, slot_base, blank_bias=blank_bias)
    wl.run(trace=True)
    A_j, A_l = roofline.lockstep_counts(wl.traces(), 0, dec.info.blank)
    t_roof, bound = roof_time(roofline, cost, A_j, A_l)
    wall, loop, enc, iters = timed(wl, 1, timed_calls)
    st = int(wl.steps().sum())
    wl.free()
    return {"utterances": len(Ts), "frames_total": int(np.sum(Ts)), "decode_steps": st,
            "steps_per_s": round(st * timed_calls / wall, 1), "loop_ms": round(loop, 3),
            "enc_proj_ms": round(enc, 3), "iterations": iters,
            "us_per_iteration": round(loop * 1e3 / max(1, iters), 3),
            "roofline": {"bound": bound, "t_roof_over_t_kernel": round(t_roof / (loop * 1e-3), 5)}}


def eou_stream_extra(pk, hipmem, roofline, gguf, synth, tmp, B=128, chunks=40, F=2):
    """EOU-120m-shaped q8_0 decoder: B sessions fed `chunks` chunks of F frames,
    state carried in the slots.  Frames are resident in HBM; each chunk call
    reads its token counts back (the caller needs them for the next call's
    segment base), and that copy is inside the timed wall.  The stream runs
    three times: traced (decisions for the cost model), with the timing events
    on (kernel times), and with them off (the wall per call, as a latency-bound
    caller runs it)."""
    path = os.path.join(tmp, "eou-120m-q8_0.gguf")
    synth.make_shape(path, "eou-120m")
    rd = gguf.GGUFReader(path)
    dec = pk.Decoder(rd, n_slots=3 * B)
    info = dec.info
    cost = roofline.DecoderCost(info, matrix_types(rd, "eou"))
    MS, D = info.max_symbols, info.D
    frames = np.empty((B * chunks * F, D), np.float32)
    for u in range(B):
        frames[u * chunks * F:(u + 1) * chunks * F] = synth.encoder_frames(u, chunks * F, D)
    enc = hipmem.DeviceArray.from_numpy(frames)
    del frames
    cap, tcap, scap = F * max(1, MS) + 1, F * (max(1, MS) + 1) + 1, F * max(1, MS) + 2
    tok = hipmem.DeviceArray(4 * B * cap * chunks)
    seg = hipmem.DeviceArray(4 * B * scap * chunks)
    steps = hipmem.DeviceArray(4 * B * chunks)
    nseg = hipmem.DeviceArray(4 * B * chunks)
    ntok = [hipmem.DeviceArray(4 * B) for _ in range(chunks)]
    tr = hipmem.DeviceArray(8 * B * tcap * chunks)
    Ts = np.full(B, F, np.int32)

    def stream(slot_base, trace, timing=True):
        total = np.zeros(B, np.int32)
        loop = enc_ms = 0.0
        slots = np.arange(B, dtype=np.int32) + slot_base
        for c in range(chunks):
            rows = np.arange(B, dtype=np.int64) * chunks * F + c * F
            ptrs = dict(tokens=tok.ptr + 4 * B * cap * c, n_tokens=ntok[c].ptr, steps=steps.ptr + 4 * B * c,
                        segments=seg.ptr + 4 * B * scap * c, seg_cap=scap, n_segments=nseg.ptr + 4 * B * c)
            if trace:
                ptrs["trace"] = tr.ptr + 8 * B * tcap * c
            dec.decode_device(enc.ptr, rows, Ts, slots, MS, ptrs, cap, trace_cap=tcap if trace else 0,
                              tokens_base=total)
            total += ntok[c].to_numpy(np.int32, B)
            if timing:
                t = dec.last_timing()
                loop += t["loop_ms"]
                enc_ms += t["enc_proj_ms"]
        return total, loop, enc_ms

    stream(0, True)                                        # untimed: decisions for the cost model
    st = steps.to_numpy(np.int32, B * chunks).reshape(chunks, B)
    trs = tr.to_numpy(np.int32, chunks * B * tcap * 2).reshape(chunks, B, tcap, 2)
    t_roof, bound = 0.0, "hbm"
    for c in range(chunks):
        A_j, A_l = roofline.lockstep_counts([trs[c, u, :st[c, u]] for u in range(B)], 1, info.blank,
                                            info.eou_id, info.eob_id, info.special, fresh=(c == 0))
        t, bound = roof_time(roofline, cost, A_j, A_l)
        t_roof += t
    hipmem.synchronize()
    t0 = time.perf_counter()
    total, loop, enc_ms = stream(B, False)
    wall_timed = time.perf_counter() - t0
    dec.set_timing(False)
    hipmem.synchronize()
    t0 = time.perf_counter()
    total, _, _ = stream(2 * B, False, timing=False)
    wall = time.perf_counter() - t0
    n_steps = int(steps.to_numpy(np.int32, B * chunks).sum())
    for a in (enc, tok, seg, steps, nseg, tr, *ntok):
        a.free()
    dec.close()
    return {"sessions": B, "chunks": chunks, "frames_per_chunk": F, "decode_steps": n_steps,
            "tokens": int(total.sum()), "steps_per_s": round(n_steps / wall, 1),
            "us_per_chunk_call": round(wall / chunks * 1e6, 1),
            "us_per_chunk_call_timing_events": round(wall_timed / chunks * 1e6, 1),
            "loop_ms_per_call": round(loop / chunks, 4), "enc_proj_ms_per_call": round(enc_ms / chunks, 4),
            "roofline": {"bound": bound, "t_roof_over_t_kernel": round(t_roof / (loop * 1e-3), 5)}}


def run_extra(name, pk, hipmem, roofline, gguf, synth, dec, cost, tmp, D, MS, base, n_b1):
    """One of the other workload shapes on the q8_0 0.6b decoder `dec` (slots from `base` on),
    or on a decoder of its own."""
    if name == "b1":
        # B=1, T=125 (10 s of audio): per-step latency
        wl1 = Workload(pk, hipmem, dec, np.full(1, 125), D, MS, n_b1, base)
        wall1, loop1, enc1, it1 = timed(wl1, 2, 20)
        st1 = int(wl1.steps().sum())
        wall1u = untimed_wall(wl1, 2, 20)
        wl1.free()
        return {"frames": 125, "decode_steps": st1, "us_per_step_loop": round(loop1 * 1e3 / st1, 3),
                "us_per_step_incl_enc_proj": round((loop1 + enc1) * 1e3 / st1, 3),
                "us_per_step_wall": round(wall1u / 20 * 1e6 / st1, 3),
                "us_per_step_wall_timing_events": round(wall1 / 20 * 1e6 / st1, 3)}
    base += n_b1
    if name == "b1_blank4":
        res = {}
        for label, env in (("", None), ("_without_runs", "0")):
            if env is not None:
                os.environ["PK_SPEC"] = env
            try:
                wlb = Workload(pk, hipmem, dec, np.full(1, 125), D, MS, n_b1, base,
                               blank_bias=np.full(1, 4.0, np.float32))
                wallb, loopb, encb, itb = timed(wlb, 2, 20)
                stb = int(wlb.steps().sum())
                wlb.free()
            finally:
                os.environ.pop("PK_SPEC", None)
            base += n_b1
            res["us_per_step_loop" + label] = round(loopb * 1e3 / stb, 3)
            res["iterations" + label] = itb
        res.update(frames=125, blank_bias=4.0, decode_steps=stb)
        return res
    base += 2 * n_b1
    if name == "b256":
        # B=256, T=750: lockstep throughput on the same decoder
        return lockstep_extra(pk, hipmem, roofline, dec, cost, np.full(256, 750), D, MS, base)
    base += 256 * 4
    if name == "ragged_b512":
        # B=512, T ~ U{50..1500}, blank-logit offsets {0, +2, +4}
        Tr = synth.ragged_lengths(512)
        return lockstep_extra(pk, hipmem, roofline, dec, cost, Tr, D, MS, base, blank_bias=synth.blank_offsets(512))
    if name == "tdt11b_f16_b256":
        # TDT-1.1b shapes, f16 weights, B=256, T=375
        p11 = os.path.join(tmp, "tdt-1.1b-f16.gguf")
        synth.make_shape(p11, "tdt-1.1b")
        rd11 = gguf.GGUFReader(p11)
        dec11 = pk.Decoder(rd11, n_slots=256 * 4)
        cost11 = roofline.DecoderCost(dec11.info, matrix_types(rd11, "tdt"))
        r = lockstep_extra(pk, hipmem, roofline, dec11, cost11, np.full(256, 375), dec11.info.D, MS, 0)
        dec11.close()
        return r
    if name == "eou_stream_b128":
        # EOU-120m shapes, q8_0: 128 sessions x 40 chunks of 2 frames, state carried
        return eou_stream_extra(pk, hipmem, roofline, gguf, synth, tmp)
    raise ValueError(name)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: the decode path shards as independent "
                                   "utterances per GPU with no collective, and only --gpus 1 is run"}))
        sys.exit(2)
    traffic_csvs, traffic_note = None, None
    if args.traffic:
        traffic_csvs = list(args.traffic)
    elif not (args.no_traffic or args.no_extras or args.only):
        traffic_csvs, traffic_note = traffic_passes(args)
    b1_cpp = eou_cpp = None
    if not (args.no_extras or args.only):
        b1_cpp = cpp_b1()
        eou_cpp = cpp_eou_stream()
    import __graft_entry__ as graft
    graft.load_package()
    from parakeet_amd import gguf, hipmem, pk, roofline, synth

    copy_probe = None
    if args.copy_probe > 0:
        import ctypes
        lib = ctypes.CDLL(os.path.join(ROOT, "parakeet.cpp_amd", "libpk_calib.so"))
        lib.pk_calib_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
        nbytes = args.copy_probe << 20
        src, dst = hipmem.DeviceArray(nbytes), hipmem.DeviceArray(nbytes)
        src.zero()
        rc = lib.pk_calib_copy(dst.ptr, src.ptr, nbytes)
        if rc != 0:
            raise RuntimeError(f"pk_calib_copy failed: {rc}")
        src.free()
        dst.free()
        copy_probe = {"kernel": "calib_copy_kernel", "bytes_read": nbytes, "bytes_written": nbytes}

    B, T, D, MS = args.batch, args.frames, 1024, 10
    tmp = tempfile.mkdtemp()
    path = os.path.join(tmp, "tdt-0.6b-v3-q8_0.gguf")
    synth.make_shape(path, "tdt-0.6b-v3")
    rd = gguf.GGUFReader(path)
    n_calls = args.warmup + args.steps + 1
    n_b1 = 48
    dec = pk.Decoder(rd, n_slots=B * n_calls + (0 if args.no_extras and not args.only else 3 * n_b1 + 256 * 4 + 512 * 4))
    info = dec.info
    cost = roofline.DecoderCost(info, matrix_types(rd, "tdt"))

    if args.only:
        r = run_extra(args.only, pk, hipmem, roofline, gguf, synth, dec, cost, tmp, D, MS, B * n_calls, n_b1)
        print(json.dumps({"workload": args.only, **r}), flush=True)
        dec.close()
        return

    wl = Workload(pk, hipmem, dec, np.full(B, T), D, MS, n_calls, 0)
    wl.run(trace=True)                                     # untimed: decisions for the cost model
    traces = wl.traces()
    steps_per_call = int(sum(len(t) for t in traces))
    A_j, A_l = roofline.lockstep_counts(traces, 0, info.blank)
    bytes_i, flops_i = cost.iteration(A_j, A_l)
    wall, loop_ms, enc_ms, iters = timed(wl, args.warmup, args.steps)
    assert int(wl.steps().sum()) == steps_per_call
    ms_per_step = wall * 1e3 / args.steps
    value = steps_per_call * args.steps / wall

    alg_bytes = float(bytes_i.sum())
    alg_flops = float(flops_i.sum())
    achieved_gbs = alg_bytes / (loop_ms * 1e-3) / 1e9
    t_roof = float(np.maximum(bytes_i / (roofline.HBM_PEAK_GBS * 1e9),
                              flops_i / (roofline.BF16_PEAK_TFLOPS * 1e12)).sum())
    enc_bytes, enc_flops = cost.enc_proj(B * T)

    out = {
        "metric": "TDT greedy decode steps/sec (B=64 utterances x 750 frames, TDT-0.6b-v3 q8_0)",
        "value": round(value, 1),
        "unit": "decode steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded random-init decoder weights, fp32 N(0,1) encoder frames)",
        "config": {"workload": "tdt-0.6b-v3 q8_0 greedy decode", "batch_utterances": B,
                   "frames_per_utterance": T, "d_enc": D, "max_symbols_per_step": MS,
                   "decode_steps_per_call": steps_per_call, "lockstep_iterations": iters},
        "roofline": {"bound": "hbm", "achieved": round(achieved_gbs, 2), "peak": roofline.HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved_gbs / roofline.HBM_PEAK_GBS, 5),
                     "traffic": None,
                     "kernel": "decode_loop_kernel",
                     "kernel_ms": round(loop_ms, 4),
                     "algorithmic_bytes_per_launch": alg_bytes,
                     "algorithmic_flops_per_launch": alg_flops,
                     "t_roof_over_t_kernel": round(t_roof / (loop_ms * 1e-3), 5)},
        "enc_proj": {"kernel_ms": round(enc_ms, 4),
                     "achieved_tflops": round(enc_flops / (enc_ms * 1e-3) / 1e12, 3) if enc_ms > 0 else None,
                     "algorithmic_bytes": enc_bytes, "algorithmic_flops": enc_flops},
    }

    if copy_probe:
        out["copy_probe"] = copy_probe
    if traffic_csvs:
        tr = roofline.pmc_traffic(*traffic_csvs)
        out["roofline"]["traffic"] = round(tr["bytes_per_launch"], 0)
        out["roofline"]["traffic_detail"] = {
            k: {"kib_per_dispatch": round(v["kib_per_dispatch"], 1), "copy_factor": round(v["factor"], 4)}
            for k, v in tr.items() if k != "bytes_per_launch"}
        out["roofline"]["traffic_detail"]["source"] = ("rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, one pass each, "
                                                       "one step of this workload, scaled by a 256 MiB copy")
    elif traffic_note:
        out["roofline"]["traffic_detail"] = {"missing": traffic_note}

    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle
        om = oracle.OracleModel.from_gguf(path, gguf)
        nu = min(args.cpu_utts, B)
        host_cpus = os.cpu_count() or 1
        # the reference CLI runs one decoder per hardware thread (std::thread::hardware_concurrency,
        # src/main.cpp:57); the GPU box grants this process a 16-thread CPU share (OMP_NUM_THREADS)
        share = int(os.environ.get("OMP_NUM_THREADS", "16") or 16)
        threads = max(1, min(share, host_cpus, nu))
        encs = [synth.encoder_frames(u, T, D) for u in range(nu)]
        t0 = time.perf_counter()
        r = om.decode_batch(encs, MS, n_threads=threads)
        dt = time.perf_counter() - t0
        cpu_steps = int(np.sum(r["steps"]))
        out["cpu_baseline"] = {"value": round(cpu_steps / dt, 1), "unit": "decode steps/s", "cores": threads,
                               "kind": "port",
                               "sample": f"all {nu} of the {B} utterances (full {T} frames each), "
                                         f"{cpu_steps} steps in {dt:.2f} s, one utterance per thread task on "
                                         f"{threads} threads, oracle built with -O3 -ffast-math -funroll-loops",
                               "host_cpus": host_cpus, "cpu_model": cpu_model()}
        # the same utterances decoded on the device emit the same tokens
        # every utterance's full token sequence against the device's (free-running on both
        # sides: a differing utterance would need a near-tie, which the parity sample counts)
        dev_n = wl.out["n_tokens"].to_numpy(np.int32, B)
        dev_t = wl.out["tokens"].to_numpy(np.int32, B * wl.cap).reshape(B, wl.cap)
        same = sum(int(np.array_equal(r["tokens"][u], dev_t[u, :dev_n[u]])) for u in range(nu))
        out["cpu_baseline"]["token_sequences_equal"] = f"{same}/{nu}"
        out["cpu_baseline"]["steps_equal"] = bool(np.array_equal(r["steps"][:nu], wl.steps()[:nu]))
        # B=1 latency of the scalar reference loop: one thread, the 125-frame utterance
        e1 = synth.encoder_frames(0, 125, D)
        t0 = time.perf_counter()
        r1 = om.decode_window(e1, om.new_state(), MS)
        dt1 = time.perf_counter() - t0
        out["cpu_baseline"]["b1"] = {"us_per_step": round(dt1 * 1e6 / max(1, r1["steps"]), 1), "cores": 1,
                                     "steps": int(r1["steps"]), "frames": 125}
        # parity of the timed workload, outside the timed region: a sample of its
        # utterances replayed through the oracle following the device's decisions
        out["parity"] = sampled_parity(om, wl, traces, encs_of=lambda u: synth.encoder_frames(u, T, D),
                                       sample=(0, 21, 42, 63), max_symbols=MS)

    if not args.no_extras:
        base = B * n_calls
        for name in EXTRAS:
            out[name] = run_extra(name, pk, hipmem, roofline, gguf, synth, dec, cost, tmp, D, MS, base, n_b1)
            if name == "b1":
                wl.free()   # the B=64 frames are not needed past here
        out["b1_cpp"] = b1_cpp
        out["eou_stream_cpp"] = eou_cpp
    print(json.dumps(out), flush=True)
    # every device buffer is released before the interpreter exits (no HIP call
    # runs from a finaliser after the runtime has been torn down)
    wl.free()
    dec.close()


if __name__ == "__main__":
    main()
