#!/usr/bin/env python3
"""Benchmark: TDT greedy decode steps/s on one MI355X.

Workload (one bench step = one batched decode call, inputs resident in HBM):
TDT-0.6b-v3-shaped decoder, q8_0 weights (seeded random, GGUF decoder
layout), B=64 independent utterances of T=750 encoder frames each (fp32
N(0,1), 1024-d, seed 1000+u), max_symbols_per_step 10, every utterance
decoded in lockstep with on-device compaction.  A decode step is one joint
evaluation for one utterance (the reference's out_steps counter).

Prints one JSON line.  Extra fields: the B=1, T=125 latency (us/step) and the
B=256, T=750 throughput on the same decoder, the roofline of the dominant
kernel (the decode loop), and the CPU baseline (the oracle, a C restatement
of the reference's scalar decoder, timed on this host on a bounded sample).
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


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--frames", type=int, default=750)
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-utts", type=int, default=16)
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="first run a plain device copy of MIB MiB (calibrates hardware byte counters)")
    ap.add_argument("--traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="counter_collection.csv of two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) of "
                         "this bench with --copy-probe 256: fills roofline.traffic")
    return ap.parse_args()


class Workload:
    """B utterances of T frames resident on the device, with output buffers and
    fresh state slots for every call."""

    def __init__(self, pk, hipmem, dec, B, T, D, max_sym, n_calls, slot_base, first_seed=1000,
                 blank_bias=None):
        from parakeet_amd import synth
        self.pk, self.hm, self.dec = pk, hipmem, dec
        self.B, self.T, self.max_sym = B, T, max_sym
        frames = np.empty((B * T, D), np.float32)
        for u in range(B):
            frames[u * T:(u + 1) * T] = synth.encoder_frames(u, T, D, base_seed=first_seed)
        self.enc = hipmem.DeviceArray.from_numpy(frames)
        del frames
        self.rows = np.arange(B, dtype=np.int64) * T
        self.Ts = np.full(B, T, np.int32)
        self.cap = T * max(1, max_sym) + 1
        self.tcap = T * (max(1, max_sym) + 1) + 1
        self.out = dict(tokens=hipmem.DeviceArray(4 * B * self.cap), n_tokens=hipmem.DeviceArray(4 * B),
                        steps=hipmem.DeviceArray(4 * B))
        self.trace = hipmem.DeviceArray(8 * B * self.tcap)
        self.blank_bias = blank_bias
        self.calls = 0
        self.n_calls = n_calls
        self.slot_base = slot_base
        assert slot_base + B * n_calls <= dec.n_slots

    def run(self, trace=False):
        assert self.calls < self.n_calls, "every call decodes fresh slots"
        slots = np.arange(self.B, dtype=np.int32) + self.slot_base + self.calls * self.B
        self.calls += 1
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


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: the decode path shards as independent "
                                   "utterances per GPU with no collective, and only --gpus 1 is run"}))
        sys.exit(2)
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
    n_b1, n_b256 = 24, 3
    dec = pk.Decoder(rd, n_slots=B * n_calls + (0 if args.no_extras else n_b1 + 256 * n_b256))
    info = dec.info
    types = dict(embed=rd.tensors["tdt.predict.embed.weight"].ggml_type,
                 lstm=rd.tensors["tdt.predict.lstm.0.w_ih"].ggml_type,
                 pred=rd.tensors["tdt.joint.pred.weight"].ggml_type,
                 out=rd.tensors["tdt.joint.out.weight"].ggml_type,
                 enc=rd.tensors["tdt.joint.enc.weight"].ggml_type)
    cost = roofline.DecoderCost(info, types)

    wl = Workload(pk, hipmem, dec, B, T, D, MS, n_calls, 0)
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
    if args.traffic:
        tr = roofline.pmc_traffic(*args.traffic)
        out["roofline"]["traffic"] = round(tr["bytes_per_launch"], 0)
        out["roofline"]["traffic_detail"] = {
            k: {"kib_per_dispatch": round(v["kib_per_dispatch"], 1), "copy_factor": round(v["factor"], 4)}
            for k, v in tr.items() if k != "bytes_per_launch"}

    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle
        om = oracle.OracleModel.from_gguf(path, gguf)
        nu = min(args.cpu_utts, B)
        threads = max(1, min(16, os.cpu_count() or 1, nu))
        encs = [synth.encoder_frames(u, T, D) for u in range(nu)]
        t0 = time.perf_counter()
        r = om.decode_batch(encs, MS, n_threads=threads)
        dt = time.perf_counter() - t0
        cpu_steps = int(np.sum(r["steps"]))
        out["cpu_baseline"] = {"value": round(cpu_steps / dt, 1), "unit": "decode steps/s", "cores": threads,
                               "kind": "port",
                               "sample": f"first {nu} of the {B} utterances (full {T} frames each), "
                                         f"{cpu_steps} steps in {dt:.2f} s, one utterance per thread task, "
                                         f"oracle built with -O3 -ffast-math -funroll-loops"}
        # the same utterances decoded on the device agree token for token
        dev_tok = wl.out["n_tokens"].to_numpy(np.int32, B)[:nu]
        out["cpu_baseline"]["token_counts_equal"] = bool(
            all(len(r["tokens"][u]) == dev_tok[u] for u in range(nu)))

    if not args.no_extras:
        # B=1, T=125 (10 s of audio): per-step latency
        wl1 = Workload(pk, hipmem, dec, 1, 125, D, MS, n_b1, B * n_calls)
        wall1, loop1, enc1, it1 = timed(wl1, 2, 20)
        st1 = int(wl1.steps().sum())
        out["b1"] = {"frames": 125, "decode_steps": st1, "us_per_step_loop": round(loop1 * 1e3 / st1, 3),
                     "us_per_step_incl_enc_proj": round((loop1 + enc1) * 1e3 / st1, 3),
                     "us_per_step_wall": round(wall1 / 20 * 1e6 / st1, 3)}
        del wl1
        # B=256, T=750: lockstep throughput
        wl256 = Workload(pk, hipmem, dec, 256, 750, D, MS, n_b256, B * n_calls + n_b1)
        wall2, loop2, enc2, it2 = timed(wl256, 1, 2)
        st2 = int(wl256.steps().sum())
        out["b256"] = {"frames": 750, "decode_steps": st2, "steps_per_s": round(st2 * 2 / wall2, 1),
                       "loop_ms": round(loop2, 3), "enc_proj_ms": round(enc2, 3), "iterations": it2}
        del wl256

    print(json.dumps(out), flush=True)
    dec.close()


if __name__ == "__main__":
    main()
