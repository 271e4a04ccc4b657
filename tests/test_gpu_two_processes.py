"""Two processes decoding on one GPU at once.

The decode loop needs every CU of the GPU for its barriers.  Calls from two
processes are serialised by the per-GPU loop lock (an exclusive flock held from
a call's loop launch to its last stream synchronisation), so both processes'
calls succeed and give the tokens of a decode run alone.  Without it, two
overlapping loops would each end with PK_ERR_TIMEOUT after the kernel's 2 s
barrier limit (the loops never hang either way)."""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

from conftest import ROOT, small_tdt

pytestmark = pytest.mark.gpu

CHILD = r"""
import json, sys, time
sys.path.insert(0, sys.argv[1])
import __graft_entry__ as g
g.load_package()
from parakeet_amd import pk, synth
dec = pk.Decoder.from_gguf(sys.argv[2], n_slots=4 * 30)
encs = [synth.encoder_frames(500 + u, 60, 128) for u in range(4)]
start = float(sys.argv[3])
while time.time() < start:   # both processes begin together
    time.sleep(0.001)
out = []
for call in range(30):
    res = dec.decode(encs, slots=list(range(4 * call, 4 * call + 4)))
    out.append([r["tokens"].tolist() for r in res])
dec.close()
print(json.dumps(out))
"""


def test_two_processes_share_the_gpu(tmp_path):
    from parakeet_amd import pk, synth
    path = str(tmp_path / "m.gguf")
    small_tdt(path)
    import time
    start = time.time() + 20.0   # after both children have imported and uploaded
    print("two processes x 30 calls, B=4 T=60", flush=True)
    procs = [subprocess.Popen([sys.executable, "-c", CHILD, ROOT, path, str(start)], stdout=subprocess.PIPE,
                              stderr=subprocess.PIPE, text=True) for _ in range(2)]
    outs = []
    for pr in procs:
        o, e = pr.communicate(timeout=240)
        assert pr.returncode == 0, e[-3000:]
        outs.append(json.loads(o.strip().splitlines()[-1]))
    dec = pk.Decoder.from_gguf(path, n_slots=4)
    want = [r["tokens"].tolist() for r in dec.decode([synth.encoder_frames(500 + u, 60, 128) for u in range(4)])]
    dec.close()
    for o in outs:
        assert len(o) == 30
        for call in o:
            assert call == want
