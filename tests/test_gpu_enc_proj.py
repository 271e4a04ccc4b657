"""enc_proj (b_e + W_e . enc for every frame, src/parakeet_tdt.cpp:433-483 on
the reference's GPU path, its CPU loop's host_joint_step input at :154-177)
has two kernels: a tiled one for many rows and a narrow one, one wave per 16x16
block, for few rows (streaming chunks, short windows).  The host picks one by
row count, so a window's result must not depend on the choice: with each kernel
forced (PK_ENC_PROJ), the joint logits (which add the encp rows), decisions,
tokens and final states are equal bit for bit.  Shapes cover K in whole and
partial batches of the narrow kernel (d_enc 1024, 128, 64), a joint width that
is not a multiple of 64 (96), and ragged windows that share row tiles."""
import os

import numpy as np
import pytest

from conftest import small_eou, small_tdt

pytestmark = pytest.mark.gpu


def _run(dev, encs, slot0, kernel, **kw):
    old = os.environ.get("PK_ENC_PROJ")
    os.environ["PK_ENC_PROJ"] = kernel
    try:
        res = dev.decode(encs, slots=list(range(slot0, slot0 + len(encs))), trace=True, **kw)
    finally:
        if old is None:
            os.environ.pop("PK_ENC_PROJ")
        else:
            os.environ["PK_ENC_PROJ"] = old
    return res


def _same(dev, a, b, n, base_a, base_b):
    for u in range(n):
        assert np.array_equal(a[u]["trace"], b[u]["trace"]), u
        assert a[u]["tokens"].tolist() == b[u]["tokens"].tolist(), u
        if "logits" in a[u]:
            la, lb = a[u]["logits"], b[u]["logits"]
            live = ~np.isnan(la)
            assert np.array_equal(live, ~np.isnan(lb)), u
            assert np.array_equal(la[live].view(np.uint32), lb[live].view(np.uint32)), u
        x, y = dev.read_state(base_a + u), dev.read_state(base_b + u)
        assert np.array_equal(x["h"], y["h"]) and np.array_equal(x["c"], y["c"]), u


@pytest.mark.parametrize("shape", ["tdt06b", "small_tdt", "small_eou"])
def test_enc_proj_kernels_bit_identical(tmp_path, shape):
    from parakeet_amd import pk, synth
    path = str(tmp_path / "m.gguf")
    if shape == "tdt06b":
        synth.make_shape(path, "tdt-0.6b-v3")
    elif shape == "small_tdt":
        small_tdt(path)
    else:
        small_eou(path)
    Ts = [1, 15, 16, 17, 130, 3]
    dev = pk.Decoder.from_gguf(path, n_slots=2 * len(Ts))
    encs = [synth.encoder_frames(300 + u, T, dev.info.D) for u, T in enumerate(Ts)]
    print(f"enc_proj kernels, {shape}: D={dev.info.D} J={dev.info.J}, T={Ts}", flush=True)
    kw = dict(logit_steps=3) if shape != "small_eou" else {}
    a = _run(dev, encs, 0, "tile", **kw)
    b = _run(dev, encs, len(Ts), "narrow", **kw)
    _same(dev, a, b, len(Ts), 0, len(Ts))
