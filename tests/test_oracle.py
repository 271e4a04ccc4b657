"""Pins the oracle (CPU restatement of the reference decoder) against things
the reference does not get to define: library routines (numpy float16,
torch.nn.LSTM golden vectors), float64 brute force, closed forms of scripted
decoders, invariants (linearity, chunked == one-shot), and a planted mistake
that the replay must flag."""
import os

import numpy as np
import pytest

from conftest import small_eou, small_tdt

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ---------------------------------------------------------------- primitives

def test_f16_to_f32_all_bit_patterns(oracle_mod):
    lib = oracle_mod.lib()
    bits = np.arange(1 << 16, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([lib.ora_f16_to_f32(int(b)) for b in bits[::7]], np.float32)
    exp = ref[::7]
    finite = np.isfinite(exp)
    assert np.array_equal(got[finite].view(np.uint32), exp[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(exp)]))
    assert np.array_equal(np.isinf(got), np.isinf(exp))


def test_q8_0_dequant_known_blocks(oracle_mod):
    """Hand-built q8_0 blocks {f16 d; int8 q[32]}: value = q * d."""
    d = np.array([0.5, -0.25, 3.0], np.float16)
    q = np.stack([np.arange(-16, 16), np.full(32, -128), np.arange(32) * 4 - 64]).astype(np.int8)
    raw = np.zeros((3, 34), np.uint8)
    raw[:, :2] = d.view(np.uint8).reshape(3, 2)
    raw[:, 2:] = q.view(np.uint8)
    out = np.zeros(96, np.float32)
    oracle_mod.lib().ora_dequant(raw.ctypes.data, 8, 96, oracle_mod.fptr(out))
    assert out[:32].tolist() == [0.5 * v for v in range(-16, 16)]
    assert out[32:64].tolist() == [32.0] * 32
    assert out[64:].tolist() == [3.0 * (4 * i - 64) for i in range(32)]


def test_q8_0_quantizer_roundtrip(pkg):
    from parakeet_amd import gguf
    rng = np.random.default_rng(0)
    x = rng.standard_normal((7, 64)).astype(np.float32)
    raw = gguf.quantize_q8_0(x)
    assert len(raw) == 7 * 2 * 34
    y = gguf.dequantize(raw, gguf.GGML_Q8_0, x.size).reshape(x.shape)
    amax = np.abs(x.reshape(-1, 32)).max(1)
    err = np.abs(x - y).reshape(-1, 32).max(1)
    assert np.all(err <= amax / 127 * 0.5 * 1.01 + 1e-7)


def _blocks(d, body):
    """Raw blocks: f16 scale d then the body bytes of each block."""
    d = np.asarray(d, np.float16)
    body = np.asarray(body, np.uint8)
    return np.concatenate([d.view(np.uint8).reshape(-1, 2), body], axis=1)


def _oracle_dequant(oracle_mod, raw, t, n):
    out = np.zeros(n, np.float32)
    raw = np.ascontiguousarray(raw)
    oracle_mod.lib().ora_dequant(raw.ctypes.data, t, n, oracle_mod.fptr(out))
    return out


def test_q4_0_dequant_known_blocks(oracle_mod, pkg):
    """q4_0 {f16 d; u8 qs[16]}: weight j = (low nibble of qs[j] - 8) d, weight j+16 = (high
    nibble - 8) d.  Each block has one obvious answer: all-zero bytes give -8d, all-0xFF
    give +7d, low nibble 1 / high nibble 2 give -7d then -6d (a swap of the halves fails),
    and nibble j in the low half with 15-j in the high half walks -8..7 then 7..-8."""
    from parakeet_amd import gguf
    qs = np.stack([np.zeros(16), np.full(16, 0xFF), np.full(16, 0x21),
                   np.arange(16) | ((15 - np.arange(16)) << 4)]).astype(np.uint8)
    raw = _blocks([0.5, 2.0, -0.25, 1.0], qs)
    want = np.concatenate([np.full(32, -4.0), np.full(32, 14.0),
                           np.r_[np.full(16, 1.75), np.full(16, 1.5)],
                           np.r_[np.arange(-8, 8), np.arange(7, -9, -1)]]).astype(np.float32)
    assert np.array_equal(_oracle_dequant(oracle_mod, raw, 2, 128), want)
    assert np.array_equal(gguf.dequantize(raw.tobytes(), gguf.GGML_Q4_0, 128), want)


def test_q5_0_dequant_known_blocks(oracle_mod, pkg):
    """q5_0 {f16 d; u8 qh[4]; u8 qs[16]}: weight j = ((nibble | bit j of qh << 4) - 16) d, the
    high nibbles and bits 16..31 of qh for weights 16..31.  All-zero gives -16d, all-ones
    +15d; qh = 0x0000FFFF (only the first half high) gives 0 then -16d; qh = 0x00010000
    raises weight 16 alone (a wrong bit index or half fails)."""
    from parakeet_amd import gguf
    def body(qh, qs):
        return np.concatenate([np.frombuffer(np.uint32(qh).tobytes(), np.uint8), np.full(16, qs, np.uint8)])
    raw = _blocks([1.0, 0.5, 2.0, 1.0], np.stack([body(0, 0), body(0xFFFFFFFF, 0xFF), body(0x0000FFFF, 0),
                                                    body(0x00010000, 0)]))
    want = np.concatenate([np.full(32, -16.0), np.full(32, 7.5), np.r_[np.zeros(16), np.full(16, -32.0)],
                           np.r_[np.full(16, -16.0), [0.0], np.full(15, -16.0)]]).astype(np.float32)
    assert np.array_equal(_oracle_dequant(oracle_mod, raw, 6, 128), want)
    assert np.array_equal(gguf.dequantize(raw.tobytes(), gguf.GGML_Q5_0, 128), want)


@pytest.mark.parametrize("qtype,lo,hi", [(2, -8, 7), (6, -16, 15)])
def test_q4_q5_quantizer_exact_on_grid(oracle_mod, pkg, qtype, lo, hi):
    """Values k*d with k in the type's integer range and one element at the most negative k:
    the reference rule d = max / lo recovers d exactly (d a power of two), so quantize then
    dequantize returns the input bit for bit, through the Python and the C paths alike."""
    from parakeet_amd import gguf
    rng = np.random.default_rng(qtype)
    k = rng.integers(lo, hi + 1, size=(6, 32))
    k[:, 5] = lo
    d = 2.0 ** rng.integers(-6, 3, size=(6, 1))
    x = (k * d).astype(np.float32)
    raw = gguf.QUANTIZE[qtype](x)
    assert len(raw) == 6 * gguf.BLOCK_BYTES[qtype]
    assert np.array_equal(gguf.dequantize(raw, qtype, x.size).reshape(x.shape), x)
    assert np.array_equal(_oracle_dequant(oracle_mod, np.frombuffer(raw, np.uint8), qtype, x.size).reshape(x.shape), x)


@pytest.mark.parametrize("qtype,levels", [(2, 8), (6, 16)])
def test_q4_q5_quantizer_error_bound_and_paths_agree(oracle_mod, pkg, qtype, levels):
    """Random rows: every weight within half a step of its input (except the clamped top
    code, within one step), and the C oracle, the Python reader and the integer view agree."""
    from parakeet_amd import gguf
    rng = np.random.default_rng(10 + qtype)
    x = rng.standard_normal((9, 64)).astype(np.float32)
    raw = gguf.QUANTIZE[qtype](x)
    y = gguf.dequantize(raw, qtype, x.size).reshape(x.shape)
    b = x.reshape(-1, 32)
    step = np.abs(b).max(1) / levels
    err = np.abs(b - y.reshape(-1, 32))
    assert np.all(err <= step[:, None] * 1.0 + 1e-6)
    assert np.mean(err <= step[:, None] * 0.5 * 1.01 + 1e-7) > 0.95
    c = _oracle_dequant(oracle_mod, np.frombuffer(raw, np.uint8), qtype, x.size).reshape(x.shape)
    assert np.array_equal(c, y)
    d, q = gguf.block_ints(raw, qtype, x.size // 32)
    assert q.min() >= -levels and q.max() <= levels - 1
    assert np.array_equal((q * d[:, None]).astype(np.float32).reshape(x.shape), y)


def test_argmax_first_index(oracle_mod):
    am = lambda a: oracle_mod.lib().ora_argmax(oracle_mod.fptr(np.asarray(a, np.float32)), len(a))
    assert am([1, 3, 3, 2]) == 1
    assert am([0, 0, 0]) == 0
    assert am([-5]) == 0
    assert am([-1, -0.5, -0.5000001]) == 1
    assert am([2, 1, 2]) == 0


@pytest.mark.parametrize("seed", [0, 1])
def test_gemv_vs_float64(oracle_mod, seed):
    rng = np.random.default_rng(seed)
    W = rng.standard_normal((13, 40)).astype(np.float32)
    x = rng.standard_normal(40).astype(np.float32)
    b = rng.standard_normal(13).astype(np.float32)
    y = np.zeros(13, np.float32)
    lib = oracle_mod.lib()
    lib.ora_gemv(oracle_mod.fptr(W), oracle_mod.fptr(x), oracle_mod.fptr(b), oracle_mod.fptr(y), 13, 40)
    ref = W.astype(np.float64) @ x + b
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-5)
    # gemv_add accumulates; W(2x) = 2 W x (linearity), bias-free
    y2 = np.ones(13, np.float32)
    x2 = (2 * x).astype(np.float32)
    lib.ora_gemv_add(oracle_mod.fptr(W), oracle_mod.fptr(x2), oracle_mod.fptr(y2), 13, 40)
    assert np.allclose(y2 - 1.0, 2 * (W.astype(np.float64) @ x), rtol=1e-5, atol=1e-5)


def _golden_model(oracle_mod, g):
    H = 16
    weights = {"tdt.predict.embed.weight": np.zeros((2, H), np.float32)}
    for l in range(2):
        weights[f"tdt.predict.lstm.{l}.w_ih"] = g[f"weight_ih_l{l}"]
        weights[f"tdt.predict.lstm.{l}.w_hh"] = g[f"weight_hh_l{l}"]
        weights[f"tdt.predict.lstm.{l}.b_ih"] = g[f"bias_ih_l{l}"]
        weights[f"tdt.predict.lstm.{l}.b_hh"] = g[f"bias_hh_l{l}"]
    for n, shp in (("joint.enc.weight", (4, 4)), ("joint.enc.bias", (4,)), ("joint.pred.weight", (4, H)),
                   ("joint.pred.bias", (4,)), ("joint.out.weight", (3, 4)), ("joint.out.bias", (3,))):
        weights["tdt." + n] = np.zeros(shp, np.float32)
    return oracle_mod.OracleModel(weights, "tdt", H, 2, 4, 4, 1, durations=[0])


def test_lstm_matches_torch_golden(oracle_mod):
    g = np.load(os.path.join(GOLDEN, "lstm_golden.npz"))
    om = _golden_model(oracle_mod, g)
    st = om.new_state()
    for step in range(2):
        om.lstm_step(g["x"][step], st)
        assert np.allclose(st.h, g[f"h{step}"], rtol=2e-5, atol=2e-6), step
        assert np.allclose(st.c, g[f"c{step}"], rtol=2e-5, atol=2e-6), step


def test_lstm_golden_catches_gate_swap(oracle_mod):
    """Planted mistake: swapping the f and g gate blocks must fail the golden check."""
    g = dict(np.load(os.path.join(GOLDEN, "lstm_golden.npz")))
    H = 16
    for l in range(2):
        for k in (f"weight_ih_l{l}", f"weight_hh_l{l}", f"bias_ih_l{l}", f"bias_hh_l{l}"):
            a = g[k].copy()
            a[H:2 * H], a[2 * H:3 * H] = g[k][2 * H:3 * H], g[k][H:2 * H]
            g[k] = a
    om = _golden_model(oracle_mod, g)
    st = om.new_state()
    om.lstm_step(g["x"][0], st)
    assert not np.allclose(st.h, g["h0"], rtol=1e-3, atol=1e-4)


def test_joint_closed_form(oracle_mod, tmp_path):
    w = small_tdt(str(tmp_path / "m.gguf"))
    from parakeet_amd import gguf
    om = oracle_mod.OracleModel.from_gguf(str(tmp_path / "m.gguf"), gguf)
    rng = np.random.default_rng(3)
    enc = rng.standard_normal(128).astype(np.float32)
    pred = rng.standard_normal(64).astype(np.float32)
    f = lambda k: w[k].astype(np.float64)
    hid = np.maximum(0, f("tdt.joint.enc.weight") @ enc + f("tdt.joint.enc.bias")
                     + f("tdt.joint.pred.weight") @ pred + f("tdt.joint.pred.bias"))
    ref = f("tdt.joint.out.weight") @ hid + f("tdt.joint.out.bias")
    assert np.allclose(om.joint(enc, pred), ref, rtol=1e-4, atol=1e-4)


# ---------------------------------------------------------------- control flow

def _scripted(tmp_path, writer, bias, name="s.gguf", **kw):
    from parakeet_amd import gguf
    import oracle
    p = "tdt" if writer is small_tdt else "eou"
    J = 96
    ov = {f"{p}.joint.out.weight": np.zeros((len(bias), J), np.float32),
          f"{p}.joint.out.bias": np.asarray(bias, np.float32)}
    path = str(tmp_path / name)
    writer(path, overrides=ov, **kw)
    return oracle.OracleModel.from_gguf(path, gguf)


def test_tdt_symbol_cap_closed_form(tmp_path):
    V1 = 62
    bias = np.zeros(V1 + 5, np.float32)
    bias[5], bias[V1] = 3.0, 2.0
    om = _scripted(tmp_path, small_tdt, bias)
    enc = np.zeros((9, 128), np.float32)
    for ms in (1, 3, 10):
        r = om.decode_window(enc, om.new_state(), ms)
        assert r["tokens"].tolist() == [5] * (9 * ms) and r["steps"] == 9 * ms


def test_tdt_duration_carry_closed_form(tmp_path):
    V1 = 62
    bias = np.zeros(V1 + 5, np.float32)
    bias[7], bias[V1 + 4] = 1.0, 1.0
    om = _scripted(tmp_path, small_tdt, bias)
    st = om.new_state()
    emitted, carry = [], []
    for _ in range(5):
        r = om.decode_window(np.zeros((3, 128), np.float32), st, 10)
        emitted.append(len(r["tokens"]))
        carry.append(st.st.carry_frames)
    assert emitted == [1, 1, 1, 0, 1] and carry == [1, 2, 3, 0, 1]


def test_tdt_blank_with_duration(tmp_path):
    """blank with duration 3 advances 3 frames per step: ceil(T/3) steps."""
    V1 = 62
    bias = np.zeros(V1 + 5, np.float32)
    bias[61], bias[V1 + 3] = 1.0, 1.0
    om = _scripted(tmp_path, small_tdt, bias)
    r = om.decode_window(np.zeros((10, 128), np.float32), om.new_state(), 10)
    assert r["steps"] == 4 and len(r["tokens"]) == 0


def test_tdt_duration_table_closed_form(tmp_path):
    """The duration is the table's value at the argmax index
    (src/parakeet_tdt.cpp:938-940): table {0, 2, 3, 5, 8}."""
    V1, table = 62, [0, 2, 3, 5, 8]
    bias = np.zeros(V1 + 5, np.float32)
    bias[61], bias[V1 + 3] = 1.0, 1.0                      # blank, index 3 -> 5 frames
    om = _scripted(tmp_path, small_tdt, bias, durations=table)
    st = om.new_state()
    r = om.decode_window(np.zeros((12, 128), np.float32), st, 10)
    assert r["steps"] == 3 and len(r["tokens"]) == 0 and st.st.carry_frames == 3
    bias = np.zeros(V1 + 5, np.float32)
    bias[7], bias[V1 + 1] = 1.0, 1.0                       # token 7, index 1 -> 2 frames
    om = _scripted(tmp_path, small_tdt, bias, name="t.gguf", durations=table)
    st = om.new_state()
    r = om.decode_window(np.zeros((9, 128), np.float32), st, 10)
    assert r["tokens"].tolist() == [7] * 5 and st.st.carry_frames == 1


def test_tdt_three_durations_without_zero(tmp_path):
    """num_durations 3, table {1, 4, 7}: V1 + 3 joint rows; a token at index 0
    advances one frame, so the symbol cap is never reached."""
    V1 = 62
    bias = np.zeros(V1 + 3, np.float32)
    bias[7], bias[V1] = 1.0, 1.0
    om = _scripted(tmp_path, small_tdt, bias, durations=[1, 4, 7])
    assert om.Dn == 3 and om.Vo == V1 + 3
    r = om.decode_window(np.zeros((6, 128), np.float32), om.new_state(), 2)
    assert r["tokens"].tolist() == [7] * 6 and r["steps"] == 6


def test_tdt_empty_duration_table_uses_the_index(tmp_path):
    """An empty table with num_durations 5: the duration is the argmax index."""
    V1 = 62
    bias = np.zeros(V1 + 5, np.float32)
    bias[61], bias[V1 + 3] = 1.0, 1.0                      # blank, index 3 -> 3 frames
    om = _scripted(tmp_path, small_tdt, bias, durations=[], num_durations=5)
    assert om.Dn == 5
    r = om.decode_window(np.zeros((10, 128), np.float32), om.new_state(), 10)
    assert r["steps"] == 4 and len(r["tokens"]) == 0
    bias = np.zeros(V1 + 5, np.float32)
    bias[9], bias[V1] = 1.0, 1.0                           # token, index 0 -> symbol cap
    om = _scripted(tmp_path, small_tdt, bias, name="t.gguf", durations=[], num_durations=5)
    r = om.decode_window(np.zeros((4, 128), np.float32), om.new_state(), 3)
    assert r["tokens"].tolist() == [9] * 12 and r["steps"] == 12


@pytest.mark.parametrize("variant", [dict(durations=[], num_durations=5),
                                     dict(durations=None, num_durations=5)])
def test_tdt_index_tables_decode_alike(oracle_mod, tmp_path, variant):
    """An empty table (duration = index) and an absent key (the {0, 1, 2, 3, 4}
    default) decode a random model exactly as the explicit {0, 1, 2, 3, 4}."""
    from parakeet_amd import gguf, synth
    small_tdt(str(tmp_path / "a.gguf"))
    small_tdt(str(tmp_path / "b.gguf"), **variant)
    oa = oracle_mod.OracleModel.from_gguf(str(tmp_path / "a.gguf"), gguf)
    ob = oracle_mod.OracleModel.from_gguf(str(tmp_path / "b.gguf"), gguf)
    for u in range(3):
        enc = synth.encoder_frames(60 + u, 40, 128)
        ra = oa.decode_window(enc, oa.new_state(), 10, trace=True)
        rb = ob.decode_window(enc, ob.new_state(), 10, trace=True)
        assert np.array_equal(ra["trace"], rb["trace"]) and ra["steps"] == rb["steps"]
        assert len(set(ra["trace"][:, 1].tolist())) >= 3      # several duration indices taken


def test_tdt_table_longer_than_count(oracle_mod, tmp_path):
    """num_durations 3 with a 5-entry table: only the first 3 entries exist as
    logits, so the decode equals the one with table {0, 1, 2}; an index-3
    entry of 9 is never taken.  A table shorter than the count is refused."""
    from parakeet_amd import gguf, synth
    small_tdt(str(tmp_path / "a.gguf"), durations=[0, 1, 2])
    small_tdt(str(tmp_path / "b.gguf"), durations=[0, 1, 2, 9, 9], num_durations=3)
    oa = oracle_mod.OracleModel.from_gguf(str(tmp_path / "a.gguf"), gguf)
    ob = oracle_mod.OracleModel.from_gguf(str(tmp_path / "b.gguf"), gguf)
    assert ob.Dn == 3 and ob.Vo == 62 + 3
    enc = synth.encoder_frames(70, 40, 128)
    ra = oa.decode_window(enc, oa.new_state(), 10, trace=True)
    rb = ob.decode_window(enc, ob.new_state(), 10, trace=True)
    assert np.array_equal(ra["trace"], rb["trace"]) and set(rb["trace"][:, 1].tolist()) == {0, 1, 2}
    small_tdt(str(tmp_path / "c.gguf"), durations=[0, 1], num_durations=3)
    with pytest.raises(ValueError):
        oracle_mod.OracleModel.from_gguf(str(tmp_path / "c.gguf"), gguf)


def test_tdt_blank_id_zero_closed_form(tmp_path):
    """blank_id 0 (the reference takes any id from parakeet.tdt.blank_id): id 0
    is the blank, id 61 (the converter's blank) an ordinary token."""
    V1 = 62
    bias = np.zeros(V1 + 5, np.float32)
    bias[0], bias[V1 + 2] = 1.0, 1.0                       # id 0, index 2 -> blank, 2 frames
    om = _scripted(tmp_path, small_tdt, bias, blank_id=0)
    r = om.decode_window(np.zeros((10, 128), np.float32), om.new_state(), 10)
    assert om.blank == 0 and r["steps"] == 5 and len(r["tokens"]) == 0
    bias = np.zeros(V1 + 5, np.float32)
    bias[61], bias[V1 + 1] = 1.0, 1.0                      # id 61, index 1 -> a token, 1 frame
    om = _scripted(tmp_path, small_tdt, bias, name="t.gguf", blank_id=0)
    r = om.decode_window(np.zeros((10, 128), np.float32), om.new_state(), 10)
    assert r["tokens"].tolist() == [61] * 10


def swap_blank(w, p, vocab, b):
    """Tensor overrides that swap ids ``b`` and ``vocab`` (the blank) in the
    embedding and the joint output: with blank_id ``b`` the model is the same
    decoder with those two ids renamed."""
    ov = {}
    for name in (f"{p}.predict.embed.weight", f"{p}.joint.out.weight", f"{p}.joint.out.bias"):
        a = np.array(w[name]).reshape(w[name].shape[0], -1) if w[name].ndim > 1 else np.array(w[name])
        a[[b, vocab]] = a[[vocab, b]]
        ov[name] = a
    return ov


@pytest.mark.parametrize("kind", ["tdt", "eou"])
def test_blank_id_relabelling(oracle_mod, tmp_path, kind):
    """Renaming the blank and an ordinary id (rows swapped, blank_id moved)
    decodes the same: traces equal once the two ids are swapped back, segment
    boundaries and step counts equal."""
    from parakeet_amd import gguf, synth
    writer, vocab, D, b = (small_tdt, 61, 128, 0) if kind == "tdt" else (small_eou, 35, 64, 5)
    w = writer(str(tmp_path / "a.gguf"), quant="f32")
    bias = w[f"{kind}.joint.out.bias"].copy()
    bias[b] += 1.0                     # both renamed ids taken often
    bias[vocab] += 2.0
    w = writer(str(tmp_path / "a.gguf"), quant="f32", overrides={f"{kind}.joint.out.bias": bias})
    shaped = dict(w)
    shaped[f"{kind}.predict.embed.weight"] = w[f"{kind}.predict.embed.weight"].reshape(-1, 64)
    shaped[f"{kind}.joint.out.weight"] = w[f"{kind}.joint.out.weight"].reshape(-1, 96)
    writer(str(tmp_path / "b.gguf"), quant="f32", blank_id=b, overrides=swap_blank(shaped, kind, vocab, b))
    oa = oracle_mod.OracleModel.from_gguf(str(tmp_path / "a.gguf"), gguf)
    ob = oracle_mod.OracleModel.from_gguf(str(tmp_path / "b.gguf"), gguf)
    assert ob.blank == b
    ms = 10 if kind == "tdt" else 5
    n_tok, n_b, n_blank = 0, 0, 0
    for u in range(3):
        enc = synth.encoder_frames(80 + u, 40, D)
        ra = oa.decode_window(enc, oa.new_state(), ms, trace=True)
        rb = ob.decode_window(enc, ob.new_state(), ms, trace=True)
        tb = np.array(rb["trace"])
        col = tb[:, 0] if tb.ndim == 2 else tb
        col[:] = np.where(col == b, vocab, np.where(col == vocab, b, col))
        assert np.array_equal(np.asarray(ra["trace"]), tb) and ra["steps"] == rb["steps"]
        if kind == "eou":
            assert np.array_equal(ra["segments"], rb["segments"])
        n_tok += len(ra["tokens"])
        ids = np.asarray(ra["trace"])[:, 0]
        n_b, n_blank = n_b + int((ids == b).sum()), n_blank + int((ids == vocab).sum())
    assert n_tok > 0 and n_b >= 5 and n_blank >= 5, (n_tok, n_b, n_blank)


def test_eou_closed_forms(tmp_path):
    V1 = 36
    bias = np.zeros(V1, np.float32)
    bias[33] = 1.0                                          # <EOU> always
    om = _scripted(tmp_path, small_eou, bias)
    st = om.new_state()
    r = om.decode_window(np.zeros((6, 64), np.float32), st, 5, tokens_before=3)
    assert r["steps"] == 6 and r["segments"].tolist() == [3]
    assert st.st.last_token == 35 and st.st.segment_start_token == 3
    bias = np.zeros(V1, np.float32)
    bias[12] = 1.0                                          # ordinary token always
    om = _scripted(tmp_path, small_eou, bias, name="t.gguf")
    st = om.new_state()
    r = om.decode_window(np.zeros((4, 64), np.float32), st, 5)
    assert r["tokens"].tolist() == [12] * 20 and r["steps"] == 20
    assert st.st.symbols_this_step == 5


def test_chunked_equals_one_shot(oracle_mod, tmp_path):
    from parakeet_amd import gguf, synth
    small_tdt(str(tmp_path / "m.gguf"))
    om = oracle_mod.OracleModel.from_gguf(str(tmp_path / "m.gguf"), gguf)
    enc = synth.encoder_frames(5, 37, 128)
    one = om.decode_window(enc, om.new_state(), 10)["tokens"].tolist()
    for chunk in (3, 4, 8):
        st = om.new_state()
        toks = []
        for s0 in range(0, 37, chunk):
            toks += om.decode_window(enc[s0:s0 + chunk], st, 10)["tokens"].tolist()
        assert toks == one, chunk


def test_replay_flags_planted_mistake(oracle_mod, tmp_path):
    from parakeet_amd import gguf, synth
    small_tdt(str(tmp_path / "m.gguf"))
    om = oracle_mod.OracleModel.from_gguf(str(tmp_path / "m.gguf"), gguf)
    enc = synth.encoder_frames(9, 30, 128)
    r = om.decode_window(enc, om.new_state(), 10, trace=True)
    ok = om.replay_window(enc, om.new_state(), 10, r["trace"])
    assert ok["stats"]["unexplained"] == 0 and ok["stats"]["structure_error"] == 0
    assert ok["tokens"].tolist() == r["tokens"].tolist()
    bad = r["trace"].copy()
    bad[3, 0] = (bad[3, 0] + 1) % 61                     # a wrong token at step 3
    rep = om.replay_window(enc, om.new_state(), 10, bad)
    assert rep["stats"]["unexplained"] >= 1 and rep["stats"]["first_unexplained"] == 3


def test_batch_driver_matches_single(oracle_mod, tmp_path):
    from parakeet_amd import gguf, synth
    small_tdt(str(tmp_path / "m.gguf"))
    om = oracle_mod.OracleModel.from_gguf(str(tmp_path / "m.gguf"), gguf)
    encs = [synth.encoder_frames(u, 10 + 3 * u, 128) for u in range(6)]
    bb = np.array([0, 2, 4, 0, 2, 4], np.float32)
    b = om.decode_batch(encs, 10, blank_bias=bb, n_threads=3)
    assert b["rc"] == 0
    for u, e in enumerate(encs):
        r = om.decode_window(e, om.new_state(), 10, blank_bias=float(bb[u]))
        assert b["tokens"][u].tolist() == r["tokens"].tolist() and b["steps"][u] == r["steps"]


def test_carry_larger_than_window_is_dropped(tmp_path):
    """Reference quirk kept on purpose: a carry that exceeds the next window is
    consumed only up to that window's length, then overwritten with
    max(0, t - n) (src/parakeet_tdt.cpp:906-910, 979)."""
    V1 = 62
    bias = np.zeros(V1 + 5, np.float32)
    bias[7], bias[V1 + 4] = 1.0, 1.0            # token 7, duration 4, always
    om = _scripted(tmp_path, small_tdt, bias)
    st = om.new_state()
    om.decode_window(np.zeros((1, 128), np.float32), st, 10)
    assert st.st.carry_frames == 3
    r = om.decode_window(np.zeros((1, 128), np.float32), st, 10)
    assert r["steps"] == 0 and st.st.carry_frames == 0   # 2 frames of carry dropped
    r = om.decode_window(np.zeros((1, 128), np.float32), st, 10)
    assert r["steps"] == 1


def test_replay_counts_planted_near_tie(tmp_path):
    """The replay's classifier: a decision that differs from the oracle argmax by
    less than the tie bound (top-2 margin < 1e-4) is a near-tie, not an
    unexplained mismatch; the same decision at a margin above the bound is
    unexplained.  Scripted logits (zero joint weights, biases only): token 5 at
    1.0 and token 9 just below it, duration index 1 (duration 1) on top, so the
    margin is exactly what the bias sets, whatever the state."""
    V1 = 62
    for gap, tie in ((5e-5, True), (3e-4, False)):
        bias = np.zeros(V1 + 5, np.float32)
        bias[5], bias[9], bias[V1 + 1], bias[V1 + 2] = 1.0, 1.0 - gap, 1.0, 1.0 - gap
        om = _scripted(tmp_path, small_tdt, bias, name=f"tie{int(tie)}.gguf")
        enc = np.zeros((8, 128), np.float32)
        r = om.decode_window(enc, om.new_state(), 10, trace=True)
        assert r["tokens"].tolist() == [5] * 8
        planted = r["trace"].copy()
        planted[3, 0] = 9                                  # the runner-up token at step 3
        planted[7, 1] = 2                                  # the runner-up duration index at the last step
        rep = om.replay_window(enc, om.new_state(), 10, planted)
        s = rep["stats"]
        assert s["structure_error"] == 0
        assert rep["tokens"].tolist() == [5, 5, 5, 9, 5] + [5] * (len(rep["tokens"]) - 5)
        if tie:
            assert s["near_ties"] == 2 and s["unexplained"] == 0, s
        else:
            assert s["near_ties"] == 0 and s["unexplained"] == 2 and s["first_unexplained"] == 3, s
