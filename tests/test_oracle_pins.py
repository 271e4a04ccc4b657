"""Pins the oracle functions that the primitive checks in test_oracle.py leave
open, each against something the reference does not define:

  ora_init_state (src/parakeet_tdt.cpp:813-863, src/parakeet_eou.cpp:206-230)
      torch.nn.LSTM golden vectors: zero state -> one LSTM step on
      embed[blank] must give the golden (h, c); pred = h of the last layer.
  EOU reset on <EOU> (src/parakeet_eou.cpp:289-306)
      the same golden: after the reset the state is the init state, whatever
      it held before.
  EOU branches (src/parakeet_eou.cpp:275-320)
      a frame-driven scripted model (the argmax of frame t is the index of
      its one-hot encoder frame) with a closed-form token / segment / step
      stream over blank, <EOB>, <EOU> with and without tokens since the
      segment start, a "<...>" piece, and the symbol cap.
  blank-logit offset (a build addition; 0 reproduces the reference)
      scripted logits where the offset decides between blank and a token,
      including the exact tie (first index wins) and a neighbour row that
      would win if the offset landed on the wrong row.

Each check is chosen so that a plausible mistake fails it (planted mistakes
are asserted to fail where the check could otherwise pass vacuously)."""
import os

import numpy as np

from conftest import small_eou, small_tdt

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
H = 16


def _golden():
    return np.load(os.path.join(GOLDEN, "lstm_golden.npz"))


def _golden_model(oracle_mod, g, kind, L, embed_rows, out_bias=None):
    """Oracle model on the golden LSTM weights (layers 0 .. L-1) with a given
    embedding table; the joint is zero except for the output bias."""
    p = "tdt" if kind == "tdt" else "eou"
    V1 = len(embed_rows)
    weights = {f"{p}.predict.embed.weight": np.stack(embed_rows).astype(np.float32)}
    for l in range(L):
        weights[f"{p}.predict.lstm.{l}.w_ih"] = g[f"weight_ih_l{l}"]
        weights[f"{p}.predict.lstm.{l}.w_hh"] = g[f"weight_hh_l{l}"]
        weights[f"{p}.predict.lstm.{l}.b_ih"] = g[f"bias_ih_l{l}"]
        weights[f"{p}.predict.lstm.{l}.b_hh"] = g[f"bias_hh_l{l}"]
    Dn = 1 if kind == "tdt" else 0
    Vo = V1 + Dn
    for n, shp in (("joint.enc.weight", (4, 4)), ("joint.enc.bias", (4,)), ("joint.pred.weight", (4, H)),
                   ("joint.pred.bias", (4,)), ("joint.out.weight", (Vo, 4))):
        weights[f"{p}.{n}"] = np.zeros(shp, np.float32)
    weights[f"{p}.joint.out.bias"] = (np.zeros(Vo, np.float32) if out_bias is None
                                      else np.asarray(out_bias, np.float32))
    if kind == "tdt":
        return oracle_mod.OracleModel(weights, "tdt", H, L, 4, 4, V1 - 1, durations=[0])
    return oracle_mod.OracleModel(weights, "eou", H, L, 4, 4, V1 - 1, eou_id=1, eob_id=2)


def _spoil(st, rng):
    """Put arbitrary values into a state, as if it had decoded something."""
    st.h[:] = rng.standard_normal(st.h.shape).astype(np.float32)
    st.c[:] = rng.standard_normal(st.c.shape).astype(np.float32)
    st.pred[:] = 7.0
    st.st.symbols_this_step = 3
    st.st.carry_frames = 2
    st.st.last_token = 0
    st.st.segment_start_token = 9


# ---------------------------------------------------------------- init state

def test_init_state_tdt_matches_torch_golden(oracle_mod):
    """Two layers; blank = 1 holds the golden input x[0], row 0 holds x[1]."""
    g = _golden()
    om = _golden_model(oracle_mod, g, "tdt", 2, [g["x"][1], g["x"][0]])
    assert om.blank == 1
    st = om.new_state()
    _spoil(st, np.random.default_rng(0))
    om.init_state(st)
    assert np.allclose(st.h, g["h0"], rtol=2e-5, atol=2e-6)
    assert np.allclose(st.c, g["c0"], rtol=2e-5, atol=2e-6)
    assert np.array_equal(st.pred, st.h[H:2 * H])          # pred = h of the last layer
    assert st.st.initialized == 1 and st.st.symbols_this_step == 0 and st.st.carry_frames == 0


def test_init_state_golden_is_discriminative(oracle_mod):
    """Planted mistake: an init that primed with embed[0] (or not at all) would
    not reproduce the golden, so the check above can fail."""
    g = _golden()
    om = _golden_model(oracle_mod, g, "tdt", 2, [g["x"][0], g["x"][1]])   # blank row holds x[1] now
    st = om.new_state()
    om.init_state(st)
    assert not np.allclose(st.h, g["h0"], rtol=1e-3, atol=1e-4)
    unprimed = np.zeros_like(st.h)
    assert not np.allclose(unprimed, g["h0"], rtol=1e-3, atol=1e-4)


def test_init_state_eou_matches_torch_golden(oracle_mod):
    """One layer (layer 0 of the golden is a one-layer LSTM on its own):
    h, c = the golden's layer-0 half; last_token -1, segment start 0."""
    g = _golden()
    om = _golden_model(oracle_mod, g, "eou", 1, [g["x"][1], g["x"][1], g["x"][1], g["x"][0]])
    assert om.blank == 3
    st = om.new_state()
    _spoil(st, np.random.default_rng(1))
    om.init_state(st)
    assert np.allclose(st.h, g["h0"][:H], rtol=2e-5, atol=2e-6)
    assert np.allclose(st.c, g["c0"][:H], rtol=2e-5, atol=2e-6)
    assert np.array_equal(st.pred, st.h)
    assert st.st.last_token == -1 and st.st.segment_start_token == 0 and st.st.symbols_this_step == 0


def test_eou_reset_matches_torch_golden(oracle_mod):
    """<EOU> forced by the output bias: whatever h, c held, one frame later the
    state is zero -> LSTM(embed[blank]) = the golden, and last_token = blank.
    Planted mistake: a reset that kept c would carry the spoiled c into the cell."""
    g = _golden()
    bias = np.zeros(4, np.float32)
    bias[1] = 1.0                                           # <EOU> (eou_id 1) always
    om = _golden_model(oracle_mod, g, "eou", 1, [g["x"][1], g["x"][1], g["x"][1], g["x"][0]], bias)
    st = om.new_state()
    om.init_state(st)
    _spoil(st, np.random.default_rng(2))
    st.st.segment_start_token = 0                           # 4 earlier tokens since the segment start
    r = om.decode_window(np.zeros((1, 4), np.float32), st, 5, tokens_before=4)
    assert r["steps"] == 1 and r["tokens"].size == 0
    assert r["segments"].tolist() == [4]
    assert np.allclose(st.h, g["h0"][:H], rtol=2e-5, atol=2e-6)
    assert np.allclose(st.c, g["c0"][:H], rtol=2e-5, atol=2e-6)
    assert st.st.last_token == 3 and st.st.segment_start_token == 4


# ---------------------------------------------------------------- EOU branches

def _frame_driven_eou(tmp_path, pieces_special=True):
    """small_eou (vocab 35: <unk> 0, <EOU> 33, <EOB> 34, blank 35) whose joint
    makes the argmax of frame t the index k of its one-hot frame: W_e = I,
    W_p = 0, W_o[v, v] = 1, all biases 0."""
    from parakeet_amd import gguf
    import oracle
    J, D, V1 = 96, 64, 36
    we = np.zeros((J, D), np.float32)
    we[:D, :D] = np.eye(D, dtype=np.float32)
    wo = np.zeros((V1, J), np.float32)
    wo[np.arange(V1), np.arange(V1)] = 1.0
    ov = {"eou.joint.enc.weight": we, "eou.joint.enc.bias": np.zeros(J, np.float32),
          "eou.joint.pred.weight": np.zeros((J, 64), np.float32), "eou.joint.pred.bias": np.zeros(J, np.float32),
          "eou.joint.out.weight": wo, "eou.joint.out.bias": np.zeros(V1, np.float32)}
    path = str(tmp_path / "fd.gguf")
    small_eou(path, overrides=ov)
    om = oracle.OracleModel.from_gguf(path, gguf)
    if not pieces_special:
        om.m.n_special = 0
    return om


def _onehot_frames(ks, D=64):
    enc = np.zeros((len(ks), D), np.float32)
    enc[np.arange(len(ks)), ks] = 1.0
    return enc


def test_eou_branches_closed_form(tmp_path):
    """Frames: token 5, blank, <EOU>, <EOU>, <EOB>, <unk>, token 7, <EOU>.
      token 5   5 emissions (symbol cap 5), 5 steps
      blank     1 step
      <EOU>     boundary at 5 (5 tokens since segment start 0), reset, 1 step
      <EOU>     no boundary (no token since the last one), reset, 1 step
      <EOB>     1 step, nothing
      <unk>     a "<...>" piece: 1 step, nothing
      token 7   5 emissions, 5 steps
      <EOU>     boundary at 10, 1 step"""
    om = _frame_driven_eou(tmp_path)
    enc = _onehot_frames([5, 35, 33, 33, 34, 0, 7, 33])
    st = om.new_state()
    r = om.decode_window(enc, st, 5, trace=True)
    assert r["rc"] == 0
    assert r["tokens"].tolist() == [5] * 5 + [7] * 5
    assert r["segments"].tolist() == [5, 10]
    assert r["steps"] == 16
    assert r["trace"][:, 0].tolist() == [5] * 5 + [35, 33, 33, 34, 0] + [7] * 5 + [33]
    assert st.st.last_token == 35 and st.st.segment_start_token == 10 and st.st.symbols_this_step == 0
    # the caller's earlier tokens shift every boundary (the reference compares out_tokens.size())
    r2 = om.decode_window(enc, om.new_state(), 5, tokens_before=3)
    assert r2["segments"].tolist() == [8, 13] and r2["tokens"].tolist() == r["tokens"].tolist()


def test_eou_branches_are_discriminative(tmp_path):
    """Planted mistakes in the piece table and the symbol cap change the closed form:
    without "<...>" pieces <unk>, <EOU>-less pieces are emitted; a cap of 2 halves the runs."""
    om = _frame_driven_eou(tmp_path, pieces_special=False)
    enc = _onehot_frames([5, 35, 33, 33, 34, 0, 7, 33])
    r = om.decode_window(enc, om.new_state(), 5)
    assert r["tokens"].tolist() == [5] * 5 + [0] * 5 + [7] * 5 and r["segments"].tolist() == [5, 15]
    om = _frame_driven_eou(tmp_path)
    r = om.decode_window(enc, om.new_state(), 2)
    assert r["tokens"].tolist() == [5] * 2 + [7] * 2 and r["steps"] == 10


def test_eou_symbol_cap_resets_per_frame(tmp_path):
    """max_symbols 3 over two token frames: 3 + 3 emissions; sym counts from 0 each frame."""
    om = _frame_driven_eou(tmp_path)
    st = om.new_state()
    r = om.decode_window(_onehot_frames([9, 11]), st, 3)
    assert r["tokens"].tolist() == [9, 9, 9, 11, 11, 11] and r["steps"] == 6
    assert st.st.symbols_this_step == 3 and st.st.last_token == 11


# ---------------------------------------------------------------- blank offset

def _scripted_tdt(tmp_path, bias):
    from parakeet_amd import gguf
    import oracle
    ov = {"tdt.joint.out.weight": np.zeros((len(bias), 96), np.float32),
          "tdt.joint.out.bias": np.asarray(bias, np.float32)}
    path = str(tmp_path / "bb.gguf")
    small_tdt(path, overrides=ov)
    return oracle.OracleModel.from_gguf(path, gguf)


def test_blank_bias_closed_form_tdt(tmp_path):
    """Token 5 logit 1.0, token 6 logit 0.9, blank (61) 0.5, duration index 1.
      offset 0.4  -> 0.9 < 1.0: token 5 every frame (T tokens, T steps)
      offset 0.5  -> exact tie 1.0 = 1.0: the first index (5) wins
      offset 0.6  -> blank every frame: T steps, no token
    An offset applied to row 6 instead of the blank would emit token 6 at 0.2."""
    V1 = 62
    bias = np.zeros(V1 + 5, np.float32)
    bias[5], bias[6], bias[61], bias[V1 + 1] = 1.0, 0.9, 0.5, 1.0
    om = _scripted_tdt(tmp_path, bias)
    enc = np.zeros((7, 128), np.float32)
    for off, exp in ((0.0, [5] * 7), (0.2, [5] * 7), (0.4, [5] * 7), (0.5, [5] * 7), (0.6, [])):
        r = om.decode_window(enc, om.new_state(), 10, blank_bias=off)
        assert r["tokens"].tolist() == exp and r["steps"] == 7, (off, r)
    # the batch driver passes each utterance its own offset
    b = om.decode_batch([enc, enc, enc], 10, blank_bias=np.array([0.0, 0.6, 0.4], np.float32))
    assert [len(t) for t in b["tokens"]] == [7, 0, 7]


def test_blank_bias_closed_form_eou(tmp_path):
    """EOU: token 12 logit 1.0, blank (35) 0.5.  Offset 0.6: one blank step per frame."""
    from parakeet_amd import gguf
    import oracle
    V1 = 36
    bias = np.zeros(V1, np.float32)
    bias[12], bias[35] = 1.0, 0.5
    ov = {"eou.joint.out.weight": np.zeros((V1, 96), np.float32), "eou.joint.out.bias": bias}
    path = str(tmp_path / "bbe.gguf")
    small_eou(path, overrides=ov)
    om = oracle.OracleModel.from_gguf(path, gguf)
    enc = np.zeros((4, 64), np.float32)
    r = om.decode_window(enc, om.new_state(), 5, blank_bias=0.6)
    assert r["tokens"].size == 0 and r["steps"] == 4
    r = om.decode_window(enc, om.new_state(), 5, blank_bias=0.4)
    assert r["tokens"].tolist() == [12] * 20 and r["steps"] == 20
