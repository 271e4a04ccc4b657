"""Writes lstm_golden.npz: torch.nn.LSTM (a library implementation, not the
reference) on small seeded weights, two consecutive single-token steps from a
zero state, two layers.  Used to pin the oracle's LSTM cell (gate order i, f,
g, o; b_ih + b_hh; layer l+1 fed by layer l's h).

    python tests/golden/make_lstm_golden.py
"""
import os

import numpy as np
import torch

H, L = 16, 2
torch.manual_seed(1234)
lstm = torch.nn.LSTM(input_size=H, hidden_size=H, num_layers=L).double()
with torch.no_grad():   # weights representable in f32, so both sides see the same values
    for prm in lstm.parameters():
        prm.copy_(prm.float().double())
x = torch.randn(2, 1, H, dtype=torch.float32).double()
out = {}
h = torch.zeros(L, 1, H, dtype=torch.float64)
c = torch.zeros(L, 1, H, dtype=torch.float64)
for step in range(2):
    with torch.no_grad():
        _, (h, c) = lstm(x[step:step + 1], (h, c))
    out[f"h{step}"] = h[:, 0].numpy().astype(np.float32).reshape(-1)
    out[f"c{step}"] = c[:, 0].numpy().astype(np.float32).reshape(-1)
for l in range(L):
    for name in ("weight_ih", "weight_hh", "bias_ih", "bias_hh"):
        out[f"{name}_l{l}"] = getattr(lstm, f"{name}_l{l}").detach().numpy().astype(np.float32)
out["x"] = x[:, 0].numpy().astype(np.float32)
np.savez(os.path.join(os.path.dirname(os.path.abspath(__file__)), "lstm_golden.npz"), **out)
print("wrote lstm_golden.npz")
