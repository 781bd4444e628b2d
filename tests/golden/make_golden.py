"""Writes tests/golden/gru_golden.npz: small GRU cases computed by
torch.nn.GRU in float64 on the CPU (PyTorch is the third-party library the
reference's own tests compare against; no reference code is involved).

Each case stores its inputs (x, h0, per-layer weights, output gradients) and
the expected outputs (y, h_n) and gradients (dx, dh0, per-layer weight
gradients).  Run: python tests/golden/make_golden.py
"""
import os

import numpy as np
import torch

CASES = [
    # name, L, I, H, B, T, h0 scale (0 = zeros)
    ("c1_smoke", 1, 16, 16, 2, 8, 0.0),     # BASELINE config 1 shape
    ("odd_h5", 1, 3, 5, 3, 4, 1.0),         # odd, tiny
    ("odd_h33", 1, 7, 33, 2, 6, 0.5),       # not a multiple of 4 / 32
    ("two_layer", 2, 4, 7, 3, 5, 1.0),      # stacked layers (reference test_custom_gru shape)
    ("t1_b1", 1, 2, 3, 1, 1, 0.0),          # single step, single row
]


def make_case(name, L, I, H, B, T, h0_scale, seed):
    torch.manual_seed(seed)
    gru = torch.nn.GRU(I, H, num_layers=L, batch_first=True).double()
    x = torch.randn(B, T, I, dtype=torch.float64, requires_grad=True)
    h0 = (h0_scale * torch.randn(L, B, H, dtype=torch.float64)).requires_grad_(True)
    y, hn = gru(x, h0)
    dy = torch.randn_like(y)
    dhn = torch.randn_like(hn)
    (y * dy).sum().add((hn * dhn).sum()).backward()
    out = {"x": x.detach().numpy(), "h0": h0.detach().numpy(), "dy": dy.numpy(), "dhn": dhn.numpy(),
           "y": y.detach().numpy(), "hn": hn.detach().numpy(), "dx": x.grad.numpy(), "dh0": h0.grad.numpy(),
           "dims": np.array([L, I, H, B, T])}
    for pname, p in gru.named_parameters():
        out[pname] = p.detach().numpy()
        out["grad_" + pname] = p.grad.numpy()
    return {f"{name}/{k}": v for k, v in out.items()}


def main():
    arrays = {}
    for i, case in enumerate(CASES):
        arrays.update(make_case(*case, seed=1000 + i))
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gru_golden.npz")
    np.savez_compressed(path, **arrays)
    print(path, sum(a.nbytes for a in arrays.values()), "bytes")


if __name__ == "__main__":
    main()
