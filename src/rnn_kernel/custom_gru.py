"""``CustomGRU`` import path of the reference (src/rnn_kernel/custom_gru.py:16-137).

The reference's CustomGRU is a Python time loop over torch ops with an
optional Triton pointwise backend.  Here the same constructor runs the HIP
path: ``pointwise_backend`` is accepted for signature compatibility ("torch"
or "triton"; both mean the fused in-kernel gate math, there is no Triton).
"""
from __future__ import annotations

import torch.nn as nn

from rnn_kernel_amd import GRU


class CustomGRU(GRU):
    def __init__(self, input_size: int, hidden_size: int, num_layers: int, pointwise_backend: str = "torch",
                 batch_first: bool = True) -> None:
        if not batch_first:
            raise ValueError("CustomGRU only supports batch_first=True.")
        if pointwise_backend not in {"torch", "triton"}:
            raise ValueError(f"Unsupported pointwise backend: {pointwise_backend}")
        super().__init__(input_size, hidden_size, num_layers, batch_first=True)
        self.pointwise_backend = pointwise_backend


def copy_from_torch_gru(custom_gru: GRU, torch_gru: nn.GRU) -> None:
    """Copy nn.GRU weights into a GRU of the same shape (reference custom_gru.py:120-137)."""
    if torch_gru.bidirectional:
        raise ValueError("Bidirectional GRU is not supported.")
    if not torch_gru.batch_first:
        raise ValueError("Only batch_first=True GRU is supported.")
    for attr in ("num_layers", "hidden_size", "input_size"):
        if getattr(custom_gru, attr) != getattr(torch_gru, attr):
            raise ValueError(f"{attr} mismatch.")
    custom_gru.load_state_dict(torch_gru.state_dict())
