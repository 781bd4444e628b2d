"""``rnn_kernel.a100.prod`` import path of the reference
(src/rnn_kernel/a100/prod/__init__.py): the stable module API."""
from __future__ import annotations

import rnn_kernel as _pkg  # noqa: F401
from rnn_kernel_amd import GRU as A100GRU
from rnn_kernel_amd import from_torch_gru, is_supported_gru
from rnn_kernel_amd import is_available as is_a100_available

A100GRUH256 = A100GRU

__all__ = ["A100GRU", "A100GRUH256", "from_torch_gru", "is_a100_available", "is_supported_gru"]
