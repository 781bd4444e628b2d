"""``rnn_kernel.a100`` import path of the reference (src/rnn_kernel/a100/__init__.py).

Only the names rnn_benchmark.py and the reference's prod tests use are
provided.  ``A100GRUH256`` accepts the experimental module's constructor
(src/rnn_kernel/a100/gru_autograd.py:4736-4799): ``block_threads`` and the
``use_*`` / split-count variant switches select among ~80 A100 kernel
experiments there; here there is one MI355X path, so they are accepted and
ignored.  The experimental launcher functions are not provided.
"""
from __future__ import annotations

import rnn_kernel as _pkg  # noqa: F401  (puts rnn_kernel_amd on sys.path)
from rnn_kernel_amd import GRU, from_torch_gru, is_supported_gru
from rnn_kernel_amd.gru import GRUFunction

from ..custom_gru import copy_from_torch_gru

_VARIANT_KWARGS = {"recompute_hidden_gates", "split_recurrent_count", "cooperative_split_count"}


class A100GRUH256(GRU):
    def __init__(self, input_size: int, hidden_size: int = 256, num_layers: int = 1, batch_first: bool = True,
                 bias: bool = True, dropout: float = 0.0, block_threads: int = 0, **variant_flags) -> None:
        unknown = sorted(k for k in variant_flags if not (k.startswith("use_") or k in _VARIANT_KWARGS))
        if unknown:
            raise TypeError(f"A100GRUH256 got unexpected keyword arguments {unknown}")
        super().__init__(input_size, hidden_size, num_layers, batch_first=batch_first, bias=bias, dropout=dropout)
        self.block_threads = block_threads


def a100_gru_h256(x, h0, weight_ih, weight_hh, bias_ih, bias_hh):
    """One layer through the autograd.Function: (output, h_n)."""
    return GRUFunction.apply(x, h0, weight_ih, weight_hh, bias_ih, bias_hh)


__all__ = ["A100GRUH256", "a100_gru_h256", "copy_from_torch_gru", "from_torch_gru", "is_supported_gru"]
