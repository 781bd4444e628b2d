"""Drop-in import surface of the reference package (``rnn_kernel``) backed by
the MI355X HIP path in ``rnn_kernel_amd``.

The reference's callers (rnn_benchmark.py, its tests) import
``rnn_kernel.custom_gru.CustomGRU``, ``rnn_kernel.a100.A100GRUH256`` and
``rnn_kernel.a100.prod.*`` with ``PYTHONPATH=src``; these modules resolve those
names to the one product implementation.
"""
import os as _os
import sys as _sys

try:
    import rnn_kernel_amd as _rka  # noqa: F401
except ImportError:  # source-tree layout: the package sits two levels up
    _root = _os.path.dirname(_os.path.dirname(_os.path.dirname(_os.path.abspath(__file__))))
    if _root not in _sys.path:
        _sys.path.insert(0, _root)
    import rnn_kernel_amd as _rka  # noqa: F401

from .custom_gru import CustomGRU

__all__ = ["CustomGRU"]
