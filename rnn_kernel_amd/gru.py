"""nn.GRU-compatible fp32 GRU whose forward and backward run the gfx950 HIP path.

Host-side mirror of the reference's production interface
(src/rnn_kernel/a100/prod/gru.py):

* ``GRUFunction``  — the autograd.Function (reference ``_A100GRUFunction``,
  gru.py:490-580): ``apply(x[B,T,I], h0[B,H], W_ih, W_hh, b_ih, b_hh) ->
  (output[B,T,H], h_n[1,B,H])``; backward returns the six gradients.
* ``GRU``          — the module (reference ``A100GRU``, gru.py:620-786) with
  nn.GRU parameter names ``weight_ih_l{k}`` / ``weight_hh_l{k}`` /
  ``bias_ih_l{k}`` / ``bias_hh_l{k}``, r/z/n gate order, ``hx`` [L,B,H]
  (zeros when None), batch_first layout; grad mode selects the training
  path, ``torch.no_grad()`` or ``forward_inference`` the cache-free one.
* ``from_torch_gru`` / ``is_supported_gru`` / ``is_available``
  (gru.py:109-136,780-808).

Differences from the reference are limits only: any hidden size in
[1, MAX_HIDDEN_SIZE], any input size >= 1 and any number of layers >= 1 are
accepted (the reference's H = 256, I <= 16, L <= 4 were A100-kernel limits).
Exceptions keep the reference's types: RuntimeError for device / dtype
problems, ValueError for shapes and unsupported module options.

Every tensor operation of the path is a call into librnn_kernel_amd.so; the
only torch work here is allocation (the caching allocator owns all buffers)
and the per-layer ``torch.cat`` of h_n, as in the reference.

Failure of a recurrence launch: the kernels' waits are bounded, and a launch
whose wait gave up leaves NaN in every output it did not compute (never a
finite, wrong value) and is counted by the library.  The launches are
asynchronous, so the count is read at synchronisation points:
``check_recurrences()`` raises ``RecurrenceAbortedError`` (a RuntimeError) when
it has grown since the previous check; with ``set_strict(True)`` (or the
environment variable RKA_STRICT=1) every forward and backward call checks
before returning, at the cost of a device synchronisation.  The reference
raises before launching a grid it cannot make resident
(src/rnn_kernel/a100/prod/gru.py:257-263); here such a batch is split into
resident launches instead, and the check covers what remains: a wait that
gives up.
"""
from __future__ import annotations

import math
import os
import threading
from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import _lib

HIDDEN_SIZE = 256            # default hidden size, as in the reference module
# Largest hidden size accepted: the LDS-tiled backward (hidden_size > 256)
# keeps at least 16 rows of 3H gate gradients in a workgroup's 160 KB of
# LDS, which holds up to hidden_size 810 at batch >= 16.
MAX_HIDDEN_SIZE = 768
DEFAULT_NUM_LAYERS = 1


def _device_index(device) -> int:
    if device is None:
        return torch.cuda.current_device()
    if isinstance(device, int):
        return device
    dev = torch.device(device)
    if dev.type != "cuda":
        raise ValueError("device must be a CUDA (HIP) device.")
    return torch.cuda.current_device() if dev.index is None else dev.index


def is_available(device=None) -> bool:
    """True if ``device`` is a gfx950 GPU and the HIP library loads."""
    if not torch.cuda.is_available():
        return False
    try:
        index = _device_index(device)
    except ValueError:
        return False
    try:
        lib = _lib.load()
    except (RuntimeError, OSError):
        return False
    return bool(lib.rka_device_supported(index))


def is_supported_gru(gru: nn.Module) -> bool:
    """Whether ``gru`` can be replaced by ``GRU`` without changing results."""
    if not isinstance(gru, nn.GRU) or not gru.bias:
        return False
    try:
        first_param = next(gru.parameters())
    except StopIteration:
        return False
    return (
        gru.input_size >= 1
        and 1 <= gru.hidden_size <= MAX_HIDDEN_SIZE
        and gru.num_layers >= 1
        and gru.batch_first
        and not gru.bidirectional
        and gru.dropout == 0.0
        and getattr(gru, "proj_size", 0) == 0
        and first_param.dtype == torch.float32
    )


def _validate_inputs(x, h0, weight_ih, weight_hh, bias_ih, bias_hh) -> Tuple[int, int, int, int, int]:
    """Shape / device / dtype checks (reference gru.py:184-223)."""
    if not x.is_cuda:
        raise RuntimeError("rnn_kernel_amd GRU requires GPU (HIP) tensors.")
    if x.dtype != torch.float32:
        raise RuntimeError("rnn_kernel_amd GRU currently supports fp32 only.")
    if x.dim() != 3:
        raise ValueError("x must have shape [batch, seq, input].")
    if h0.dim() != 2:
        raise ValueError("h0 must have shape [batch, hidden].")
    tensors = (x, h0, weight_ih, weight_hh, bias_ih, bias_hh)
    if len({t.device for t in tensors}) != 1:
        raise ValueError("All tensors must be on the same CUDA device.")
    if any(t.dtype != torch.float32 for t in tensors):
        raise RuntimeError("rnn_kernel_amd GRU currently supports fp32 only.")
    batch, seq_len, input_size = x.shape
    hidden = h0.size(1)
    if not 1 <= hidden <= MAX_HIDDEN_SIZE:
        raise ValueError(f"rnn_kernel_amd GRU requires 1 <= hidden_size <= {MAX_HIDDEN_SIZE}.")
    if batch < 1 or seq_len < 1 or input_size < 1:
        raise ValueError("x must have batch, seq and input dimensions >= 1.")
    if h0.size(0) != batch:
        raise ValueError("h0 batch dimension must match x.")
    if weight_ih.shape != (3 * hidden, input_size):
        raise ValueError("weight_ih must have shape [3 * hidden, input].")
    if weight_hh.shape != (3 * hidden, hidden):
        raise ValueError("weight_hh must have shape [3 * hidden, hidden].")
    if bias_ih.shape != (3 * hidden,) or bias_hh.shape != (3 * hidden,):
        raise ValueError("bias tensors must have shape [3 * hidden].")
    index = x.device.index if x.device.index is not None else torch.cuda.current_device()
    return batch, seq_len, input_size, hidden, index


class RecurrenceAbortedError(RuntimeError):
    """A recurrence launch gave up waiting for another workgroup; its outputs
    hold NaN where they were not computed."""


_abort_lock = threading.Lock()
_abort_seen = {}  # device index -> abort count already reported
_strict = os.environ.get("RKA_STRICT", "0") not in ("", "0")


def set_strict(on: bool) -> None:
    """When on, every GRUFunction forward / backward synchronises its device
    and calls check_recurrences() before returning."""
    global _strict
    _strict = bool(on)


def check_recurrences(device=None) -> None:
    """Raise RecurrenceAbortedError if a recurrence call (one direction of
    one layer) on ``device`` aborted since the previous check (synchronises
    the device)."""
    index = _device_index(device)
    with torch.cuda.device(index):
        count = _lib.recurrence_abort_count()
    with _abort_lock:
        seen = _abort_seen.get(index, 0)
        _abort_seen[index] = count
    if count > seen:
        raise RecurrenceAbortedError(
            f"{count - seen} GRU recurrence call(s) on cuda:{index} aborted (a wait for another workgroup "
            "gave up); their outputs and gradients hold NaN")


def _stream(device) -> int:
    return torch.cuda.current_stream(device=device).cuda_stream


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def _run_forward(x, h0, weight_ih, weight_hh, bias_ih, bias_hh, training: bool):
    batch, seq_len, input_size, hidden, index = _validate_inputs(x, h0, weight_ih, weight_hh, bias_ih, bias_hh)
    lib = _lib.load()
    device = x.device
    x, h0, weight_ih, weight_hh, bias_ih, bias_hh = (
        t.contiguous() for t in (x, h0, weight_ih, weight_hh, bias_ih, bias_hh)
    )
    output = torch.empty(batch, seq_len, hidden, device=device, dtype=torch.float32)
    h_n = torch.empty(1, batch, hidden, device=device, dtype=torch.float32)
    reserve = None
    if training:
        reserve = torch.empty(batch, seq_len, hidden, 4, device=device, dtype=torch.float32)  # (r, z, n, a_n) per unit
    ws_bytes = lib.rka_gru_forward_workspace_bytes(batch, seq_len, input_size, hidden)
    with torch.cuda.device(index):
        ws = _workspace(ws_bytes, device)
        rc = lib.rka_gru_forward(
            _lib.ptr(x), _lib.ptr(h0), _lib.ptr(weight_ih), _lib.ptr(weight_hh), _lib.ptr(bias_ih),
            _lib.ptr(bias_hh), _lib.ptr(output), _lib.ptr(h_n), _lib.ptr(reserve), _lib.ptr(ws), ws_bytes,
            batch, seq_len, input_size, hidden, _stream(device))
        _lib.check(rc, "rka_gru_forward")
    if _strict:
        check_recurrences(index)
    return x, h0, weight_ih, weight_hh, output, h_n, reserve


class GRUFunction(torch.autograd.Function):
    """One GRU layer: forward = input GEMM + persistent recurrence; backward =
    persistent BPTT + gradient GEMMs (reference _A100GRUFunction,
    src/rnn_kernel/a100/prod/gru.py:490-580)."""

    @staticmethod
    def forward(ctx, x, h0, weight_ih, weight_hh, bias_ih, bias_hh):
        x, h0, weight_ih, weight_hh, output, h_n, reserve = _run_forward(
            x, h0, weight_ih, weight_hh, bias_ih, bias_hh, training=True)
        ctx.save_for_backward(x, h0, weight_ih, weight_hh, output, reserve)
        # An unused output's gradient arrives as None (passed to the kernels
        # as NULL) instead of a materialised zero tensor.
        ctx.set_materialize_grads(False)
        return output, h_n

    @staticmethod
    def backward(ctx, grad_output, grad_h_n):
        x, h0, weight_ih, weight_hh, output, reserve = ctx.saved_tensors
        batch, seq_len, input_size = x.shape
        hidden = h0.size(1)
        device = x.device
        lib = _lib.load()
        # grad_output None -> zeros and grad_h_n None -> no seed, as gru.py:534-554;
        # both are passed to the kernel as NULL instead of materialised zeros.
        dy = grad_output.contiguous() if grad_output is not None else None
        dhn = grad_h_n[0].contiguous() if grad_h_n is not None else None
        grad_x = torch.empty_like(x) if ctx.needs_input_grad[0] else None
        grad_h0 = torch.empty_like(h0)
        grad_w_ih = torch.empty_like(weight_ih)
        grad_w_hh = torch.empty_like(weight_hh)
        grad_b_ih = torch.empty(3 * hidden, device=device, dtype=torch.float32)
        grad_b_hh = torch.empty(3 * hidden, device=device, dtype=torch.float32)
        ws_bytes = lib.rka_gru_backward_workspace_bytes(batch, seq_len, input_size, hidden)
        index = device.index if device.index is not None else torch.cuda.current_device()
        with torch.cuda.device(index):
            ws = _workspace(ws_bytes, device)
            rc = lib.rka_gru_backward(
                _lib.ptr(x), _lib.ptr(h0), _lib.ptr(weight_ih), _lib.ptr(weight_hh), _lib.ptr(output),
                _lib.ptr(reserve), _lib.ptr(dy), _lib.ptr(dhn), _lib.ptr(grad_x), _lib.ptr(grad_h0),
                _lib.ptr(grad_w_ih), _lib.ptr(grad_w_hh), _lib.ptr(grad_b_ih), _lib.ptr(grad_b_hh),
                _lib.ptr(ws), ws_bytes, batch, seq_len, input_size, hidden, _stream(device))
            _lib.check(rc, "rka_gru_backward")
        if _strict:
            check_recurrences(index)
        return grad_x, grad_h0, grad_w_ih, grad_w_hh, grad_b_ih, grad_b_hh


def gru_forward_inference(x, h0, weight_ih, weight_hh, bias_ih, bias_hh):
    """Cache-free forward of one layer (reference _a100_gru_forward_inference,
    gru.py:583-617)."""
    with torch.no_grad():
        _, _, _, _, output, h_n, _ = _run_forward(x, h0, weight_ih, weight_hh, bias_ih, bias_hh, training=False)
    return output, h_n


class GRU(nn.Module):
    """Drop-in for unidirectional, batch_first, fp32 ``nn.GRU`` with bias."""

    def __init__(
        self,
        input_size: int,
        hidden_size: int = HIDDEN_SIZE,
        num_layers: int = DEFAULT_NUM_LAYERS,
        batch_first: bool = True,
        bias: bool = True,
        dropout: float = 0.0,
    ) -> None:
        super().__init__()
        if not 1 <= hidden_size <= MAX_HIDDEN_SIZE:
            raise ValueError(f"GRU only supports 1 <= hidden_size <= {MAX_HIDDEN_SIZE}.")
        if input_size < 1:
            raise ValueError("GRU only supports input_size >= 1.")
        if num_layers < 1:
            raise ValueError("GRU only supports num_layers >= 1.")
        if not batch_first:
            raise ValueError("GRU only supports batch_first=True.")
        if not bias:
            raise ValueError("GRU currently requires bias=True.")
        if dropout != 0.0:
            raise ValueError("GRU currently requires dropout=0.")
        self.input_size = input_size
        self.hidden_size = hidden_size
        self.num_layers = num_layers
        self.batch_first = batch_first
        self.bias = bias
        self.dropout = float(dropout)
        for layer in range(num_layers):
            layer_input = input_size if layer == 0 else hidden_size
            setattr(self, f"weight_ih_l{layer}", nn.Parameter(torch.empty(3 * hidden_size, layer_input)))
            setattr(self, f"weight_hh_l{layer}", nn.Parameter(torch.empty(3 * hidden_size, hidden_size)))
            setattr(self, f"bias_ih_l{layer}", nn.Parameter(torch.empty(3 * hidden_size)))
            setattr(self, f"bias_hh_l{layer}", nn.Parameter(torch.empty(3 * hidden_size)))
        self.reset_parameters()

    def reset_parameters(self) -> None:
        stdv = 1.0 / math.sqrt(self.hidden_size)
        for weight in self.parameters():
            nn.init.uniform_(weight, -stdv, stdv)

    def _layer_parameters(self, layer: int):
        return (
            getattr(self, f"weight_ih_l{layer}"),
            getattr(self, f"weight_hh_l{layer}"),
            getattr(self, f"bias_ih_l{layer}"),
            getattr(self, f"bias_hh_l{layer}"),
        )

    def _prepare_hx(self, x: torch.Tensor, hx: Optional[torch.Tensor]) -> torch.Tensor:
        if x.dim() != 3:
            raise ValueError("x must have shape [batch, seq, input].")
        if hx is None:
            return x.new_zeros(self.num_layers, x.size(0), self.hidden_size)
        expected = (self.num_layers, x.size(0), self.hidden_size)
        if tuple(hx.shape) != expected:
            raise ValueError(f"hx must have shape {expected}.")
        return hx

    def _run(self, x: torch.Tensor, hx: torch.Tensor, layer_fn):
        # Per-layer initial states as views whose backward needs no kernel
        # for one layer (a reshape of the gradient) and one stack for
        # several; hx[layer] would zero-fill a [L, B, H] gradient and copy
        # into it for every layer.
        if self.num_layers == 1:
            h_layers = (hx.reshape(hx.shape[1:]),)
        else:
            h_layers = hx.unbind(0)
        layer_input, h_list = x, []
        for layer in range(self.num_layers):
            layer_input, h_layer = layer_fn(layer_input, h_layers[layer], *self._layer_parameters(layer))
            h_list.append(h_layer)
        h_n = h_list[0] if len(h_list) == 1 else torch.cat(h_list, dim=0)
        return layer_input, h_n

    def forward(self, x: torch.Tensor, hx: Optional[torch.Tensor] = None):
        hx = self._prepare_hx(x, hx)
        if not torch.is_grad_enabled():
            return self._run(x, hx, gru_forward_inference)
        return self._run(x, hx, GRUFunction.apply)

    def forward_inference(self, x: torch.Tensor, hx: Optional[torch.Tensor] = None):
        """Explicit cache-free forward (reference gru.py:771-778)."""
        hx = self._prepare_hx(x, hx)
        return self._run(x, hx, gru_forward_inference)

    def forward_output_only(self, x: torch.Tensor, hx: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Output sequence only, as rnn_benchmark.py:521-522 calls it."""
        return self.forward(x, hx)[0]

    @classmethod
    def from_torch_gru(cls, gru: nn.GRU) -> "GRU":
        return from_torch_gru(gru)

    def extra_repr(self) -> str:
        return f"{self.input_size}, {self.hidden_size}, num_layers={self.num_layers}, batch_first=True"


def from_torch_gru(gru: nn.GRU) -> GRU:
    """Build a ``GRU`` with the weights of a supported ``nn.GRU``
    (reference gru.py:789-808)."""
    if not is_supported_gru(gru):
        raise ValueError(
            "Only unidirectional batch_first fp32 GRU with "
            f"1 <= hidden_size <= {MAX_HIDDEN_SIZE}, dropout=0 and bias=True is supported."
        )
    device = next(gru.parameters()).device
    module = GRU(input_size=gru.input_size, hidden_size=gru.hidden_size, num_layers=gru.num_layers,
                 dropout=gru.dropout).to(device=device)
    with torch.no_grad():
        for layer in range(gru.num_layers):
            for name in ("weight_ih", "weight_hh", "bias_ih", "bias_hh"):
                getattr(module, f"{name}_l{layer}").copy_(getattr(gru, f"{name}_l{layer}"))
    return module
