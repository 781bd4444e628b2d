"""Training-step operations around the GRU, on the HIP library.

The reference's benchmark model is the recurrent layer followed by
``nn.Linear(hidden_size, 1)``; it is trained with ``F.mse_loss`` and
``torch.optim.AdamW(lr, weight_decay=1e-4)`` (rnn_benchmark.py:510,525,
628-639,722).  This module provides the same three pieces with their
arithmetic in librnn_kernel_amd.so:

* ``LinearHead`` / ``HeadFunction``: pred = out @ w^T + b, squeezed to
  [..., ] (nn.Linear's parameter names and initialisation);
* ``mse_loss`` / ``MSELossFunction``: mean squared error (reduction 'mean');
* ``AdamW``: a ``torch.optim.Optimizer`` whose step is one library call per
  parameter group (torch.optim.AdamW's update rule and defaults).

Like the GRU, they raise RuntimeError for non-GPU or non-fp32 tensors and
have no CPU fallback.
"""
from __future__ import annotations

import ctypes
import math
from typing import Iterable, List

import torch
from torch import nn

from . import _lib


def _stream(device) -> int:
    return torch.cuda.current_stream(device=device).cuda_stream


def _check_tensor(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA/HIP tensor")
    if t.dtype != torch.float32:
        raise RuntimeError(f"{name} must be float32")


class HeadFunction(torch.autograd.Function):
    """pred[..., ] = out[..., :] . weight[0] + bias[0] (nn.Linear(H, 1) then
    squeeze(-1))."""

    @staticmethod
    def forward(ctx, out, weight, bias):
        for t, n in ((out, "out"), (weight, "weight"), (bias, "bias")):
            _check_tensor(t, n)
        hidden = out.size(-1)
        if weight.shape != (1, hidden) or bias.shape != (1,):
            raise ValueError(f"head expects weight [1, {hidden}] and bias [1], got {tuple(weight.shape)} and "
                             f"{tuple(bias.shape)}")
        if weight.device != out.device or bias.device != out.device:
            raise ValueError("head tensors must be on one device")
        out_c, w_c, b_c = out.contiguous(), weight.contiguous(), bias.contiguous()
        rows = out_c.numel() // hidden
        pred = torch.empty(out.shape[:-1], device=out.device, dtype=torch.float32)
        if rows > 0:
            lib = _lib.load()
            with torch.cuda.device(out.device):
                _lib.check(lib.rka_head_forward(_lib.ptr(out_c), _lib.ptr(w_c), _lib.ptr(b_c), _lib.ptr(pred),
                                                rows, hidden, _stream(out.device)), "rka_head_forward")
        ctx.save_for_backward(out_c, w_c)
        return pred

    @staticmethod
    def backward(ctx, grad_pred):
        out, weight = ctx.saved_tensors
        hidden = out.size(-1)
        rows = out.numel() // hidden
        grad_out = torch.empty_like(out) if ctx.needs_input_grad[0] else None
        grad_w = torch.empty_like(weight)
        grad_b = torch.empty(1, device=out.device, dtype=torch.float32)
        if rows == 0:
            grad_w.zero_()
            grad_b.zero_()
            return grad_out, grad_w, grad_b
        g = grad_pred.contiguous()
        lib = _lib.load()
        ws_bytes = lib.rka_head_backward_workspace_bytes(rows, hidden)
        with torch.cuda.device(out.device):
            ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=out.device)
            _lib.check(lib.rka_head_backward(_lib.ptr(out), _lib.ptr(weight), _lib.ptr(g), _lib.ptr(grad_out),
                                             _lib.ptr(grad_w), _lib.ptr(grad_b), _lib.ptr(ws), ws_bytes, rows,
                                             hidden, _stream(out.device)), "rka_head_backward")
        return grad_out, grad_w, grad_b


class LinearHead(nn.Module):
    """``nn.Linear(hidden_size, 1)`` followed by ``squeeze(-1)``, with
    nn.Linear's parameter names, shapes and initialisation."""

    def __init__(self, hidden_size: int) -> None:
        super().__init__()
        self.in_features = hidden_size
        self.out_features = 1
        self.weight = nn.Parameter(torch.empty(1, hidden_size))
        self.bias = nn.Parameter(torch.empty(1))
        self.reset_parameters()

    def reset_parameters(self) -> None:
        # nn.Linear: kaiming_uniform_(a=sqrt(5)) on the weight, i.e.
        # U(-1/sqrt(fan_in), 1/sqrt(fan_in)), and the same bound for the bias
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        bound = 1.0 / math.sqrt(self.in_features)
        nn.init.uniform_(self.bias, -bound, bound)

    def forward(self, out: torch.Tensor) -> torch.Tensor:
        return HeadFunction.apply(out, self.weight, self.bias)


class MSELossFunction(torch.autograd.Function):
    """mean((pred - target)^2) over all elements."""

    @staticmethod
    def forward(ctx, pred, target):
        _check_tensor(pred, "pred")
        _check_tensor(target, "target")
        if pred.shape != target.shape:
            raise ValueError(f"mse_loss: pred {tuple(pred.shape)} and target {tuple(target.shape)} differ")
        if pred.device != target.device:
            raise ValueError("mse_loss: pred and target must be on one device")
        if target.requires_grad:
            raise RuntimeError("mse_loss: gradients with respect to the target are not supported")
        p, t = pred.contiguous(), target.contiguous()
        n = p.numel()
        if n == 0:
            raise ValueError("mse_loss of an empty tensor")
        loss = torch.empty((), device=pred.device, dtype=torch.float32)
        lib = _lib.load()
        ws_bytes = lib.rka_mse_workspace_bytes(n)
        with torch.cuda.device(pred.device):
            ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=pred.device)
            _lib.check(lib.rka_mse_forward(_lib.ptr(p), _lib.ptr(t), _lib.ptr(loss), _lib.ptr(ws), ws_bytes, n,
                                           _stream(pred.device)), "rka_mse_forward")
        ctx.save_for_backward(p, t)
        return loss

    @staticmethod
    def backward(ctx, grad_loss):
        p, t = ctx.saved_tensors
        g = grad_loss.contiguous()
        grad = torch.empty_like(p)
        lib = _lib.load()
        with torch.cuda.device(p.device):
            _lib.check(lib.rka_mse_backward(_lib.ptr(p), _lib.ptr(t), _lib.ptr(g), _lib.ptr(grad), p.numel(),
                                            _stream(p.device)), "rka_mse_backward")
        return grad, None


def mse_loss(pred: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    """``F.mse_loss(pred, target)`` (reduction 'mean') on the HIP library."""
    return MSELossFunction.apply(pred, target)


class AdamW(torch.optim.Optimizer):
    """torch.optim.AdamW (decoupled weight decay, bias-corrected moments) with
    the update of a parameter group done in one library call.

    Same defaults as torch.optim.AdamW; ``amsgrad`` and ``maximize`` are not
    supported.  State per parameter: ``step`` (int), ``exp_avg``,
    ``exp_avg_sq`` (as torch's, so ``state_dict`` round-trips its tensors).
    """

    def __init__(self, params: Iterable, lr: float = 1e-3, betas=(0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 1e-2, amsgrad: bool = False, maximize: bool = False) -> None:
        if lr < 0.0 or eps < 0.0 or weight_decay < 0.0:
            raise ValueError("AdamW: lr, eps and weight_decay must be non-negative")
        if not (0.0 <= betas[0] < 1.0 and 0.0 <= betas[1] < 1.0):
            raise ValueError(f"AdamW: invalid betas {betas}")
        if amsgrad or maximize:
            raise NotImplementedError("AdamW: amsgrad and maximize are not supported")
        super().__init__(params, dict(lr=lr, betas=tuple(betas), eps=eps, weight_decay=weight_decay))

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        lib = _lib.load()
        for group in self.param_groups:
            by_step: dict = {}
            for p in group["params"]:
                if p.grad is None:
                    continue
                if p.grad.is_sparse:
                    raise RuntimeError("AdamW: sparse gradients are not supported")
                _check_tensor(p, "parameter")
                if not p.is_contiguous() or not p.grad.is_contiguous():
                    raise RuntimeError("AdamW: parameters and gradients must be contiguous")
                state = self.state[p]
                if len(state) == 0:
                    state["step"] = 0
                    state["exp_avg"] = torch.zeros_like(p, memory_format=torch.contiguous_format)
                    state["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.contiguous_format)
                state["step"] += 1
                by_step.setdefault((state["step"], p.device), []).append(p)
            beta1, beta2 = group["betas"]
            for (step, device), plist in by_step.items():
                n = len(plist)
                P = ctypes.c_void_p * n
                params = P(*[p.data_ptr() for p in plist])
                grads = P(*[p.grad.data_ptr() for p in plist])
                m = P(*[self.state[p]["exp_avg"].data_ptr() for p in plist])
                v = P(*[self.state[p]["exp_avg_sq"].data_ptr() for p in plist])
                numels = (ctypes.c_size_t * n)(*[p.numel() for p in plist])
                with torch.cuda.device(device):
                    _lib.check(lib.rka_adamw_step(params, grads, m, v, numels, n, group["lr"], beta1, beta2,
                                                  group["eps"], group["weight_decay"], step, _stream(device)),
                               "rka_adamw_step")
        return loss


__all__: List[str] = ["HeadFunction", "LinearHead", "MSELossFunction", "mse_loss", "AdamW"]
