"""numpy front end of the C GRU oracle.

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module; the product
package ``rnn_kernel_amd`` never does.  It is the checker the HIP path is
compared against, never a fallback for it.

The arithmetic lives in ``gru_oracle_impl.h`` (a scalar C restatement of the
reference's forward recurrence, gate cache, BPTT and gradient GEMMs, with
file:line citations there).  This module adds:

* ``forward`` / ``backward`` for one layer (fp64 or fp32);
* ``stack_forward_backward`` for a stack of layers with the reference's layer
  composition (layer l's input is layer l-1's output, ``hx`` sliced per
  layer, zeros when ``hx`` is None): src/rnn_kernel/a100/prod/gru.py:673-728.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np

_DIR = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_DIR, "liboracle_gru.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile the oracle with the committed Makefile (gcc)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _DIR] + (["-B"] if force else []), check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    for suffix in ("_f64", "_f32"):
        fwd = getattr(lib, "oracle_gru_forward" + suffix)
        fwd.restype = ctypes.c_int
        fwd.argtypes = [ctypes.c_int] * 4 + [ctypes.c_void_p] * 9
        bwd = getattr(lib, "oracle_gru_backward" + suffix)
        bwd.restype = ctypes.c_int
        bwd.argtypes = [ctypes.c_int] * 4 + [ctypes.c_void_p] * 14
    _lib = lib
    return lib


def _suffix(dtype) -> str:
    dtype = np.dtype(dtype)
    if dtype == np.float64:
        return "_f64"
    if dtype == np.float32:
        return "_f32"
    raise TypeError(f"oracle supports float32/float64, got {dtype}")


def _c(a: Optional[np.ndarray], dtype) -> Optional[np.ndarray]:
    if a is None:
        return None
    return np.ascontiguousarray(np.asarray(a, dtype=dtype))


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


@dataclass
class ForwardResult:
    y: np.ndarray       # [B, T, H]
    hn: np.ndarray      # [B, H]
    cache: Optional[np.ndarray]  # [B, T, 4H] = (r, z, n, a_n)


@dataclass
class BackwardResult:
    dx: Optional[np.ndarray]
    dh0: np.ndarray
    dw_ih: np.ndarray
    dw_hh: np.ndarray
    db_ih: np.ndarray
    db_hh: np.ndarray


def forward(x, h0, w_ih, w_hh, b_ih, b_hh, dtype=np.float64, with_cache: bool = True) -> ForwardResult:
    """One layer forward; x [B,T,I], h0 [B,H], weights in nn.GRU layout."""
    lib = _load()
    x, h0, w_ih, w_hh, b_ih, b_hh = (_c(a, dtype) for a in (x, h0, w_ih, w_hh, b_ih, b_hh))
    B, T, I = x.shape
    H = h0.shape[1]
    assert h0.shape == (B, H) and w_ih.shape == (3 * H, I) and w_hh.shape == (3 * H, H)
    assert b_ih.shape == (3 * H,) and b_hh.shape == (3 * H,)
    y = np.empty((B, T, H), dtype=dtype)
    hn = np.empty((B, H), dtype=dtype)
    cache = np.empty((B, T, 4 * H), dtype=dtype) if with_cache else None
    rc = getattr(lib, "oracle_gru_forward" + _suffix(dtype))(
        B, T, I, H, _p(x), _p(h0), _p(w_ih), _p(w_hh), _p(b_ih), _p(b_hh), _p(y), _p(hn), _p(cache))
    if rc != 0:
        raise MemoryError("oracle_gru_forward failed to allocate")
    return ForwardResult(y, hn, cache)


def backward(x, h0, w_ih, w_hh, y, cache, dy, dhn, dtype=np.float64, need_dx: bool = True) -> BackwardResult:
    """One layer backward from the forward's y and cache; dy/dhn may be None."""
    lib = _load()
    x, h0, w_ih, w_hh, y, cache, dy, dhn = (_c(a, dtype) for a in (x, h0, w_ih, w_hh, y, cache, dy, dhn))
    B, T, I = x.shape
    H = h0.shape[1]
    dx = np.empty((B, T, I), dtype=dtype) if need_dx else None
    dh0 = np.empty((B, H), dtype=dtype)
    dw_ih = np.empty((3 * H, I), dtype=dtype)
    dw_hh = np.empty((3 * H, H), dtype=dtype)
    db_ih = np.empty((3 * H,), dtype=dtype)
    db_hh = np.empty((3 * H,), dtype=dtype)
    rc = getattr(lib, "oracle_gru_backward" + _suffix(dtype))(
        B, T, I, H, _p(x), _p(h0), _p(w_ih), _p(w_hh), _p(y), _p(cache), _p(dy), _p(dhn),
        _p(dx), _p(dh0), _p(dw_ih), _p(dw_hh), _p(db_ih), _p(db_hh))
    if rc != 0:
        raise MemoryError("oracle_gru_backward failed to allocate")
    return BackwardResult(dx, dh0, dw_ih, dw_hh, db_ih, db_hh)


def _row_chunks(B: int, threads: int):
    n = max(1, min(int(threads), B))
    edges = [B * k // n for k in range(n + 1)]
    return [(edges[k], edges[k + 1]) for k in range(n) if edges[k + 1] > edges[k]]


def forward_rows_parallel(x, h0, w_ih, w_hh, b_ih, b_hh, threads: int, dtype=np.float64) -> ForwardResult:
    """``forward`` with the batch rows split over ``threads`` threads.

    Batch rows are independent sequences, so every row's result is the one
    ``forward`` computes for it (the C calls release the GIL)."""
    from concurrent.futures import ThreadPoolExecutor

    x, h0 = np.asarray(x), np.asarray(h0)
    chunks = _row_chunks(x.shape[0], threads)
    with ThreadPoolExecutor(len(chunks)) as ex:
        parts = list(ex.map(lambda c: forward(x[c[0]:c[1]], h0[c[0]:c[1]], w_ih, w_hh, b_ih, b_hh, dtype=dtype),
                            chunks))
    return ForwardResult(np.concatenate([f.y for f in parts]), np.concatenate([f.hn for f in parts]),
                         np.concatenate([f.cache for f in parts]))


def backward_rows_parallel(x, h0, w_ih, w_hh, y, cache, dy, dhn, threads: int, dtype=np.float64) -> BackwardResult:
    """``backward`` with the batch rows split over ``threads`` threads: dx and
    dh0 rows are the per-row results, and the weight and bias gradients are
    the chunks' sums added in chunk order (the same sums as ``backward``,
    grouped by chunk)."""
    from concurrent.futures import ThreadPoolExecutor

    x, h0, y, cache = np.asarray(x), np.asarray(h0), np.asarray(y), np.asarray(cache)
    chunks = _row_chunks(x.shape[0], threads)

    def run(c):
        a, b = c
        return backward(x[a:b], h0[a:b], w_ih, w_hh, y[a:b], cache[a:b], None if dy is None else np.asarray(dy)[a:b],
                        None if dhn is None else np.asarray(dhn)[a:b], dtype=dtype)

    with ThreadPoolExecutor(len(chunks)) as ex:
        parts = list(ex.map(run, chunks))
    acc = {k: getattr(parts[0], k).copy() for k in ("dw_ih", "dw_hh", "db_ih", "db_hh")}
    for part in parts[1:]:
        for k in acc:
            acc[k] += getattr(part, k)
    return BackwardResult(np.concatenate([b.dx for b in parts]), np.concatenate([b.dh0 for b in parts]),
                          acc["dw_ih"], acc["dw_hh"], acc["db_ih"], acc["db_hh"])


@dataclass
class StackResult:
    y: np.ndarray                 # [B, T, H] output of the last layer
    hn: np.ndarray                # [L, B, H]
    dx: np.ndarray                # [B, T, I]
    dhx: np.ndarray               # [L, B, H]
    grads: List[dict]             # per layer: weight_ih/weight_hh/bias_ih/bias_hh


def stack_forward_backward(x, hx, params: Sequence[dict], dy, dhn=None, dtype=np.float64) -> StackResult:
    """Multi-layer forward + backward with nn.GRU parameter naming.

    ``params[l]`` holds ``weight_ih``, ``weight_hh``, ``bias_ih``, ``bias_hh``;
    ``hx`` is [L,B,H] or None (zeros); ``dy`` is the gradient of the last
    layer's output and ``dhn`` [L,B,H] (or None) the gradient of h_n.
    """
    L = len(params)
    x = np.asarray(x, dtype=dtype)
    B, T, _ = x.shape
    H = np.asarray(params[0]["weight_hh"]).shape[1]
    if hx is None:
        hx = np.zeros((L, B, H), dtype=dtype)
    layer_in, fwds, hns = [x], [], []
    for l in range(L):
        p = params[l]
        f = forward(layer_in[-1], hx[l], p["weight_ih"], p["weight_hh"], p["bias_ih"], p["bias_hh"], dtype=dtype)
        fwds.append(f)
        hns.append(f.hn)
        layer_in.append(f.y)
    grads: List[dict] = [None] * L  # type: ignore[list-item]
    dhx = np.zeros((L, B, H), dtype=dtype)
    g_out = np.asarray(dy, dtype=dtype)
    for l in reversed(range(L)):
        p = params[l]
        b = backward(layer_in[l], hx[l], p["weight_ih"], p["weight_hh"], fwds[l].y, fwds[l].cache,
                     g_out, None if dhn is None else dhn[l], dtype=dtype, need_dx=True)
        grads[l] = {"weight_ih": b.dw_ih, "weight_hh": b.dw_hh, "bias_ih": b.db_ih, "bias_hh": b.db_hh}
        dhx[l] = b.dh0
        g_out = b.dx
    return StackResult(fwds[-1].y, np.stack(hns, 0), g_out, dhx, grads)


def stack_rows_parallel(x, hx, params: Sequence[dict], dy_of, threads: int, dhn=None,
                        dtype=np.float64) -> StackResult:
    """``stack_forward_backward`` with the batch rows split over ``threads``
    threads.  ``dy_of(y, a, b)`` gives the gradient of the last layer's
    output for rows ``a:b`` from their output ``y`` (e.g. the MSE gradient
    against the target's rows), so that the gradient can depend on the
    forward's result.  Rows are independent sequences: y, h_n, dx and d hx
    are each row's own results, and every weight and bias gradient is the
    chunks' sums added in chunk order."""
    from concurrent.futures import ThreadPoolExecutor

    x = np.asarray(x)
    B = x.shape[0]
    L = len(params)
    chunks = _row_chunks(B, threads)

    def run(c):
        a, b = c
        hxc = None if hx is None else np.asarray(hx)[:, a:b]
        # forward of the stack for these rows, then the output gradient
        layer_in, fwds = [np.asarray(x[a:b], dtype=dtype)], []
        Hh = np.asarray(params[0]["weight_hh"]).shape[1]
        h0s = np.zeros((L, b - a, Hh), dtype=dtype) if hxc is None else np.asarray(hxc, dtype=dtype)
        for l in range(L):
            p = params[l]
            f = forward(layer_in[-1], h0s[l], p["weight_ih"], p["weight_hh"], p["bias_ih"], p["bias_hh"], dtype=dtype)
            fwds.append(f)
            layer_in.append(f.y)
        g_out = np.asarray(dy_of(fwds[-1].y, a, b), dtype=dtype)
        grads, dhx = [None] * L, np.zeros((L, b - a, Hh), dtype=dtype)
        for l in reversed(range(L)):
            p = params[l]
            bw = backward(layer_in[l], h0s[l], p["weight_ih"], p["weight_hh"], fwds[l].y, fwds[l].cache, g_out,
                          None if dhn is None else np.asarray(dhn)[l, a:b], dtype=dtype, need_dx=True)
            grads[l] = {"weight_ih": bw.dw_ih, "weight_hh": bw.dw_hh, "bias_ih": bw.db_ih, "bias_hh": bw.db_hh}
            dhx[l] = bw.dh0
            g_out = bw.dx
        return fwds[-1].y, np.stack([f.hn for f in fwds], 0), g_out, dhx, grads

    with ThreadPoolExecutor(len(chunks)) as ex:
        parts = list(ex.map(run, chunks))
    grads = [{k: v.copy() for k, v in parts[0][4][l].items()} for l in range(L)]
    for part in parts[1:]:
        for l in range(L):
            for k in grads[l]:
                grads[l][k] += part[4][l][k]
    return StackResult(np.concatenate([p[0] for p in parts]), np.concatenate([p[1] for p in parts], axis=1),
                       np.concatenate([p[2] for p in parts]), np.concatenate([p[3] for p in parts], axis=1), grads)


# ------------------------------------------------ harness-side operations ---
# float64 restatements of the benchmark harness's head, loss and optimiser
# (train_ops_oracle.c; reference rnn_benchmark.py:510,525,636,722).
def _load_train():
    lib = _load()
    if not getattr(lib, "_train_ready", False):
        D, P, I, SZ = ctypes.c_double, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
        lib.oracle_head_forward_f64.restype = None
        lib.oracle_head_forward_f64.argtypes = [I, I, P, P, D, P]
        lib.oracle_head_backward_f64.restype = None
        lib.oracle_head_backward_f64.argtypes = [I, I, P, P, P, P, P, P]
        lib.oracle_mse_forward_f64.restype = D
        lib.oracle_mse_forward_f64.argtypes = [SZ, P, P]
        lib.oracle_mse_backward_f64.restype = None
        lib.oracle_mse_backward_f64.argtypes = [SZ, P, P, D, P]
        lib.oracle_adamw_step_f64.restype = None
        lib.oracle_adamw_step_f64.argtypes = [SZ, P, P, P, P, D, D, D, D, D, I]
        lib._train_ready = True
    return lib


def head_forward(out, w, b) -> np.ndarray:
    """pred[r] = out[r] . w + b for out [..., H] (leading dims flattened)."""
    lib = _load_train()
    out = _c(out, np.float64)
    lead = out.shape[:-1]
    H = out.shape[-1]
    rows = int(np.prod(lead)) if lead else 1
    w = _c(np.reshape(w, (H,)), np.float64)
    pred = np.empty(rows, dtype=np.float64)
    lib.oracle_head_forward_f64(rows, H, _p(out), _p(w), float(np.reshape(b, (-1,))[0]), _p(pred))
    return pred.reshape(lead)


def head_backward(out, w, dpred, need_dout: bool = True):
    """Returns (dout [..., H] or None, dw [H], db scalar)."""
    lib = _load_train()
    out = _c(out, np.float64)
    H = out.shape[-1]
    rows = out.size // H
    w = _c(np.reshape(w, (H,)), np.float64)
    dpred = _c(np.reshape(dpred, (rows,)), np.float64)
    dout = np.empty_like(out) if need_dout else None
    dw = np.empty(H, dtype=np.float64)
    db = np.zeros(1, dtype=np.float64)
    lib.oracle_head_backward_f64(rows, H, _p(out), _p(w), _p(dpred), _p(dout), _p(dw), _p(db))
    return dout, dw, float(db[0])


def mse_forward(pred, target) -> float:
    lib = _load_train()
    pred, target = _c(pred, np.float64), _c(target, np.float64)
    assert pred.shape == target.shape
    return float(lib.oracle_mse_forward_f64(pred.size, _p(pred), _p(target)))


def mse_backward(pred, target, grad_loss: float = 1.0) -> np.ndarray:
    lib = _load_train()
    pred, target = _c(pred, np.float64), _c(target, np.float64)
    grad = np.empty_like(pred)
    lib.oracle_mse_backward_f64(pred.size, _p(pred), _p(target), float(grad_loss), _p(grad))
    return grad


def adamw_step(p, g, m, v, lr, beta1, beta2, eps, weight_decay, step):
    """One AdamW step; returns new (p, m, v) as float64 arrays."""
    lib = _load_train()
    p, g, m, v = (np.array(a, dtype=np.float64, copy=True) for a in (p, g, m, v))
    lib.oracle_adamw_step_f64(p.size, _p(p), _p(g), _p(m), _p(v), lr, beta1, beta2, eps, weight_decay, int(step))
    return p, m, v
