"""ctypes binding of librnn_kernel_amd.so (the C ABI in include/rnn_kernel_amd.h).

The reference launches its kernels through cuda-python's driver API with raw
pointers on torch's current stream (src/rnn_kernel/a100/prod/gru.py:265-300);
this module is the equivalent thin layer over the HIP library.  There is no
fallback: if the library is missing or fails to load, every call raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG_DIR, "librnn_kernel_amd.so")

# Every exported symbol with (restype, argtypes).
_P = ctypes.c_void_p
_I = ctypes.c_int
_SZ = ctypes.c_size_t
SIGNATURES = {
    "rka_version": (_I, []),
    "rka_last_error": (ctypes.c_char_p, []),
    "rka_device_supported": (_I, [_I]),
    "rka_gru_reserve_bytes": (_SZ, [_I, _I, _I]),
    "rka_gru_forward_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "rka_gru_forward": (_I, [_P] * 9 + [_P, _SZ, _I, _I, _I, _I, _P]),
    "rka_gru_backward_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "rka_gru_backward": (_I, [_P] * 14 + [_P, _SZ, _I, _I, _I, _I, _P]),
    "rka_gemm_f32": (_I, [_I, _I, _I, _P, _I, _I, _P, _I, _I, _P, _P, _I, _P]),
    "rka_gru_recurrence_workspace_bytes": (_SZ, [_I, _I]),
    "rka_gru_recurrence_forward": (_I, [_P] * 7 + [_P, _SZ, _I, _I, _I, _P]),
    "rka_gru_recurrence_forward_noalloc": (_I, [_P] * 7 + [_I, _I, _I, _P]),
    "rka_gru_recurrence_backward": (_I, [_P] * 8 + [_P, _SZ, _I, _I, _I, _P]),
    "rka_set_recurrence_config": (_I, [_I, _I, _I, _I]),
    "rka_set_spin_limit": (_I, [_I]),
    "rka_set_gemm_tiles": (_I, [_I]),
    "rka_set_exchange_stores": (_I, [_I]),
    "rka_recurrence_abort_count": (_I, [ctypes.POINTER(ctypes.c_ulonglong)]),
    "rka_set_stall_block": (_I, [_I]),
    "rka_describe_recurrence": (_I, [_I, _I, _I, ctypes.POINTER(_I), _I]),
    "rka_eval_gate_functions": (_I, [_P, _P, _P, _I, _P]),
    "rka_exchange_probe_workspace_bytes": (_SZ, [_I]),
    "rka_measure_exchange_latency": (_I, [_I, _I, _P, _SZ, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_I)]),
    "rka_fma_probe_workspace_bytes": (_SZ, []),
    "rka_measure_fma_rate": (_I, [_P, _SZ, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
    "rka_profile_enable": (_I, [_I]),
    "rka_profile_read": (_I, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_I)]),
    "rka_profile_stage_name": (ctypes.c_char_p, [_I]),
    "rka_mse_workspace_bytes": (_SZ, [_SZ]),
    "rka_mse_forward": (_I, [_P, _P, _P, _P, _SZ, _SZ, _P]),
    "rka_mse_backward": (_I, [_P, _P, _P, _P, _SZ, _P]),
    "rka_head_forward": (_I, [_P, _P, _P, _P, _I, _I, _P]),
    "rka_head_backward_workspace_bytes": (_SZ, [_I, _I]),
    "rka_head_backward": (_I, [_P] * 7 + [_SZ, _I, _I, _P]),
    "rka_adamw_step": (_I, [ctypes.POINTER(_P)] * 4 + [ctypes.POINTER(_SZ), _I] + [ctypes.c_double] * 5 + [_I, _P]),
}
NUM_STAGES = 6

_lib: Optional[ctypes.CDLL] = None
_lock = threading.Lock()


class RKAError(RuntimeError):
    """A nonzero status returned by the HIP library."""


def load() -> ctypes.CDLL:
    """Load the library (after torch, so it binds torch's HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        import torch  # noqa: F401  (binds libamdhip64.so.7 to torch's copy first)

        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"rnn_kernel_amd HIP library not built: {LIB_PATH} is missing. "
                "Build it with `python -m rnn_kernel_amd.build` (hipcc, gfx950)."
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def last_error() -> str:
    msg = load().rka_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RKAError(f"{what} failed with status {rc}: {last_error()}")


def ptr(t) -> Optional[int]:
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else t.data_ptr()


def profile_enable(on: bool) -> None:
    check(load().rka_profile_enable(1 if on else 0), "rka_profile_enable")


def profile_read() -> dict:
    """{stage name: (total ms, launches)} since the last read; waits for the
    recorded events."""
    lib = load()
    ms = (ctypes.c_double * NUM_STAGES)()
    cnt = (ctypes.c_int * NUM_STAGES)()
    check(lib.rka_profile_read(ms, cnt), "rka_profile_read")
    return {lib.rka_profile_stage_name(i).decode(): (ms[i], cnt[i]) for i in range(NUM_STAGES)}


REC_KINDS = {0: "auto", 1: "tiled", 2: "register"}


def describe_recurrence(direction: int, batch: int, hidden: int) -> dict:
    """Decomposition the next recurrence call would use (0 forward, 1 backward)."""
    out = (ctypes.c_int * 10)()
    check(load().rka_describe_recurrence(direction, batch, hidden, out, 10), "rka_describe_recurrence")
    keys = ("kind", "groups", "slices", "units", "rows", "pair_waves", "chunk", "lds_bytes", "launches",
            "batch_per_launch")
    d = dict(zip(keys, list(out)))
    d["kind"] = REC_KINDS.get(d["kind"], d["kind"])
    return d


def set_recurrence_config(direction: int, kind: int = 0, units: int = 0, param: int = 0) -> None:
    check(load().rka_set_recurrence_config(direction, kind, units, param), "rka_set_recurrence_config")


def set_spin_limit(polls: int) -> None:
    """Poll rounds a recurrence wait makes before it gives up (0 = the
    default, 2^24); see rka_set_spin_limit."""
    check(load().rka_set_spin_limit(polls), "rka_set_spin_limit")


def set_gemm_tiles(mode: int) -> None:
    """GEMM tile families: 0 = automatic (large persistent tiles where they
    divide evenly), 1 = 128x128 everywhere; see rka_set_gemm_tiles."""
    check(load().rka_set_gemm_tiles(mode), "rka_set_gemm_tiles")


def set_exchange_stores(mode: int) -> None:
    """Recurrence exchange stores: 0 = automatic (XCD-local plain stores
    when a group shares one XCD), 1 = agent scope always; see
    rka_set_exchange_stores."""
    check(load().rka_set_exchange_stores(mode), "rka_set_exchange_stores")


def set_stall_block(block: int) -> None:
    """Failure injection for tests (-1 = off); see rka_set_stall_block."""
    check(load().rka_set_stall_block(block), "rka_set_stall_block")


def recurrence_abort_count() -> int:
    """Aborted recurrence calls on the current device so far (synchronises
    the device); see rka_recurrence_abort_count."""
    n = ctypes.c_ulonglong(0)
    check(load().rka_recurrence_abort_count(ctypes.byref(n)), "rka_recurrence_abort_count")
    return int(n.value)


def measure_exchange_latency(pairs: int = 128, iters: int = 2000) -> dict:
    """Mean round trip (ns) of the recurrences' cross-workgroup exchange,
    measured by a ping-pong of `pairs` workgroup pairs on the current device;
    see rka_measure_exchange_latency."""
    import torch

    lib = load()
    nbytes = lib.rka_exchange_probe_workspace_bytes(pairs)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    rt = ctypes.c_double(0.0)
    same = ctypes.c_int(0)
    check(lib.rka_measure_exchange_latency(pairs, iters, ws.data_ptr(), nbytes, ctypes.byref(rt), ctypes.byref(same)),
          "rka_measure_exchange_latency")
    return {"round_trip_ns": rt.value, "same_xcd": bool(same.value), "pairs": pairs, "iters": iters}


def measure_fma_rate() -> dict:
    """Issue rate of non-packed fp32 FMAs on the current device (ns per wave64
    instruction per SIMD, TFLOP/s over the device); see rka_measure_fma_rate."""
    import torch

    lib = load()
    nbytes = lib.rka_fma_probe_workspace_bytes()
    if nbytes == 0:
        raise RuntimeError("rka_fma_probe_workspace_bytes: no device")
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    ns = ctypes.c_double(0.0)
    tf = ctypes.c_double(0.0)
    check(lib.rka_measure_fma_rate(ws.data_ptr(), nbytes, ctypes.byref(ns), ctypes.byref(tf)), "rka_measure_fma_rate")
    return {"ns_per_instruction": ns.value, "tflops": tf.value}
