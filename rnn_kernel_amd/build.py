"""Build librnn_kernel_amd.so (HIP, gfx950) in-tree with hipcc.

Usage: ``python -m rnn_kernel_amd.build`` (or ``__graft_entry__.build()``).
The library is written next to this file so that it travels with the source
tree; it links the HIP runtime by SONAME (libamdhip64.so.7), which resolves to
the runtime PyTorch already loaded when imported after ``torch``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_NAME = "librnn_kernel_amd.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
SOURCES = ["rka_capi.hip", "gemm_f32.hip", "gru_recurrence.hip", "gru_rec_tiled.hip", "gru_rec_reg.hip",
           "gru_rec_bwd1.hip", "gru_rec_fwd1.hip", "train_ops.hip", "probes.hip"]
ARCH = "gfx950"
# Flags of single sources on top of compile_flags().  The machine-scheduler
# strategy is an option per translation unit: the one-row kernels that
# measured faster under another strategy sit in files of their own (see
# their headers).
EXTRA_FLAGS = {
    "gru_rec_bwd1.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"],
    "gru_rec_fwd1.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-minreg"],
}


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; set HIPCC or install ROCm")


def compile_flags() -> list:
    return [
        "-O3",
        "-std=c++17",
        "-fPIC",
        f"--offload-arch={ARCH}",
        # Packed fp32 VALU ops are kept off on this pool (known-bad forms);
        # the hot dot products are written as scalar fmaf chains.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-command-line-argument",
        # Loop heads on 64-byte boundaries: without it a kernel's k loop moved
        # with every change to the code in front of it (the dx GEMM at c2 ran
        # 2 us slower after four scalar instructions left its prologue).
        "-falign-loops=64",
    ]


def _run(cmds: list, verbose: bool) -> None:
    """Runs the commands concurrently; raises if any fails."""
    procs = []
    for cmd in cmds:
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append(subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True))
    failed = None
    for proc in procs:
        out, err = proc.communicate()
        if proc.returncode != 0 and failed is None:
            failed = proc.returncode
            sys.stderr.write(out + err)
        elif verbose and err.strip():
            sys.stderr.write(err)
    if failed is not None:
        raise RuntimeError(f"hipcc failed with exit code {failed}")


def build(verbose: bool = False) -> str:
    """Compile every source (one object each, concurrently) and link the shared
    library; returns its path."""
    hipcc = hipcc_path()
    tmp = LIB_PATH + ".tmp"
    objdir = tempfile.mkdtemp(prefix="rka_build_")
    try:
        objs = [os.path.join(objdir, s + ".o") for s in SOURCES]
        _run([[hipcc] + compile_flags() + EXTRA_FLAGS.get(s, []) + ["-c", os.path.join(CSRC, s), "-o", o]
              for s, o in zip(SOURCES, objs)], verbose)
        _run([[hipcc] + compile_flags() + ["-shared", "-o", tmp] + objs], verbose)
    finally:
        shutil.rmtree(objdir, ignore_errors=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
