"""CPU-only checks of the host side: the C ABI library loads and exports every
symbol include/rnn_kernel_amd.h declares, module construction / validation
behaves like the reference's (error types and messages), and the drop-in
shims for the reference's import paths resolve."""
import ctypes
import json
import os
import re
import subprocess
import sys

import pytest
import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "rnn_kernel_amd.h")


def _declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rka_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_expected_entry_points():
    syms = _declared_symbols()
    for name in ("rka_gru_forward", "rka_gru_backward", "rka_gemm_f32", "rka_gru_recurrence_forward",
                 "rka_gru_recurrence_backward", "rka_last_error"):
        assert name in syms


def test_library_loads_and_exports_every_declared_symbol(hip_lib):
    from rnn_kernel_amd import _lib

    missing = [s for s in _declared_symbols() if not hasattr(hip_lib, s)]
    assert not missing, missing
    # the ctypes table covers every declared symbol, so no call goes unprototyped
    assert set(_declared_symbols()) <= set(_lib.SIGNATURES)


def test_library_size_queries_without_gpu(hip_lib):
    B, T, I, H = 64, 512, 256, 256
    assert hip_lib.rka_gru_reserve_bytes(B, T, H) == B * T * 4 * H * 4
    fwd = hip_lib.rka_gru_forward_workspace_bytes(B, T, I, H)
    assert fwd >= B * T * 3 * H * 4 + 2 * B * H * 8
    bwd = hip_lib.rka_gru_backward_workspace_bytes(B, T, I, H)
    assert bwd >= B * T * 4 * H * 4
    assert hip_lib.rka_gru_forward_workspace_bytes(0, T, I, H) == 0
    assert hip_lib.rka_version() == 2


def test_library_rejects_bad_arguments_without_touching_a_gpu(hip_lib):
    from rnn_kernel_amd import _lib

    rc = hip_lib.rka_gru_forward(*([None] * 10), 0, 0, 8, 4, 4, None)
    assert rc == 1001  # RKA_ERR_INVALID_ARGUMENT
    assert "must be >= 1" in _lib.last_error()
    rc = hip_lib.rka_gru_forward(*([None] * 10), 0, 2, 8, 4, 4, None)
    assert rc == 1001 and "null tensor pointer" in _lib.last_error()
    assert hip_lib.rka_set_recurrence_config(2, 0, 0, 0) == 1001   # bad direction
    assert hip_lib.rka_set_recurrence_config(0, 5, 0, 0) == 1001   # bad kind
    assert hip_lib.rka_set_recurrence_config(0, 1, 3, 0) == 1001   # units must divide 64
    assert hip_lib.rka_set_recurrence_config(1, 2, 0, 3) == 1001   # rows 1, 2 or 4
    assert hip_lib.rka_set_recurrence_config(0, 3, 0, 0) == 1001   # bad kind
    assert hip_lib.rka_set_recurrence_config(0, 4, 0, 0) == 1001   # bad kind
    assert hip_lib.rka_set_recurrence_config(0, 0, 0, 0) == 0
    assert hip_lib.rka_set_spin_limit(-1) == 1001
    assert hip_lib.rka_set_spin_limit((1 << 30) + 1) == 1001   # above the largest poll bound
    assert hip_lib.rka_recurrence_abort_count(None) == 1001
    assert hip_lib.rka_set_stall_block(-2) == 1001
    assert hip_lib.rka_set_stall_block(-1) == 0
    assert hip_lib.rka_set_spin_limit(0) == 0
    out = (ctypes.c_int * 2)()
    assert hip_lib.rka_describe_recurrence(0, 4, 16, out, 0) == 1001  # n_out must be >= 1
    assert hip_lib.rka_describe_recurrence(2, 4, 16, out, 2) == 1001  # bad direction
    rt, same = ctypes.c_double(0), ctypes.c_int(0)
    assert hip_lib.rka_measure_exchange_latency(0, 10, None, 0, ctypes.byref(rt), ctypes.byref(same)) == 1001
    assert hip_lib.rka_exchange_probe_workspace_bytes(0) == 0 and hip_lib.rka_exchange_probe_workspace_bytes(128) > 0
    ns, tf = ctypes.c_double(0), ctypes.c_double(0)
    assert hip_lib.rka_measure_fma_rate(None, 0, None, ctypes.byref(tf)) == 1001  # null output
    assert hip_lib.rka_set_gemm_tiles(2) == 1001
    assert hip_lib.rka_set_gemm_tiles(-1) == 1001
    assert hip_lib.rka_set_gemm_tiles(1) == 0 and hip_lib.rka_set_gemm_tiles(0) == 0
    assert hip_lib.rka_set_exchange_stores(2) == 1001
    assert hip_lib.rka_set_exchange_stores(-1) == 1001
    assert hip_lib.rka_set_exchange_stores(1) == 0 and hip_lib.rka_set_exchange_stores(0) == 0


def test_backward_workspace_holds_gate_gradients_exchange_and_partials(hip_lib):
    """The backward workspace holds the G buffer [B,T,4H], the recurrence's
    exchange state and the split-K partials of both weight-gradient products."""
    B, T, I, H = 64, 100, 256, 256
    need = hip_lib.rka_gru_backward_workspace_bytes(B, T, I, H)
    g_bytes = B * T * 4 * H * 4
    assert need > g_bytes + hip_lib.rka_gru_recurrence_workspace_bytes(B, H) + 2 * 3 * H * H * 4


def test_module_construction_and_validation_messages():
    from rnn_kernel_amd import GRU, MAX_HIDDEN_SIZE

    m = GRU(16)
    assert m.hidden_size == 256 and m.num_layers == 1
    names = [n for n, _ in m.named_parameters()]
    assert names == ["weight_ih_l0", "weight_hh_l0", "bias_ih_l0", "bias_hh_l0"]
    bound = 1.0 / 256 ** 0.5
    assert all(p.abs().max() <= bound for p in m.parameters())
    with pytest.raises(ValueError, match="hidden_size"):
        GRU(4, hidden_size=MAX_HIDDEN_SIZE + 1)
    with pytest.raises(ValueError, match="num_layers"):
        GRU(4, num_layers=0)
    with pytest.raises(ValueError, match="batch_first"):
        GRU(4, batch_first=False)
    with pytest.raises(ValueError, match="bias=True"):
        GRU(4, bias=False)
    with pytest.raises(ValueError, match="dropout=0"):
        GRU(4, dropout=0.1)


def test_state_dict_is_interchangeable_with_nn_gru():
    from rnn_kernel_amd import GRU

    ref = torch.nn.GRU(5, 12, num_layers=3, batch_first=True)
    ours = GRU(5, 12, num_layers=3)
    ours.load_state_dict(ref.state_dict())
    for name, p in ref.named_parameters():
        assert torch.equal(getattr(ours, name), p)


def test_from_torch_gru_support_matrix():
    from rnn_kernel_amd import from_torch_gru, is_supported_gru

    ok = torch.nn.GRU(256, 256, num_layers=2, batch_first=True)
    assert is_supported_gru(ok)
    ours = from_torch_gru(ok)
    assert torch.equal(ours.weight_hh_l1, ok.weight_hh_l1)
    for bad in (torch.nn.GRU(4, 8, batch_first=False), torch.nn.GRU(4, 8, batch_first=True, bidirectional=True),
                torch.nn.GRU(4, 8, num_layers=2, batch_first=True, dropout=0.1),
                torch.nn.GRU(4, 8, batch_first=True, bias=False), torch.nn.GRU(4, 8, batch_first=True).double(),
                torch.nn.LSTM(4, 8, batch_first=True)):
        assert not is_supported_gru(bad)
        with pytest.raises(ValueError, match="batch_first fp32 GRU"):
            from_torch_gru(bad)


def test_forward_rejects_cpu_tensors_loudly():
    """No CPU fallback: a CPU input is a RuntimeError, as in the reference."""
    from rnn_kernel_amd import GRU, GRUFunction

    m = GRU(4, 8)
    with pytest.raises(RuntimeError, match="GPU"):
        m(torch.randn(2, 3, 4))
    with torch.no_grad(), pytest.raises(RuntimeError, match="GPU"):
        m(torch.randn(2, 3, 4))
    with pytest.raises(ValueError, match="hx must have shape"):
        m(torch.randn(2, 3, 4), torch.zeros(2, 2, 8))
    args = [torch.randn(2, 3, 4), torch.zeros(2, 8)] + [p for p in m.parameters()]
    with pytest.raises(RuntimeError, match="GPU"):
        GRUFunction.apply(*args)


def test_is_available_false_without_gpu():
    from rnn_kernel_amd import is_available

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    assert is_available() is False
    assert is_available("cpu") is False


def test_drop_in_shims_resolve_reference_import_paths():
    """rnn_benchmark.py imports rnn_kernel.custom_gru.CustomGRU and
    rnn_kernel.a100.A100GRUH256; the prod tests import rnn_kernel.a100.prod."""
    from rnn_kernel.a100 import A100GRUH256
    from rnn_kernel.a100.prod import A100GRU, from_torch_gru, is_a100_available, is_supported_gru
    from rnn_kernel.custom_gru import CustomGRU, copy_from_torch_gru
    import rnn_kernel_amd

    assert A100GRU is rnn_kernel_amd.GRU or issubclass(A100GRU, rnn_kernel_amd.GRU)
    assert not is_a100_available(torch.device("cpu"))
    # rnn_benchmark.py passes block_threads and ~55 variant booleans; they are accepted and ignored.
    m = A100GRUH256(input_size=16, hidden_size=256, num_layers=2, batch_first=True, block_threads=256,
                    use_recurrent_backward_kernel=False,
                    use_persistent_state6_gate_cache_tiled_weight_shmem_split0_keep_unroll8_backward_kernel=True)
    assert isinstance(m, rnn_kernel_amd.GRU) and m.num_layers == 2
    c = CustomGRU(4, 7, 2)
    ref = torch.nn.GRU(4, 7, num_layers=2, batch_first=True)
    copy_from_torch_gru(c, ref)
    assert torch.equal(c.weight_ih_l1, ref.weight_ih_l1)
    assert is_supported_gru(ref) and from_torch_gru(ref).num_layers == 2


def test_prod_import_does_not_pull_in_build_tools_or_oracle():
    """Mirror of the reference's import-isolation test (tests/test_a100_prod.py:52-81):
    importing the product must not import the oracle, the build helper or hipcc tooling."""
    env = dict(os.environ, PYTHONPATH=f"{REPO}:{REPO}/src:" + os.environ.get("PYTHONPATH", ""))
    script = (
        "import json, sys, torch\n"
        "from rnn_kernel.a100.prod import A100GRU, from_torch_gru\n"
        "import rnn_kernel_amd\n"
        "print(json.dumps({'oracle': any(m.startswith('oracle') for m in sys.modules),"
        " 'build': 'rnn_kernel_amd.build' in sys.modules}))\n"
    )
    out = subprocess.run([sys.executable, "-c", script], check=True, env=env, text=True, capture_output=True)
    assert json.loads(out.stdout.strip().splitlines()[-1]) == {"oracle": False, "build": False}


def test_build_compiles_every_source_with_the_pool_flags():
    """Every .hip source under csrc is built; per-file flags name built sources
    only and add to, never replace, the common flags (packed fp32 ops stay
    off for every translation unit)."""
    from rnn_kernel_amd import build as rka_build

    on_disk = sorted(f for f in os.listdir(rka_build.CSRC) if f.endswith(".hip"))
    assert sorted(rka_build.SOURCES) == on_disk
    assert set(rka_build.EXTRA_FLAGS) <= set(rka_build.SOURCES)
    common = rka_build.compile_flags()
    assert "-packed-fp32-ops" in common and f"--offload-arch={rka_build.ARCH}" in common
    for flags in rka_build.EXTRA_FLAGS.values():
        assert all(f not in ("-O0", "-O1", "-O2") and not f.startswith("--offload-arch") for f in flags)
