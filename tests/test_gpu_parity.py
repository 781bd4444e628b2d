"""Parity of the HIP path (through the C ABI) with the CPU oracle and with
torch.nn.GRU fp32 on the same GPU.

Tolerances (stated by the north star): outputs and h_n within max-abs 1e-4;
gradients within max|g - g_ref| / max|g_ref| <= 1e-3 per tensor.  Small shapes
are checked against the float64 oracle; the BASELINE configurations are
checked against torch.nn.GRU fp32 (TF32 off) on the same GPU and, for a
subset of batch rows, against the float64 oracle.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

OUT_ATOL = 1e-4
GRAD_REL = 1e-3


def _rel(a, b):
    a = a.detach().double().cpu()
    b = torch.as_tensor(b).double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def _maxabs(a, b):
    return float((a.detach().double().cpu() - torch.as_tensor(b).double().cpu()).abs().max())


def _no_tf32():
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False


# ------------------------------------------------------------------ GEMM ---
# (1000, 390, 70): eight row panels, so the XCD-aware tile order, with edge
# tiles along both m and n and a k that is not a multiple of 16
GEMM_SHAPES = [(128, 128, 16), (300, 200, 50), (1, 1, 1), (4096, 768, 256), (129, 387, 130), (768, 256, 4096),
               (1000, 390, 70)]


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
@pytest.mark.parametrize("a_kmajor,b_kmajor", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_matches_float64(gpu, hip_lib, m, n, k, a_kmajor, b_kmajor):
    from rnn_kernel_amd import _lib

    print(f"gemm m={m} n={n} k={k} a_kmajor={a_kmajor} b_kmajor={b_kmajor}", flush=True)
    g = torch.Generator().manual_seed(m * 7 + n * 3 + k)
    A = torch.randn(m, k, generator=g)
    Bm = torch.randn(n, k, generator=g)
    bias = torch.randn(n, generator=g)
    ref = A.double() @ Bm.double().T + bias.double()
    a_store = (A.T if a_kmajor else A).contiguous().to(gpu)
    b_store = (Bm.T if b_kmajor else Bm).contiguous().to(gpu)
    lda = m if a_kmajor else k
    ldb = n if b_kmajor else k
    c = torch.full((m, n), float("nan"), device=gpu)
    rc = hip_lib.rka_gemm_f32(m, n, k, a_store.data_ptr(), lda, a_kmajor, b_store.data_ptr(), ldb, b_kmajor,
                              bias.to(gpu).data_ptr(), c.data_ptr(), n, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "rka_gemm_f32")
    torch.cuda.synchronize()
    err = (c.double().cpu() - ref).abs().max().item()
    assert err <= 1e-6 * k + 1e-5, err


@pytest.fixture
def gemm_tiles(hip_lib):
    """Restores the automatic GEMM tile choice after a test that forces one."""
    from rnn_kernel_amd import _lib

    yield _lib.set_gemm_tiles
    _lib.set_gemm_tiles(0)


def test_layer_backward_large_tiles_match_128_tiles(gpu, hip_lib, gemm_tiles):
    """A c2-shaped layer (B=64, T=512, I=H=256) runs its weight-gradient pair
    in 192x256 tiles; every output and gradient equals the 128x128 kernels'
    bit for bit."""
    from rnn_kernel_amd import GRU

    print("layer large tiles vs 128 tiles B=64 T=512 I=H=256", flush=True)
    torch.manual_seed(7)
    model = GRU(256, 256).to(gpu)
    x = torch.randn(64, 512, 256, device=gpu)
    h0 = 0.1 * torch.randn(1, 64, 256, device=gpu)
    results = []
    for mode in (0, 1):
        gemm_tiles(mode)
        model.zero_grad()
        xi = x.clone().requires_grad_(True)
        y, hn = model(xi, h0)
        (y.sin().sum() + hn.sum()).backward()
        torch.cuda.synchronize()
        results.append([y.detach().clone(), hn.detach().clone(), xi.grad.clone()] +
                       [p.grad.clone() for p in model.parameters()])
    for a, b in zip(*results):
        assert torch.equal(a, b)


@pytest.mark.parametrize("B,T,I,H", [(64, 512, 256, 256), (5, 7, 3, 33), (16, 9, 8, 130)])
def test_weight_gradients_with_and_without_dx_agree_bitwise(gpu, hip_lib, B, T, I, H):
    """With dx the weight-gradient reductions run in the input-gradient GEMM's
    launch; without it (x needs no gradient) in a launch of their own.  The
    weight and bias gradients are equal bit for bit."""
    from rnn_kernel_amd import GRUFunction

    print(f"dW with / without dx B={B} T={T} I={I} H={H}", flush=True)
    p, x, h0, dy, dhn = _layer_inputs(B, T, I, H, seed=B + T + I + H)
    results = []
    for need_dx in (True, False):
        xd = x.to(gpu).requires_grad_(need_dx)
        h0d = h0.to(gpu).requires_grad_(True)
        pd = {k: v.to(gpu).requires_grad_(True) for k, v in p.items()}
        y, hn = GRUFunction.apply(xd, h0d, pd["weight_ih"], pd["weight_hh"], pd["bias_ih"], pd["bias_hh"])
        torch.autograd.backward([y, hn], [dy.to(gpu), dhn.to(gpu)[None]])
        torch.cuda.synchronize()
        assert (xd.grad is not None) == need_dx
        results.append([h0d.grad] + [pd[k].grad for k in sorted(pd)])
    for a, b in zip(*results):
        assert torch.equal(a, b)


def test_gemm_unaligned_operands_use_scalar_path(gpu, hip_lib):
    """Operands offset by one float (not 16-byte aligned) and odd leading dims."""
    from rnn_kernel_amd import _lib

    m, n, k = 77, 45, 33
    g = torch.Generator().manual_seed(5)
    A = torch.randn(m, k + 3, generator=g)
    Bm = torch.randn(n, k + 3, generator=g)
    ref = A[:, 1:k + 1].double() @ Bm[:, 1:k + 1].double().T
    ad, bd = A.to(gpu), Bm.to(gpu)
    c = torch.empty(m, n + 2, device=gpu)
    rc = hip_lib.rka_gemm_f32(m, n, k, ad.data_ptr() + 4, k + 3, 0, bd.data_ptr() + 4, k + 3, 0, None,
                              c.data_ptr(), n + 2, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "rka_gemm_f32")
    torch.cuda.synchronize()
    assert (c[:, :n].double().cpu() - ref).abs().max().item() < 1e-4


def test_gemm_rejects_leading_dimensions_from_2_pow_22(gpu, hip_lib):
    """The tile loads form 32-bit offsets from a wave-uniform base, which holds
    for leading dimensions below 2^22 floats; larger ones are refused before
    anything is launched (the buffers here are far smaller than such a
    leading dimension would imply, and are never read)."""
    a = torch.zeros(64, device=gpu)
    c = torch.zeros(16, device=gpu)
    stream = torch.cuda.current_stream().cuda_stream
    for lda, ldb in [(1 << 22, 4), (4, 1 << 22), (-1, 4)]:
        rc = hip_lib.rka_gemm_f32(4, 4, 4, a.data_ptr(), lda, 0, a.data_ptr(), ldb, 0, None, c.data_ptr(), 4, stream)
        assert rc == 1004, (lda, ldb, rc)
    torch.cuda.synchronize()
    assert torch.equal(c, torch.zeros_like(c))


# extents that are multiples of 4 (so the aligned storage takes the float4
# paths), with edge tiles along m and n, k-tails and, at m = 1000, eight row
# panels
UNALIGNED_SHAPES = [(300, 200, 52), (132, 388, 132), (1000, 392, 72), (256, 256, 64)]


@pytest.mark.parametrize("m,n,k", UNALIGNED_SHAPES)
@pytest.mark.parametrize("a_kmajor,b_kmajor", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_unaligned_storage_matches_aligned_bitwise(gpu, hip_lib, m, n, k, a_kmajor, b_kmajor):
    """An operand whose leading dimension is odd and whose base is one float
    past a 16-byte boundary is staged one float per lane; the values land in
    the same LDS places and meet the MFMAs in the same order as the float4
    paths', so the product equals that of the same matrices in aligned
    storage bit for bit (either operand unaligned, or both)."""
    from rnn_kernel_amd import _lib

    print(f"gemm storage m={m} n={n} k={k} a_kmajor={a_kmajor} b_kmajor={b_kmajor}", flush=True)
    g = torch.Generator().manual_seed(m + 5 * n + 11 * k)
    A = torch.randn(m, k, generator=g)
    Bm = torch.randn(n, k, generator=g)
    bias = torch.randn(n, generator=g).to(gpu)
    stream = torch.cuda.current_stream().cuda_stream

    def stored(M, kmajor, unaligned):
        """(buffer, byte offset, leading dimension) of M [rows, k] in the given layout."""
        S = (M.T if kmajor else M).contiguous()
        ld = S.shape[1] + (1 if unaligned else 0)
        buf = torch.zeros(S.shape[0] * ld + 8, device=gpu)
        off = 1 if unaligned else 0
        buf[off:off + S.shape[0] * ld].view(S.shape[0], ld)[:, :S.shape[1]] = S.to(gpu)
        return buf, 4 * off, ld

    outs = {}
    for ua_a, ua_b in [(0, 0), (1, 0), (0, 1), (1, 1)]:
        a_buf, a_off, lda = stored(A, a_kmajor, ua_a)
        b_buf, b_off, ldb = stored(Bm, b_kmajor, ua_b)
        c = torch.full((m, n), float("nan"), device=gpu)
        rc = hip_lib.rka_gemm_f32(m, n, k, a_buf.data_ptr() + a_off, lda, a_kmajor, b_buf.data_ptr() + b_off, ldb,
                                  b_kmajor, bias.data_ptr(), c.data_ptr(), n, stream)
        _lib.check(rc, "rka_gemm_f32")
        outs[(ua_a, ua_b)] = c
    torch.cuda.synchronize()
    ref = A.double() @ Bm.double().T + bias.double().cpu()
    assert (outs[(0, 0)].double().cpu() - ref).abs().max().item() <= 1e-6 * k + 1e-5
    for key, c in outs.items():
        assert torch.equal(c, outs[(0, 0)]), key


# ------------------------------------------------- gate nonlinearities ---
def test_gate_functions_accuracy_against_float64(gpu, hip_lib):
    """The recurrence kernels evaluate sigmoid / tanh from their definitions on
    the hardware exp2 / rcp units; bound their error over the range that
    matters (saturated tails included) against float64."""
    from rnn_kernel_amd import _lib

    x = torch.cat([torch.linspace(-30, 30, 200001), torch.tensor([0.0, -0.0, 1e-30, -1e-30, 1e-6, -1e-6, 88.0,
                                                                  -88.0, 200.0, -200.0, float("inf"), float("-inf")])])
    xd = x.to(gpu)
    sig = torch.empty_like(xd)
    th = torch.empty_like(xd)
    rc = hip_lib.rka_eval_gate_functions(xd.data_ptr(), sig.data_ptr(), th.data_ptr(), x.numel(),
                                         torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "rka_eval_gate_functions")
    torch.cuda.synchronize()
    x64 = x.double()
    ref_sig = torch.sigmoid(x64)
    ref_th = torch.tanh(x64)
    err_sig = (sig.double().cpu() - ref_sig).abs().max().item()
    err_th = (th.double().cpu() - ref_th).abs().max().item()
    print(f"gate functions: max abs err sigmoid {err_sig:.3e} tanh {err_th:.3e}", flush=True)
    assert err_sig <= 2.5e-7 and err_th <= 5e-7
    assert torch.all((sig >= 0) & (sig <= 1)) and torch.all((th >= -1) & (th <= 1))


# ------------------------------------------- single layer vs the oracle ---
LAYER_SHAPES = [
    # B, T, I, H
    (2, 8, 16, 16),
    (3, 5, 4, 129),      # odd H tails
    (2, 7, 3, 130),
    (64, 16, 256, 256),  # BASELINE config 2 width, short T
    (5, 3, 2, 1),        # H = 1
    (1, 1, 1, 64),       # single step, single row
    (9, 6, 5, 96),       # batch not a multiple of the row group
    (3, 6, 5, 200),      # four slices, the last one partial (float4 weight loads)
    (2, 5, 3, 221),      # four slices, H not a multiple of 4 (scalar weight loads)
    (4, 4, 2, 193),      # four slices, one unit in the last
    (300, 3, 8, 256),    # B x 4 workgroups not resident: four rows per workgroup, two batch-slice launches
    (130, 4, 6, 130),    # three slices, two rows per workgroup
    (400, 5, 4, 160),    # three slices at four rows not resident: batch-slice launches of 80 groups
    (1, 3, 4, 768),      # the largest hidden size at one batch row (LDS-tiled, one unit per workgroup)
    (8, 512, 135, 133),  # weight gradients' last 5 (dW_hh) / 7 (dW_ih) columns summed apart from the tiles,
                         # k = B T = 4096 in 32 chunks (c3 at H = 129, 130 runs chunks of two 256-deep slabs)
    (2, 70, 136, 136),   # ... 8 columns each, k = 140: one chunk ending inside its slab
]


def _as_reserve(cache):
    """The oracle's gate cache [B, T, 4H] (blocks r, z, n, a_n) in the
    library's reserve layout [B, T, H, 4] (the four values of a unit
    contiguous)."""
    c = torch.as_tensor(cache)
    B, T, H4 = c.shape
    return c.reshape(B, T, 4, H4 // 4).transpose(2, 3).reshape(B, T, H4)


def _layer_inputs(B, T, I, H, seed, h0_scale=1.0):
    g = torch.Generator().manual_seed(seed)
    k = 1.0 / H ** 0.5
    p = {
        "weight_ih": (torch.rand(3 * H, I, generator=g) * 2 - 1) * k,
        "weight_hh": (torch.rand(3 * H, H, generator=g) * 2 - 1) * k,
        "bias_ih": (torch.rand(3 * H, generator=g) * 2 - 1) * k,
        "bias_hh": (torch.rand(3 * H, generator=g) * 2 - 1) * k,
    }
    x = torch.randn(B, T, I, generator=g)
    h0 = h0_scale * torch.randn(B, H, generator=g)
    dy = torch.randn(B, T, H, generator=g)
    dhn = torch.randn(B, H, generator=g)
    return p, x, h0, dy, dhn


@pytest.fixture(params=["auto", "tiled"])
def rec_kind(request, hip_lib):
    """Run a test with the automatic recurrence choice (register-resident for
    H <= 256) and again with the LDS-tiled kernels forced."""
    from rnn_kernel_amd import _lib

    if request.param == "tiled":
        for d in (0, 1):
            _lib.set_recurrence_config(d, 1, 0, 0)
    yield request.param
    for d in (0, 1):
        _lib.set_recurrence_config(d, 0, 0, 0)


@pytest.mark.parametrize("B,T,I,H", LAYER_SHAPES + [(3, 4, 8, 320), (2, 3, 5, 512), (64, 3, 16, 768), (200, 2, 8, 768),
                                     (256, 2, 8, 512), (83, 4, 8, 130), (256, 6, 16, 256), (64, 1, 1, 256),
                                     (48, 4, 8, 96), (16, 4, 8, 224)])
def test_layer_forward_backward_matches_oracle(gpu, oracle, rec_kind, B, T, I, H):
    _check_layer_against_oracle(gpu, oracle, rec_kind, B, T, I, H)


@pytest.fixture
def agent_stores(hip_lib):
    """Forces agent-scope exchange stores for one test, then restores the
    automatic choice."""
    from rnn_kernel_amd import _lib

    _lib.set_exchange_stores(1)
    yield "agent-scope stores"
    _lib.set_exchange_stores(0)


# register (H <= 256) and tiled (H = 512) recurrences; G = 1, 3, 4, 5 and 64 groups
AGENT_SHAPES = [(1, 5, 8, 256), (3, 5, 7, 130), (4, 6, 8, 256), (5, 4, 8, 512), (64, 4, 16, 256)]


@pytest.mark.parametrize("B,T,I,H", AGENT_SHAPES)
def test_layer_with_agent_scope_exchange_matches_oracle(gpu, oracle, agent_stores, B, T, I, H):
    """Every launch publishes with agent-scope stores (the path a group whose
    workgroups span XCDs takes): the layer still matches the oracle."""
    _check_layer_against_oracle(gpu, oracle, agent_stores, B, T, I, H)


@pytest.mark.parametrize("B,T,I,H", AGENT_SHAPES)
def test_exchange_store_paths_agree_bitwise(gpu, hip_lib, B, T, I, H):
    """XCD-local plain stores and agent-scope stores move the same words: the
    outputs and every gradient are equal bit for bit."""
    from rnn_kernel_amd import GRUFunction, _lib

    print(f"store paths B={B} T={T} I={I} H={H}", flush=True)
    p, x, h0, dy, dhn = _layer_inputs(B, T, I, H, seed=B * 7 + H)
    results = []
    try:
        for mode in (0, 1):
            _lib.set_exchange_stores(mode)
            xd = x.to(gpu).requires_grad_(True)
            h0d = h0.to(gpu).requires_grad_(True)
            pd = {k: v.to(gpu).requires_grad_(True) for k, v in p.items()}
            y, hn = GRUFunction.apply(xd, h0d, pd["weight_ih"], pd["weight_hh"], pd["bias_ih"], pd["bias_hh"])
            torch.autograd.backward([y, hn], [dy.to(gpu), dhn.to(gpu)[None]])
            torch.cuda.synchronize()
            results.append([y.detach(), hn.detach(), xd.grad, h0d.grad] + [pd[k].grad for k in sorted(pd)])
    finally:
        _lib.set_exchange_stores(0)
    for a, b in zip(*results):
        assert torch.equal(a, b)


def _check_layer_against_oracle(gpu, oracle, rec_kind, B, T, I, H):
    from rnn_kernel_amd import GRUFunction, _lib

    print(f"layer vs oracle B={B} T={T} I={I} H={H} kind={rec_kind} "
          f"fwd={_lib.describe_recurrence(0, B, H)} bwd={_lib.describe_recurrence(1, B, H)}", flush=True)
    p, x, h0, dy, dhn = _layer_inputs(B, T, I, H, seed=B * 1000 + T * 10 + H)
    f = oracle.forward(x.numpy(), h0.numpy(), p["weight_ih"].numpy(), p["weight_hh"].numpy(),
                       p["bias_ih"].numpy(), p["bias_hh"].numpy())
    ref = oracle.backward(x.numpy(), h0.numpy(), p["weight_ih"].numpy(), p["weight_hh"].numpy(), f.y, f.cache,
                          dy.numpy(), dhn.numpy())
    xd = x.to(gpu).requires_grad_(True)
    h0d = h0.to(gpu).requires_grad_(True)
    pd = {k: v.to(gpu).requires_grad_(True) for k, v in p.items()}
    y, hn = GRUFunction.apply(xd, h0d, pd["weight_ih"], pd["weight_hh"], pd["bias_ih"], pd["bias_hh"])
    torch.autograd.backward([y, hn], [dy.to(gpu), dhn.to(gpu)[None]])
    torch.cuda.synchronize()
    assert _maxabs(y, f.y) <= OUT_ATOL
    assert _maxabs(hn[0], f.hn) <= OUT_ATOL
    assert _rel(xd.grad, ref.dx) <= GRAD_REL
    assert _rel(h0d.grad, ref.dh0) <= GRAD_REL
    assert _rel(pd["weight_ih"].grad, ref.dw_ih) <= GRAD_REL
    assert _rel(pd["weight_hh"].grad, ref.dw_hh) <= GRAD_REL
    assert _rel(pd["bias_ih"].grad, ref.db_ih) <= GRAD_REL
    assert _rel(pd["bias_hh"].grad, ref.db_hh) <= GRAD_REL


def test_recurrence_reserve_layout_matches_oracle_cache(gpu, oracle, hip_lib):
    """The forward recurrence's reserve is (r, z, n, a_n) per [b, t, unit]."""
    from rnn_kernel_amd import _lib

    B, T, I, H = 4, 6, 8, 40
    p, x, h0, _, _ = _layer_inputs(B, T, I, H, seed=77)
    f = oracle.forward(x.numpy(), h0.numpy(), p["weight_ih"].numpy(), p["weight_hh"].numpy(),
                       p["bias_ih"].numpy(), p["bias_hh"].numpy())
    gx = (x.double() @ p["weight_ih"].double().T + p["bias_ih"].double()).float().contiguous().to(gpu)
    y = torch.empty(B, T, H, device=gpu)
    hn = torch.empty(B, H, device=gpu)
    res = torch.empty(B, T, 4 * H, device=gpu)
    ws_bytes = hip_lib.rka_gru_recurrence_workspace_bytes(B, H)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=gpu)
    whh, bhh, h0d = (t.contiguous().to(gpu) for t in (p["weight_hh"], p["bias_hh"], h0))
    rc = hip_lib.rka_gru_recurrence_forward(gx.data_ptr(), h0d.data_ptr(), whh.data_ptr(), bhh.data_ptr(),
                                            y.data_ptr(), hn.data_ptr(), res.data_ptr(), ws.data_ptr(), ws_bytes,
                                            B, T, H, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "rka_gru_recurrence_forward")
    torch.cuda.synchronize()
    assert _maxabs(res, _as_reserve(f.cache)) <= 1e-5
    assert _maxabs(y, f.y) <= 1e-5


def _nan_or_equal(out, ref, name):
    """Every entry of `out` is NaN or bitwise equal to `ref`; returns the NaN count."""
    out, ref = out.detach().cpu(), ref.detach().cpu()
    nan = torch.isnan(out)
    assert not torch.isinf(out).any(), name
    assert torch.equal(out[~nan], ref[~nan]), f"{name}: a finite entry differs from the complete run"
    return int(nan.sum())


@pytest.mark.parametrize("B,T,H", [(16, 32, 256), (64, 24, 256), (6, 16, 130), (300, 9, 256)])
def test_timed_out_waits_abort_with_nan_in_every_unwritten_output(gpu, oracle, hip_lib, rec_kind, B, T, H):
    """Failure handling, forced from the host: workgroup 0 of every launch
    publishes its words where its partners never look (rka_set_stall_block)
    and the poll bound is lowered to 256 rounds (rka_set_spin_limit), so the
    partners' waits give up and the launch aborts, every kernel exiting
    normally.  Every value an aborted launch leaves (y,
    the reserve and hn of the forward; the gate-gradient rows G and dh0 of
    the backward; dW, db and dx of a whole layer's backward) must be NaN or
    bitwise equal to a complete run's, the complete run must equal the
    oracle, and the per-device count of aborted calls
    (rka_recurrence_abort_count) must grow by one per call, which
    check_recurrences() turns into RecurrenceAbortedError."""
    _check_abort_path(gpu, oracle, hip_lib, rec_kind, B, T, H)


def _check_abort_path(gpu, oracle, hip_lib, rec_kind, B, T, H):
    import rnn_kernel_amd
    from rnn_kernel_amd import _lib

    I = 8
    p, x, h0, dy, dhn = _layer_inputs(B, T, I, H, seed=B + T)
    f = oracle.forward(x.numpy(), h0.numpy(), p["weight_ih"].numpy(), p["weight_hh"].numpy(),
                       p["bias_ih"].numpy(), p["bias_hh"].numpy())
    b = oracle.backward(x.numpy(), h0.numpy(), p["weight_ih"].numpy(), p["weight_hh"].numpy(), f.y, f.cache,
                        dy.numpy(), dhn.numpy())
    gx = (x.double() @ p["weight_ih"].double().T + p["bias_ih"].double()).float().contiguous().to(gpu)
    xd, wih, whh, bih, bhh, h0d, dyd, dhnd = (t.contiguous().to(gpu) for t in (
        x, p["weight_ih"], p["weight_hh"], p["bias_ih"], p["bias_hh"], h0, dy, dhn))
    ws_bytes = hip_lib.rka_gru_recurrence_workspace_bytes(B, H)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=gpu)
    stream = torch.cuda.current_stream().cuda_stream

    def forward():
        y = torch.empty(B, T, H, device=gpu)
        hn = torch.empty(B, H, device=gpu)
        res = torch.empty(B, T, 4 * H, device=gpu)
        rc = hip_lib.rka_gru_recurrence_forward(gx.data_ptr(), h0d.data_ptr(), whh.data_ptr(), bhh.data_ptr(),
                                                y.data_ptr(), hn.data_ptr(), res.data_ptr(), ws.data_ptr(),
                                                ws_bytes, B, T, H, stream)
        _lib.check(rc, "rka_gru_recurrence_forward")
        torch.cuda.synchronize()
        return y, hn, res

    def backward(y, res):
        g = torch.empty(B, T, 4 * H, device=gpu)
        dh0 = torch.empty(B, H, device=gpu)
        rc = hip_lib.rka_gru_recurrence_backward(dyd.data_ptr(), dhnd.data_ptr(), res.data_ptr(), h0d.data_ptr(),
                                                 y.data_ptr(), whh.data_ptr(), g.data_ptr(), dh0.data_ptr(),
                                                 ws.data_ptr(), ws_bytes, B, T, H, stream)
        _lib.check(rc, "rka_gru_recurrence_backward")
        torch.cuda.synchronize()
        return g, dh0

    def layer_backward(y, res):
        lws = hip_lib.rka_gru_backward_workspace_bytes(B, T, I, H)
        lw = torch.empty(lws, dtype=torch.uint8, device=gpu)
        out = {k: torch.empty(*shape, device=gpu) for k, shape in (
            ("dx", (B, T, I)), ("dh0", (B, H)), ("dw_ih", (3 * H, I)), ("dw_hh", (3 * H, H)),
            ("db_ih", (3 * H,)), ("db_hh", (3 * H,)))}
        rc = hip_lib.rka_gru_backward(xd.data_ptr(), h0d.data_ptr(), wih.data_ptr(), whh.data_ptr(), y.data_ptr(),
                                      res.data_ptr(), dyd.data_ptr(), dhnd.data_ptr(), out["dx"].data_ptr(),
                                      out["dh0"].data_ptr(), out["dw_ih"].data_ptr(), out["dw_hh"].data_ptr(),
                                      out["db_ih"].data_ptr(), out["db_hh"].data_ptr(), lw.data_ptr(), lws,
                                      B, T, I, H, stream)
        _lib.check(rc, "rka_gru_backward")
        torch.cuda.synchronize()
        return out

    print(f"abort path: kind={rec_kind} B={B} T={T} H={H} fwd {_lib.describe_recurrence(0, B, H)} "
          f"bwd {_lib.describe_recurrence(1, B, H)}", flush=True)
    rnn_kernel_amd.check_recurrences(gpu)  # earlier aborts are not this test's
    # complete runs, pinned to the oracle
    y_c, hn_c, res_c = forward()
    g_c, dh0_c = backward(y_c, res_c)
    layer_c = layer_backward(y_c, res_c)
    assert _maxabs(y_c, f.y) <= OUT_ATOL and _maxabs(hn_c, f.hn) <= OUT_ATOL
    assert _maxabs(res_c, _as_reserve(f.cache)) <= OUT_ATOL
    assert _rel(dh0_c, b.dh0) <= GRAD_REL and _rel(layer_c["dw_hh"], b.dw_hh) <= GRAD_REL
    assert _rel(layer_c["dx"], b.dx) <= GRAD_REL
    rnn_kernel_amd.check_recurrences(gpu)
    count0 = _lib.recurrence_abort_count()
    try:
        _lib.set_spin_limit(256)
        _lib.set_stall_block(0)
        y, hn, res = forward()
        g, dh0 = backward(y_c, res_c)
        layer = layer_backward(y_c, res_c)
    finally:
        _lib.set_stall_block(-1)
        _lib.set_spin_limit(0)
    nans = {
        "y": _nan_or_equal(y, y_c, "y"), "reserve": _nan_or_equal(res, res_c, "reserve"),
        "hn": _nan_or_equal(hn, hn_c, "hn"), "G": _nan_or_equal(g, g_c, "G"),
        "dh0": _nan_or_equal(dh0, dh0_c, "dh0"),
        **{f"layer {k}": _nan_or_equal(layer[k], layer_c[k], k) for k in layer},
    }
    print("  NaN entries after the forced aborts:", nans, flush=True)
    for k in ("y", "reserve", "hn", "G", "dh0", "layer dh0", "layer dx"):
        assert nans[k] > 0, f"{k}: the forced abort left no NaN"
    # an aborted row leaves NaN G rows in every column of its slices, so the
    # weight gradients, summed over all rows, cannot be finite
    for k in ("dw_hh", "dw_ih", "db_hh", "db_ih"):
        assert nans[f"layer {k}"] == layer[k].numel(), k
    count1 = _lib.recurrence_abort_count()
    assert count1 == count0 + 3, (count0, count1)  # one per aborted call, whatever its batch slices
    with pytest.raises(rnn_kernel_amd.RecurrenceAbortedError):
        rnn_kernel_amd.check_recurrences(gpu)
    # the next launches at the default limit zero the flag with the exchange
    # words and complete
    y2, hn2, res2 = forward()
    g2, dh02 = backward(y2, res2)
    for a, c in ((y2, y_c), (hn2, hn_c), (res2, res_c), (g2, g_c), (dh02, dh0_c)):
        assert torch.equal(a, c)
    rnn_kernel_amd.check_recurrences(gpu)
    assert _lib.recurrence_abort_count() == count1


def test_strict_mode_raises_on_an_aborted_layer(gpu, hip_lib):
    """set_strict(True): GRUFunction checks the abort count after its
    launches; an abort forced from the host (rka_set_stall_block) then
    raises RecurrenceAbortedError from the forward call itself."""
    import rnn_kernel_amd
    from rnn_kernel_amd import GRU, _lib

    torch.manual_seed(3)
    model = GRU(8, 256).to(gpu)
    x = torch.randn(16, 24, 8, device=gpu)
    rnn_kernel_amd.check_recurrences(gpu)
    rnn_kernel_amd.set_strict(True)
    try:
        y, hn = model(x)  # complete: no error
        _lib.set_spin_limit(256)
        _lib.set_stall_block(0)
        with pytest.raises(rnn_kernel_amd.RecurrenceAbortedError):
            model(x)
    finally:
        _lib.set_stall_block(-1)
        _lib.set_spin_limit(0)
        rnn_kernel_amd.set_strict(False)
    y2, hn2 = model(x)
    torch.cuda.synchronize()
    assert torch.equal(y, y2) and torch.equal(hn, hn2)
    rnn_kernel_amd.check_recurrences(gpu)


@pytest.mark.parametrize("B,H,launches", [(300, 256, 2), (400, 160, 2), (64, 256, 1)])
def test_batch_slices_of_resident_launches(gpu, hip_lib, B, H, launches):
    """A batch whose grid would not be resident runs as launches over batch
    slices, each resident (the largest count of groups that fits, a multiple
    of 8 so groups share an XCD); the described split covers the batch."""
    from rnn_kernel_amd import _lib

    for d in (0, 1):
        desc = _lib.describe_recurrence(d, B, H)
        print(f"dir {d} B={B} H={H}: {desc}", flush=True)
        assert desc["launches"] == launches
        per = desc["batch_per_launch"]
        assert (desc["launches"] - 1) * per < B <= desc["launches"] * per
        assert desc["groups"] == -(-per // desc["rows"])
        if launches > 1:
            assert desc["groups"] % 8 == 0


@pytest.mark.parametrize("B,H,padded", [(64, 256, True), (8, 256, True), (12, 256, True), (4, 256, True),
                                        (1, 256, True), (3, 130, True), (83, 130, False)])
def test_xcd_check_words_record_group_placement(gpu, hip_lib, B, H, padded):
    """Each recurrence workgroup records {XCC id, launch tag} in the workspace
    (after the two [B, 4H] exchange slots) and publishes with plain stores
    only when its exchange group shares one XCD.  Workgroups are dispatched
    to the 8 XCDs round-robin (consecutive block ids on consecutive XCDs,
    from a starting XCD that varies by launch).  The grid holds the G groups
    rounded up to a multiple of 8 (at these sizes the padded grid is
    resident): the S members of group g are blocks g % 8 + 8 ((g // 8) S + k),
    all on one XCD, and the padding workgroups (g >= G) exit without
    recording anything.  Small batches (G < 8) therefore exchange within one
    XCD too.  A grid resident only unpadded (83 groups of 3 workgroups on
    256 CUs, not 88) keeps consecutive blocks g S + k, spread over XCDs, and
    those groups publish with agent-scope stores.  Both store paths give the
    oracle's results in the layer tests."""
    from rnn_kernel_amd import _lib

    T = 3
    ws_bytes = hip_lib.rka_gru_recurrence_workspace_bytes(B, H)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=gpu)
    g = torch.Generator().manual_seed(B + H)
    gx = torch.randn(B, T, 3 * H, generator=g).to(gpu)
    whh = (0.05 * torch.randn(3 * H, H, generator=g)).to(gpu)
    bhh = torch.zeros(3 * H, device=gpu)
    h0 = torch.zeros(B, H, device=gpu)
    y = torch.empty(B, T, H, device=gpu)
    hn = torch.empty(B, H, device=gpu)
    rc = hip_lib.rka_gru_recurrence_forward(gx.data_ptr(), h0.data_ptr(), whh.data_ptr(), bhh.data_ptr(),
                                            y.data_ptr(), hn.data_ptr(), None, ws.data_ptr(), ws_bytes,
                                            B, T, H, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "rka_gru_recurrence_forward")
    torch.cuda.synchronize()
    assert torch.isfinite(hn).all()
    desc = _lib.describe_recurrence(0, B, H)
    groups, slices = desc["groups"], desc["slices"]
    grid_groups = -(-groups // 8) * 8 if padded else groups
    slots = (2 * B * 4 * H * 8 + 255) // 256 * 256
    words = ws[slots:slots + 8 * grid_groups * slices].cpu().view(torch.int64)
    tags = (words >> 32).tolist()
    xcc = (words & 0xFFFFFFFF).tolist()

    def members(gi):
        if grid_groups % 8 == 0:
            return [gi % 8 + 8 * ((gi // 8) * slices + k) for k in range(slices)]
        return [gi * slices + k for k in range(slices)]

    real = sorted(b for gi in range(groups) for b in members(gi))
    assert len(set(real)) == groups * slices and max(real) < grid_groups * slices
    assert all(tags[b] == 1 for b in real), tags
    assert all(tags[b] == 0 for b in set(range(grid_groups * slices)) - set(real)), tags
    assert all(0 <= xcc[b] < 16 for b in real)
    on_one = [len({xcc[b] for b in members(gi)}) == 1 for gi in range(groups)]
    print(f"B={B} H={H} groups={groups} grid groups={grid_groups} slices={slices} "
          f"xcc of the first blocks {xcc[:16]} groups on one XCD: {sum(on_one)}/{groups}", flush=True)
    if padded:
        assert all(on_one)
    else:
        assert not all(on_one)


# ----------------------------------- module vs torch.nn.GRU on the GPU ---
@pytest.mark.parametrize("input_size", [1, 16])
@pytest.mark.parametrize("num_layers", [1, 2, 3, 4])
def test_from_torch_gru_matches_torch_gru(gpu, num_layers, input_size):
    """Mirror of the reference's prod parity test (tests/test_a100_prod.py:84-126)
    with the same shapes and tolerances."""
    from rnn_kernel_amd import from_torch_gru

    _no_tf32()
    torch.manual_seed(2130 + num_layers * 10 + input_size)
    hidden, batch, seq = 256, 2, 5
    torch_gru = torch.nn.GRU(input_size, hidden, num_layers=num_layers, batch_first=True).to(gpu)
    ours = from_torch_gru(torch_gru)
    x_t = torch.randn(batch, seq, input_size, device=gpu, requires_grad=True)
    x_o = x_t.detach().clone().requires_grad_(True)
    h_t = torch.randn(num_layers, batch, hidden, device=gpu, requires_grad=True)
    h_o = h_t.detach().clone().requires_grad_(True)
    out_t, hn_t = torch_gru(x_t, h_t)
    out_o, hn_o = ours(x_o, h_o)
    g_out = torch.randn_like(out_t)
    g_h = torch.randn_like(hn_t)
    out_t.backward(g_out, retain_graph=True)
    hn_t.backward(g_h)
    out_o.backward(g_out, retain_graph=True)
    hn_o.backward(g_h)
    assert torch.allclose(out_t, out_o, atol=4e-4, rtol=1e-4)
    assert torch.allclose(hn_t, hn_o, atol=4e-4, rtol=1e-4)
    assert torch.allclose(x_t.grad, x_o.grad, atol=1e-3, rtol=3e-4)
    assert torch.allclose(h_t.grad, h_o.grad, atol=1e-3, rtol=3e-4)
    for name, p in torch_gru.named_parameters():
        assert torch.allclose(p.grad, getattr(ours, name).grad, atol=5e-3, rtol=1e-3), name


@pytest.mark.parametrize("num_layers", [1, 3])
def test_inference_paths_match_torch_gru(gpu, num_layers):
    """no_grad and forward_inference take the cache-free path
    (reference tests/test_a100_prod.py:129-162)."""
    from rnn_kernel_amd import from_torch_gru

    _no_tf32()
    torch.manual_seed(2133 + num_layers)
    torch_gru = torch.nn.GRU(16, 256, num_layers=num_layers, batch_first=True).to(gpu)
    ours = from_torch_gru(torch_gru)
    x = torch.randn(2, 5, 16, device=gpu)
    h0 = torch.randn(num_layers, 2, 256, device=gpu)
    with torch.no_grad():
        out_t, hn_t = torch_gru(x, h0)
        out_n, hn_n = ours(x, h0)
    out_e, hn_e = ours.forward_inference(x, h0)
    assert not out_n.requires_grad and not out_e.requires_grad
    for a, b in ((out_t, out_n), (hn_t, hn_n), (out_t, out_e), (hn_t, hn_e)):
        assert torch.allclose(a, b, atol=4e-4, rtol=1e-4)


def test_loss_on_final_hidden_only_and_output_only(gpu):
    """grad_output None (loss on h_n only) and grad_h_n None (loss on output only)."""
    from rnn_kernel_amd import from_torch_gru

    _no_tf32()
    torch.manual_seed(414)
    torch_gru = torch.nn.GRU(8, 64, batch_first=True).to(gpu)
    ours = from_torch_gru(torch_gru)
    x = torch.randn(3, 7, 8, device=gpu)
    for which in ("hn", "out"):
        torch_gru.zero_grad()
        ours.zero_grad()
        out_t, hn_t = torch_gru(x)
        out_o, hn_o = ours(x)
        (hn_t.square().sum() if which == "hn" else out_t.square().sum()).backward()
        (hn_o.square().sum() if which == "hn" else out_o.square().sum()).backward()
        for name, p in torch_gru.named_parameters():
            assert _rel(getattr(ours, name).grad, p.grad) <= GRAD_REL, (which, name)


def test_repeat_runs_are_bitwise_identical(gpu):
    from rnn_kernel_amd import GRU

    torch.manual_seed(99)
    model = GRU(32, 128).to(gpu)
    x = torch.randn(16, 40, 32, device=gpu)
    results = []
    for _ in range(2):
        model.zero_grad()
        xi = x.clone().requires_grad_(True)
        y, hn = model(xi)
        (y.sin().sum() + hn.sum()).backward()
        results.append([y.detach().clone(), hn.detach().clone(), xi.grad.clone()] +
                       [p.grad.clone() for p in model.parameters()])
    for a, b in zip(*results):
        assert torch.equal(a, b)


@pytest.mark.parametrize("B,H", [(64, 256), (12, 256), (64, 96)])
def test_recurrences_progress_beside_a_concurrent_kernel(gpu, B, H):
    """The recurrences are launched without a co-residency guarantee: each
    exchange group's workgroups are consecutive in the dispatch order of the
    XCDs, so the kernel progresses when only part of the grid fits at first.
    Here long GEMMs on a second stream hold the GPU when a layer's forward and
    backward are enqueued; the results must equal the solo run bit for bit
    (B=64: groups on one XCD; B=12: groups of consecutive blocks; H=96: two
    slices)."""
    from rnn_kernel_amd import GRU

    print(f"progress beside a concurrent GEMM B={B} H={H}", flush=True)
    torch.manual_seed(B + H)
    model = GRU(64, H).to(gpu)
    x = torch.randn(B, 96, 64, device=gpu)
    big = torch.randn(6144, 6144, device=gpu)
    side = torch.cuda.Stream(device=gpu)

    def run():
        model.zero_grad()
        xi = x.clone().requires_grad_(True)
        y, hn = model(xi)
        (y.sin().sum() + hn.sum()).backward()
        return [y.detach().clone(), hn.detach().clone(), xi.grad.clone()] + [p.grad.clone() for p in model.parameters()]

    solo = run()
    torch.cuda.synchronize()
    for _ in range(2):
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                big = torch.mm(big, big) * 1e-4
        busy = run()
        torch.cuda.synchronize()
        for a, b in zip(solo, busy):
            assert torch.isfinite(b).all()
            assert torch.equal(a, b)


@pytest.mark.parametrize("H,fwd_rows,bwd_rows", [(200, 2, 4), (256, 2, 2), (160, 4, 4), (64, 4, 2), (48, 4, 4),
                                                  (100, 2, 4)])
def test_rows_per_workgroup_agree(gpu, hip_lib, H, fwd_rows, bwd_rows):
    """The local-slice recurrences with 2 or 4 batch rows per workgroup
    (batch 9: the last group partly empty; the four-row backward in two
    phases of two rows, at one to four slices) give the one-row results."""
    from rnn_kernel_amd import GRU, _lib

    torch.manual_seed(H)
    model = GRU(16, H).to(gpu)
    x = torch.randn(9, 7, 16, device=gpu)
    h0 = 0.3 * torch.randn(1, 9, H, device=gpu)

    def run():
        model.zero_grad()
        xi = x.clone().requires_grad_(True)
        hi = h0.clone().requires_grad_(True)
        y, hn = model(xi, hi)
        (y.sin().sum() + hn.sum()).backward()
        return [y.detach().clone(), hn.detach().clone(), xi.grad.clone(), hi.grad.clone()] + \
            [p.grad.clone() for p in model.parameters()]

    for d in (0, 1):
        _lib.set_recurrence_config(d, 2, 0, 1)
    try:
        base = run()
        _lib.set_recurrence_config(0, 2, 0, fwd_rows)
        _lib.set_recurrence_config(1, 2, 0, bwd_rows)
        print("rows", _lib.describe_recurrence(0, 9, H), _lib.describe_recurrence(1, 9, H), flush=True)
        alt = run()
    finally:
        for d in (0, 1):
            _lib.set_recurrence_config(d, 0, 0, 0)
    for a, b in zip(base, alt):
        assert _rel(a, b) <= 1e-5


@pytest.mark.parametrize("kind,units,param", [(1, 1, 0), (1, 4, 0), (1, 16, 2), (1, 64, 0), (2, 0, 2), (2, 0, 4)])
def test_alternative_decompositions_agree(gpu, hip_lib, kind, units, param):
    """Other tilings / kernel families of the recurrences give the same answer."""
    from rnn_kernel_amd import GRU, _lib

    torch.manual_seed(5)
    model = GRU(24, 72).to(gpu)
    x = torch.randn(10, 9, 24, device=gpu)

    def run():
        model.zero_grad()
        xi = x.clone().requires_grad_(True)
        y, hn = model(xi)
        (y.cos().sum() + hn.sum()).backward()
        return [y.detach().clone(), xi.grad.clone()] + [p.grad.clone() for p in model.parameters()]

    base = run()
    for d in (0, 1):
        _lib.set_recurrence_config(d, kind, units, param)
    try:
        print("alt", _lib.describe_recurrence(0, 10, 72), _lib.describe_recurrence(1, 10, 72), flush=True)
        alt = run()
    finally:
        for d in (0, 1):
            _lib.set_recurrence_config(d, 0, 0, 0)
    for a, b in zip(base, alt):
        assert _rel(a, b) <= 1e-5


# ------------------------------------------------- BASELINE configurations ---
def _torch_reference(gpu, L, I, H, B, T, seed, h0_scale, x_hook=None, chunks=1):
    """Our model and torch.nn.GRU with identical weights/inputs; MSE loss vs
    N(0,1) target.  Returns (ours, theirs) dicts of results."""
    from rnn_kernel_amd import from_torch_gru

    _no_tf32()
    torch.manual_seed(seed)
    torch_gru = torch.nn.GRU(I, H, num_layers=L, batch_first=True)
    x = torch.randn(B, T, I)
    if x_hook is not None:
        x = x_hook(x)
    h0 = h0_scale * torch.randn(L, B, H)
    target = torch.randn(B, T, H)
    torch_gru = torch_gru.to(gpu)
    ours = from_torch_gru(torch_gru)
    res = {}
    for name, model in (("ours", ours), ("torch", torch_gru)):
        xi = x.to(gpu).requires_grad_(True)
        hi = h0.to(gpu).requires_grad_(True)
        if chunks == 1:
            out, hn = model(xi, hi)
        else:
            outs, hidden = [], hi
            for c in xi.chunk(chunks, dim=1):
                o, hidden = model(c, hidden)
                outs.append(o)
            out, hn = torch.cat(outs, dim=1), hidden
        loss = torch.nn.functional.mse_loss(out, target.to(gpu))
        loss.backward()
        res[name] = {"out": out.detach(), "hn": hn.detach(), "dx": xi.grad, "dh0": hi.grad,
                     **{n: p.grad for n, p in model.named_parameters()}}
    return res, (torch_gru, x, h0, target)


def _assert_parity(res, label):
    o, t = res["ours"], res["torch"]
    assert _maxabs(o["out"], t["out"]) <= OUT_ATOL, label
    assert _maxabs(o["hn"], t["hn"]) <= OUT_ATOL, label
    for k in o:
        if k in ("out", "hn"):
            continue
        assert _rel(o[k], t[k]) <= GRAD_REL, (label, k, _rel(o[k], t[k]))


def test_config2_north_star_matches_torch_gru_and_the_oracle(gpu, oracle):
    """I=256, H=256, B=64, T=512, h0 ~ 0.1 N(0,1), MSE loss: every output and
    gradient against torch.nn.GRU fp32 on the GPU (MIOpen) and against the
    float64 oracle at full size (run on the host CPU, batch rows split over
    up to 16 threads)."""
    import os

    print("config2 B=64 T=512 I=256 H=256", flush=True)
    res, (torch_gru, x, h0, target) = _torch_reference(gpu, 1, 256, 256, 64, 512, seed=42, h0_scale=0.1)
    _assert_parity(res, "c2")
    p = {n: getattr(torch_gru, f"{n}_l0").detach().cpu().double().numpy()
         for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")}
    threads = min(16, os.cpu_count() or 1)
    xd, h0d = x.double().numpy(), h0[0].double().numpy()
    f = oracle.forward_rows_parallel(xd, h0d, p["weight_ih"], p["weight_hh"], p["bias_ih"], p["bias_hh"],
                                     threads=threads)
    # d(mean squared error)/d(out) of the oracle's own output
    dy = (2.0 / target.numel()) * (f.y - target.double().numpy())
    b = oracle.backward_rows_parallel(xd, h0d, p["weight_ih"], p["weight_hh"], f.y, f.cache, dy, None,
                                      threads=threads)
    ours = res["ours"]
    errs = {"out": _maxabs(ours["out"], f.y), "hn": _maxabs(ours["hn"][0], f.hn),
            "dx": _rel(ours["dx"], b.dx), "dh0": _rel(ours["dh0"][0], b.dh0),
            "weight_ih_l0": _rel(ours["weight_ih_l0"], b.dw_ih), "weight_hh_l0": _rel(ours["weight_hh_l0"], b.dw_hh),
            "bias_ih_l0": _rel(ours["bias_ih_l0"], b.db_ih), "bias_hh_l0": _rel(ours["bias_hh_l0"], b.db_hh)}
    print("  c2 vs the float64 oracle:", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    assert errs["out"] <= OUT_ATOL and errs["hn"] <= OUT_ATOL
    for k, v in errs.items():
        if k not in ("out", "hn"):
            assert v <= GRAD_REL, (k, v)


@pytest.mark.parametrize("H", [64, 96, 128, 129, 130, 160, 192, 224])
def test_config3_hidden_sweep_matches_torch_gru(gpu, H):
    print(f"config3 H={H}", flush=True)
    res, _ = _torch_reference(gpu, 1, H, H, 64, 512, seed=42 + H, h0_scale=0.1)
    _assert_parity(res, f"c3 H={H}")


def _oracle_errors(ours, ref, L):
    """Max-abs errors of out / h_n and relative errors of every gradient of a
    full-size run against the float64 oracle (stack_rows_parallel result)."""
    errs = {"out": _maxabs(ours["out"], ref.y), "hn": _maxabs(ours["hn"], ref.hn), "dx": _rel(ours["dx"], ref.dx),
            "dh0": _rel(ours["dh0"], ref.dhx)}
    for l in range(L):
        for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh"):
            errs[f"{n}_l{l}"] = _rel(ours[f"{n}_l{l}"], ref.grads[l][n])
    return errs


def _assert_oracle_errors(errs, label):
    print(f"  {label} vs the float64 oracle:", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    assert errs["out"] <= OUT_ATOL and errs["hn"] <= OUT_ATOL, label
    for k, v in errs.items():
        if k not in ("out", "hn"):
            assert v <= GRAD_REL, (label, k, v)


def _oracle_params(torch_gru, L):
    return [{n: getattr(torch_gru, f"{n}_l{l}").detach().cpu().double().numpy()
             for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")} for l in range(L)]


def test_config4_stacked_two_layers_matches_torch_gru_and_the_oracle(gpu, oracle):
    """L=2, I=H=256, B=256, T=1024, MSE loss: every output and gradient of both
    layers against torch.nn.GRU fp32 on the GPU and against the float64
    oracle's two-layer stack at full size (layer composition of
    src/rnn_kernel/a100/prod/gru.py:699-728; batch rows split over up to 16
    host threads, each chunk's output gradient the MSE gradient of its own
    forward result)."""
    import os

    print("config4 L=2 B=256 T=1024 H=256", flush=True)
    res, (torch_gru, x, h0, target) = _torch_reference(gpu, 2, 256, 256, 256, 1024, seed=44, h0_scale=0.0)
    _assert_parity(res, "c4")
    tgt = target.double().numpy()
    scale = 2.0 / tgt.size
    ref = oracle.stack_rows_parallel(x.double().numpy(), h0.double().numpy(), _oracle_params(torch_gru, 2),
                                     lambda y, a, b: scale * (y - tgt[a:b]), threads=min(16, os.cpu_count() or 1))
    _assert_oracle_errors(_oracle_errors(res["ours"], ref, 2), "c4")


def _config5_inputs():
    def saturate(x):
        g = torch.Generator().manual_seed(4242)
        mask = torch.rand(x.shape[0], x.shape[1], generator=g) < 0.05
        return torch.where(mask[..., None], x * 10.0, x)

    return dict(L=1, I=128, H=256, B=16, T=4096, seed=45, h0_scale=0.5, x_hook=saturate)


def test_config5_chunked_bptt_matches_torch_gru_chunked(gpu):
    """I=128, H=256, B=16, T=4096 as 8 chunks of 512 carrying h (no detach),
    h0 ~ 0.5 N(0,1), 5% of [B,T] rows of x scaled x10: the same chunked run
    through torch.nn.GRU fp32 on the GPU."""
    print("config5 chunked vs torch chunked", flush=True)
    c = _config5_inputs()
    res, _ = _torch_reference(gpu, c["L"], c["I"], c["H"], c["B"], c["T"], seed=c["seed"], h0_scale=c["h0_scale"],
                              x_hook=c["x_hook"], chunks=8)
    _assert_parity(res, "c5")


def test_config5_chunked_bptt_equals_the_full_sequence_oracle(gpu, oracle):
    """Chunked BPTT equals full BPTT (tests/test_sequence_chunking.py:17-35 of
    the reference): the 8 x 512 chunked run carrying h without detach (its
    h_n handed to the next chunk's h0, the next chunk's dh0 back as this
    chunk's d h_n) against the float64 oracle over the whole T = 4096
    sequence in one piece, for out, h_n, dx, dh0 and every weight gradient."""
    import os

    print("config5 chunked vs the full-sequence oracle", flush=True)
    c = _config5_inputs()
    res, (torch_gru, x, h0, target) = _torch_reference(gpu, c["L"], c["I"], c["H"], c["B"], c["T"], seed=c["seed"],
                                                       h0_scale=c["h0_scale"], x_hook=c["x_hook"], chunks=8)
    tgt = target.double().numpy()
    scale = 2.0 / tgt.size
    ref = oracle.stack_rows_parallel(x.double().numpy(), h0.double().numpy(), _oracle_params(torch_gru, 1),
                                     lambda y, a, b: scale * (y - tgt[a:b]), threads=min(16, os.cpu_count() or 1))
    _assert_oracle_errors(_oracle_errors(res["ours"], ref, 1), "c5")


def test_exchange_latency_probe(gpu, hip_lib):
    """The committed exchange measurement bench.py reports: one pair and
    every CU busy (128 pairs); both sides of each pair on one XCD, round
    trips finite and within the range such an exchange takes (0.1 - 10 us)."""
    from rnn_kernel_amd import _lib

    for pairs in (1, 128):
        r = _lib.measure_exchange_latency(pairs=pairs, iters=500)
        print("exchange probe", r, flush=True)
        assert r["same_xcd"]
        assert 100.0 < r["round_trip_ns"] < 10000.0


def test_fma_rate_probe(gpu, hip_lib):
    """The committed FMA issue-rate measurement bench.py prices the
    recurrences' FMAs against: a finite rate no faster than two clocks per
    wave64 instruction at 2.4 GHz (the published 157.3 TFLOP/s) and no
    slower than eight."""
    from rnn_kernel_amd import _lib

    r = _lib.measure_fma_rate()
    print("fma probe", r, flush=True)
    assert 2 / 2.4 * 0.95 < r["ns_per_instruction"] < 8 / 2.4
    assert 20.0 < r["tflops"] < 157.3 * 1.05
