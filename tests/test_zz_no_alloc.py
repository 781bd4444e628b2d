"""The allocation-free forward recurrence (rka_gru_recurrence_forward_noalloc)
against the workspace entry point it mirrors (rka_gru_recurrence_forward):
bitwise-equal y, hn and reserve on two calls in a row, the second smaller,
each run through the C ABI on the same inputs."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(B, T, H, seed, gpu):
    g = torch.Generator().manual_seed(seed)
    k = H ** -0.5
    gx = torch.randn(B, T, 3 * H, generator=g).to(gpu)
    whh = ((torch.rand(3 * H, H, generator=g) * 2 - 1) * k).to(gpu)
    bhh = ((torch.rand(3 * H, generator=g) * 2 - 1) * k).to(gpu)
    h0 = (0.5 * torch.randn(B, H, generator=g)).to(gpu)
    return gx, whh, bhh, h0


def _outputs(B, T, H, gpu, with_reserve):
    y = torch.full((B, T, H), float("nan"), device=gpu)
    hn = torch.full((B, H), float("nan"), device=gpu)
    res = torch.full((B, T, 4 * H), float("nan"), device=gpu) if with_reserve else None
    return y, hn, res


def _ptr(t):
    return None if t is None else t.data_ptr()


# calls in a row on the shared static state, each later one smaller:
#   c2-like one-row launch, then a small odd shape;
#   at the static limit (B H = 262144): B = 1024 at H = 256 runs the register
#   kernel as several batch-slice launches (the last slice's words end at the
#   array's end), H = 512 the LDS-tiled kernel; then the small odd shape
SEQUENCES = [
    ((64, 40, 256, 1), (5, 7, 130, 2)),
    ((1024, 6, 256, 3), (512, 5, 512, 4), (5, 7, 130, 5)),
]


@pytest.mark.parametrize("with_reserve", [True, False])
@pytest.mark.parametrize("sequence", SEQUENCES)
def test_noalloc_forward_matches_workspace_forward(gpu, hip_lib, with_reserve, sequence):
    from rnn_kernel_amd import _lib

    stream = torch.cuda.current_stream().cuda_stream
    for B, T, H, seed in sequence:
        print(f"noalloc forward B={B} T={T} H={H} reserve={with_reserve} fwd={_lib.describe_recurrence(0, B, H)}",
              flush=True)
        gx, whh, bhh, h0 = _inputs(B, T, H, seed, gpu)
        y_ref, hn_ref, res_ref = _outputs(B, T, H, gpu, with_reserve)
        ws_bytes = hip_lib.rka_gru_recurrence_workspace_bytes(B, H)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=gpu)
        rc = hip_lib.rka_gru_recurrence_forward(gx.data_ptr(), h0.data_ptr(), whh.data_ptr(), bhh.data_ptr(),
                                                y_ref.data_ptr(), hn_ref.data_ptr(), _ptr(res_ref), ws.data_ptr(),
                                                ws_bytes, B, T, H, stream)
        _lib.check(rc, "rka_gru_recurrence_forward")
        y, hn, res = _outputs(B, T, H, gpu, with_reserve)
        rc = hip_lib.rka_gru_recurrence_forward_noalloc(gx.data_ptr(), h0.data_ptr(), whh.data_ptr(),
                                                        bhh.data_ptr(), y.data_ptr(), hn.data_ptr(), _ptr(res),
                                                        B, T, H, stream)
        _lib.check(rc, "rka_gru_recurrence_forward_noalloc")
        torch.cuda.synchronize()
        assert torch.isfinite(y_ref).all() and torch.isfinite(hn_ref).all()
        assert torch.equal(y, y_ref)
        assert torch.equal(hn, hn_ref)
        if with_reserve:
            assert torch.equal(res, res_ref)


def test_noalloc_forward_rejects_shapes_beyond_its_static_scratch(gpu, hip_lib):
    """batch * hidden_size above 262144 is refused before anything launches."""
    from rnn_kernel_amd import _lib

    B, T, H = 2048, 2, 256
    dummy = torch.zeros(16, device=gpu)
    p = dummy.data_ptr()
    rc = hip_lib.rka_gru_recurrence_forward_noalloc(p, p, p, p, p, p, None, B, T, H,
                                                    torch.cuda.current_stream().cuda_stream)
    assert rc == 1004  # RKA_ERR_UNSUPPORTED_SHAPE
    assert "static scratch limit" in _lib.last_error()
    # step tags carry a call number in their top 8 bits: seq_len < 2^24
    rc = hip_lib.rka_gru_recurrence_forward_noalloc(p, p, p, p, p, p, None, 1, 1 << 24, 16,
                                                    torch.cuda.current_stream().cuda_stream)
    assert rc == 1004
    assert "2^24" in _lib.last_error()
    torch.cuda.synchronize()
