"""CPU checks of the harness-side operations' oracle (head, MSE, AdamW) and of
the harness's host logic.  The reference runs these steps as PyTorch ops
(rnn_benchmark.py:510,525,636,722, torch==2.6.0), so the float64 oracle is
pinned against PyTorch's own implementations on the CPU, plus closed forms
and a planted mistake."""
import numpy as np
import pytest
import torch

from oracle import gru_oracle as orc


def _rng(seed):
    return np.random.default_rng(seed)


@pytest.mark.parametrize("shape,hidden", [((2, 3), 7), ((5,), 1), ((4, 6), 130)])
def test_head_oracle_matches_torch_linear(shape, hidden):
    r = _rng(hidden)
    out = r.standard_normal(shape + (hidden,))
    w = r.standard_normal((1, hidden))
    b = r.standard_normal(1)
    lin = torch.nn.Linear(hidden, 1).double()
    with torch.no_grad():
        lin.weight.copy_(torch.from_numpy(w))
        lin.bias.copy_(torch.from_numpy(b))
    o = torch.from_numpy(out).requires_grad_(True)
    pred = lin(o).squeeze(-1)
    dpred = r.standard_normal(shape)
    pred.backward(torch.from_numpy(dpred))
    np.testing.assert_allclose(orc.head_forward(out, w, b), pred.detach().numpy(), rtol=1e-13, atol=1e-13)
    dout, dw, db = orc.head_backward(out, w, dpred)
    np.testing.assert_allclose(dout, o.grad.numpy(), rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(dw, lin.weight.grad.numpy()[0], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(db, lin.bias.grad.numpy()[0], rtol=1e-12, atol=1e-12)


def test_mse_oracle_matches_torch_and_closed_form():
    r = _rng(3)
    pred = r.standard_normal((4, 9))
    target = r.standard_normal((4, 9))
    p = torch.from_numpy(pred).requires_grad_(True)
    loss = torch.nn.functional.mse_loss(p, torch.from_numpy(target))
    loss.backward(torch.tensor(0.5, dtype=torch.float64))
    assert orc.mse_forward(pred, target) == pytest.approx(loss.item(), rel=1e-14)
    np.testing.assert_allclose(orc.mse_backward(pred, target, 0.5), p.grad.numpy(), rtol=1e-13, atol=1e-15)
    # closed form: a constant offset c gives loss c^2 and gradient 2c/n
    assert orc.mse_forward(target + 0.25, target) == pytest.approx(0.0625, rel=1e-14)
    np.testing.assert_allclose(orc.mse_backward(target + 0.25, target), np.full(target.shape, 0.5 / target.size))


def _torch_adamw(p0, grads, lr, betas, eps, wd):
    p = torch.nn.Parameter(torch.from_numpy(p0.copy()))
    opt = torch.optim.AdamW([p], lr=lr, betas=betas, eps=eps, weight_decay=wd, foreach=False)
    for g in grads:
        p.grad = torch.from_numpy(g)
        opt.step()
    st = opt.state[p]
    return p.detach().numpy(), st["exp_avg"].numpy(), st["exp_avg_sq"].numpy()


def test_adamw_oracle_matches_torch_over_several_steps():
    r = _rng(7)
    p0 = r.standard_normal(50)
    grads = [r.standard_normal(50) for _ in range(4)]
    lr, betas, eps, wd = 3e-4, (0.9, 0.999), 1e-8, 1e-4
    p, m, v = p0, np.zeros(50), np.zeros(50)
    for step, g in enumerate(grads, 1):
        p, m, v = orc.adamw_step(p, g, m, v, lr, betas[0], betas[1], eps, wd, step)
    tp, tm, tv = _torch_adamw(p0, grads, lr, betas, eps, wd)
    np.testing.assert_allclose(p, tp, rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(m, tm, rtol=1e-13, atol=1e-16)
    np.testing.assert_allclose(v, tv, rtol=1e-13, atol=1e-18)


def test_adamw_oracle_first_step_closed_form_and_planted_mistake():
    # step 1, no decay: m^ = g, v^ = g^2, so p1 = p0 - lr g / (|g| + eps)
    g = np.array([0.5, -2.0, 1e-3])
    p0 = np.array([1.0, 2.0, 3.0])
    p1, _, _ = orc.adamw_step(p0, g, np.zeros(3), np.zeros(3), 0.1, 0.9, 0.999, 1e-8, 0.0, 1)
    np.testing.assert_allclose(p1, p0 - 0.1 * g / (np.abs(g) + 1e-8), rtol=1e-12)
    # dropping the bias correction (a plausible mistake) must break the match
    r = _rng(9)
    pp, gg = r.standard_normal(20), [r.standard_normal(20) for _ in range(2)]
    tp, _, _ = _torch_adamw(pp, gg, 1e-2, (0.9, 0.999), 1e-8, 0.0)
    p, m, v = pp.copy(), np.zeros(20), np.zeros(20)
    for g_ in gg:  # Adam without bias correction
        m = 0.9 * m + 0.1 * g_
        v = 0.999 * v + 0.001 * g_ * g_
        p = p - 1e-2 * m / (np.sqrt(v) + 1e-8)
    assert np.abs(p - tp).max() > 1e-4


def test_harness_csv_schema_and_defaults_follow_the_reference(tmp_path):
    """The results CSV columns and the CLI defaults of rnn_benchmark.py
    (:874-899 and :912-998)."""
    from rnn_kernel_amd import harness

    expected = ["cell_type", "implementation", "hidden_size", "sequence_chunk_len", "a100_block_threads",
                "deterministic", "cudnn_enabled", "cudnn_benchmark", "cuda_matmul_allow_tf32", "cudnn_allow_tf32",
                "compile_model", "params", "ms_per_step", "zero_grad_ms_per_step", "forward_ms_per_step",
                "loss_ms_per_step", "backward_ms_per_step", "optimizer_ms_per_step", "measured_ms_per_step",
                "steps_per_second", "tokens_per_second", "peak_memory_gb", "last_loss", "status"]
    assert harness.CSV_FIELDS == expected
    a = harness.parse_args([])
    assert (a.batch_size, a.seq_len, a.input_dim, a.num_layers, a.lr, a.warmup_steps, a.timed_steps,
            a.dataset_batches, a.seed, a.hidden_sizes) == (16, 8000, 16, 4, 3e-4, 3, 10, 32, 42, [256])
    r = harness.BenchmarkResult(
        cell_type="GRU", implementation="x", hidden_size=8, sequence_chunk_len=0, a100_block_threads=0,
        deterministic=False, cudnn_enabled=True, cudnn_benchmark=False, cuda_matmul_allow_tf32=False,
        cudnn_allow_tf32=False, compile_model=False, params=1, ms_per_step=1.0, zero_grad_ms_per_step=None,
        forward_ms_per_step=None, loss_ms_per_step=None, backward_ms_per_step=None, optimizer_ms_per_step=None,
        measured_ms_per_step=None, steps_per_second=1.0, tokens_per_second=2.0, peak_memory_gb=0.5,
        last_loss=0.25, status="ok")
    path = tmp_path / "r.csv"
    harness.write_csv(str(path), [r])
    lines = path.read_text().splitlines()
    assert lines[0] == ",".join(expected)
    assert lines[1].startswith("GRU,x,8,0,0,False")
    assert "ms/step=" in harness.format_result(r)
