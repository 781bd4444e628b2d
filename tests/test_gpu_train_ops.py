"""GPU parity of the harness-side operations (head, MSE, AdamW) with the
float64 oracle, and of a whole benchmark-model training step with the
reference's PyTorch formulation (nn.GRU + nn.Linear + F.mse_loss +
torch.optim.AdamW, rnn_benchmark.py:510,525,628-639,722).

Tolerances: elementwise outputs within 1e-5 relative to the float64 oracle
(fp32 arithmetic), reductions within 1e-5 relative; the AdamW parameters
after several steps within 1e-6 absolute (step sizes are ~lr = 1e-2).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.mark.parametrize("shape,hidden", [((2, 8), 16), ((64, 512), 256), ((3, 5), 130), ((7,), 1)])
def test_head_forward_backward_matches_oracle(gpu, oracle, shape, hidden):
    from rnn_kernel_amd import HeadFunction

    print(f"head shape={shape} hidden={hidden}", flush=True)
    g = torch.Generator().manual_seed(hidden + len(shape))
    out = torch.randn(*shape, hidden, generator=g)
    w = torch.randn(1, hidden, generator=g) / hidden ** 0.5
    b = torch.randn(1, generator=g)
    dpred = torch.randn(*shape, generator=g)
    od = out.to(gpu).requires_grad_(True)
    wd = w.to(gpu).requires_grad_(True)
    bd = b.to(gpu).requires_grad_(True)
    pred = HeadFunction.apply(od, wd, bd)
    pred.backward(dpred.to(gpu))
    torch.cuda.synchronize()
    ref = oracle.head_forward(out.numpy(), w.numpy(), b.numpy())
    dout, dw, db = oracle.head_backward(out.numpy(), w.numpy(), dpred.numpy())
    assert pred.shape == torch.Size(shape)
    assert _rel(pred.detach().cpu(), ref) <= 1e-5
    assert _rel(od.grad.cpu(), dout) <= 1e-6
    assert _rel(wd.grad.cpu()[0], dw) <= 1e-5
    assert abs(bd.grad.item() - db) <= 1e-5 * max(abs(db), 1.0)


@pytest.mark.parametrize("n", [1, 1000, 4097, 64 * 512 * 256])
def test_mse_forward_backward_matches_oracle(gpu, oracle, n):
    from rnn_kernel_amd import mse_loss

    print(f"mse n={n}", flush=True)
    g = torch.Generator().manual_seed(n % 1000)
    pred = torch.randn(n, generator=g)
    target = torch.randn(n, generator=g)
    pd = pred.to(gpu).requires_grad_(True)
    loss = mse_loss(pd, target.to(gpu))
    loss.backward(torch.tensor(0.75, device=gpu))
    torch.cuda.synchronize()
    assert abs(loss.item() - oracle.mse_forward(pred.numpy(), target.numpy())) <= 1e-5 * max(loss.item(), 1e-3)
    assert _rel(pd.grad.cpu(), oracle.mse_backward(pred.numpy(), target.numpy(), 0.75)) <= 1e-6


def test_mse_and_head_are_bitwise_reproducible(gpu):
    from rnn_kernel_amd import HeadFunction, mse_loss

    g = torch.Generator().manual_seed(11)
    out = torch.randn(16, 300, 64, generator=g).to(gpu)
    w = torch.randn(1, 64, generator=g).to(gpu)
    b = torch.randn(1, generator=g).to(gpu)
    y = torch.randn(16, 300, generator=g).to(gpu)
    results = []
    for _ in range(3):
        o = out.clone().requires_grad_(True)
        ww = w.clone().requires_grad_(True)
        loss = mse_loss(HeadFunction.apply(o, ww, b), y)
        loss.backward()
        results.append((loss.detach().clone(), o.grad.clone(), ww.grad.clone()))
    for r in results[1:]:
        for a, b_ in zip(results[0], r):
            assert torch.equal(a, b_)


def test_adamw_matches_oracle_over_steps_and_many_tensors(gpu, oracle):
    """20 tensors (more than one launch's 16) of assorted sizes, 3 steps."""
    from rnn_kernel_amd import AdamW

    g = torch.Generator().manual_seed(5)
    sizes = [1, 3, 257, 1000, 4096] * 4
    init = [torch.randn(s, generator=g) for s in sizes]
    grads = [[torch.randn(s, generator=g) for s in sizes] for _ in range(3)]
    params = [torch.nn.Parameter(t.clone().to(gpu)) for t in init]
    opt = AdamW(params, lr=1e-2, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-4)
    for step in range(3):
        for p, gr in zip(params, grads[step]):
            p.grad = gr.to(gpu)
        opt.step()
    torch.cuda.synchronize()
    for i, t in enumerate(init):
        p, m, v = t.numpy(), np.zeros(sizes[i]), np.zeros(sizes[i])
        for step in range(3):
            p, m, v = oracle.adamw_step(p, grads[step][i].numpy(), m, v, 1e-2, 0.9, 0.999, 1e-8, 1e-4, step + 1)
        assert np.abs(params[i].detach().cpu().numpy() - p).max() <= 1e-6, i
        assert _rel(opt.state[params[i]]["exp_avg"].cpu(), m) <= 1e-6
        assert _rel(opt.state[params[i]]["exp_avg_sq"].cpu(), v) <= 1e-5


def test_benchmark_model_training_step_matches_torch(gpu):
    """One zero_grad/forward/MSE/backward/AdamW step of the harness model
    (GRU + HIP head/loss/optimiser) against nn.GRU + nn.Linear + F.mse_loss +
    torch.optim.AdamW from the same initial parameters, TF32 off."""
    from rnn_kernel_amd import harness

    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    torch.manual_seed(3)
    B, T, I, H, L = 4, 12, 8, 32, 2
    ours = harness.BenchmarkModel(I, H, L).to(gpu)
    ref_rnn = torch.nn.GRU(I, H, num_layers=L, batch_first=True).to(gpu)
    ref_head = torch.nn.Linear(H, 1).to(gpu)
    with torch.no_grad():
        for name, p in ref_rnn.named_parameters():
            p.copy_(getattr(ours.rnn, name))
        ref_head.weight.copy_(ours.head.weight)
        ref_head.bias.copy_(ours.head.bias)
    x = torch.randn(B, T, I, device=gpu)
    y = torch.randn(B, T, device=gpu)
    opt = harness.AdamW(ours.parameters(), lr=1e-2, weight_decay=1e-4)
    ref_params = list(ref_rnn.parameters()) + list(ref_head.parameters())
    ref_opt = torch.optim.AdamW(ref_params, lr=1e-2, weight_decay=1e-4)
    for _ in range(2):
        loss = harness.train_step(ours, opt, x, y, harness.mse_loss)
        ref_opt.zero_grad(set_to_none=True)
        out, _ = ref_rnn(x)
        ref_loss = torch.nn.functional.mse_loss(ref_head(out).squeeze(-1), y)
        ref_loss.backward()
        ref_opt.step()
        torch.cuda.synchronize()
        assert abs(loss.item() - ref_loss.item()) <= 1e-5 * max(ref_loss.item(), 1.0)
    for (name, p), q in zip(list(ours.rnn.named_parameters()) + list(ours.head.named_parameters()), ref_params):
        assert (p.detach() - q.detach()).abs().max().item() <= 2e-5, name


@pytest.mark.parametrize("torch_ops", [False, True])
def test_harness_run_case_end_to_end(gpu, tmp_path, torch_ops):
    from rnn_kernel_amd import harness

    args = harness.parse_args(["--hidden-sizes", "32", "--batch-size", "4", "--seq-len", "24", "--input-dim", "8",
                               "--num-layers", "2", "--sequence-chunk-len", "10", "--dataset-batches", "2",
                               "--warmup-steps", "1", "--timed-steps", "3", "--breakdown-timing"]
                              + (["--torch-ops"] if torch_ops else []))
    torch.manual_seed(args.seed)
    batches = harness.make_random_batches(args.dataset_batches, args.batch_size, args.seq_len, args.input_dim, gpu)
    r = harness.run_case(32, batches, args, gpu)
    print(harness.format_result(r), flush=True)
    assert r.status == "ok" and np.isfinite(r.last_loss) and r.ms_per_step > 0
    assert r.measured_ms_per_step == pytest.approx(r.zero_grad_ms_per_step + r.forward_ms_per_step
                                                   + r.loss_ms_per_step + r.backward_ms_per_step
                                                   + r.optimizer_ms_per_step)
    harness.write_csv(str(tmp_path / "r.csv"), [r])
