"""Pins the CPU oracle (the checker the HIP path is compared with).

The reference ships no golden vectors for this path (its tests compare live
against torch.nn.GRU), so the oracle is pinned by:
  * committed fixtures written by torch.nn.GRU in float64 (tests/golden);
  * live torch.nn.GRU float64 on shapes the fixtures do not cover;
  * brute-force central finite differences of a scalar loss (no torch);
  * closed forms: one step from h0 = 0, and W_hh = 0 (pointwise recurrence);
  * a planted mistake (swapped gate blocks) that the fixtures must reject.
"""
import os

import numpy as np
import pytest
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gru_golden.npz")
CASE_NAMES = ["c1_smoke", "odd_h5", "odd_h33", "two_layer", "t1_b1"]


def _case(name):
    data = np.load(GOLDEN)
    return {k.split("/", 1)[1]: data[k] for k in data.files if k.startswith(name + "/")}


def _params(case, L):
    return [{n: case[f"{n}_l{l}"] for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")} for l in range(L)]


@pytest.mark.parametrize("name", CASE_NAMES)
def test_oracle_matches_golden_fixtures(oracle, name):
    c = _case(name)
    L = int(c["dims"][0])
    res = oracle.stack_forward_backward(c["x"], c["h0"], _params(c, L), c["dy"], c["dhn"])
    np.testing.assert_allclose(res.y, c["y"], rtol=0, atol=1e-12)
    np.testing.assert_allclose(res.hn, c["hn"], rtol=0, atol=1e-12)
    np.testing.assert_allclose(res.dx, c["dx"], rtol=0, atol=1e-11)
    np.testing.assert_allclose(res.dhx, c["dh0"], rtol=0, atol=1e-11)
    for l in range(L):
        for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh"):
            np.testing.assert_allclose(res.grads[l][n], c[f"grad_{n}_l{l}"], rtol=0, atol=1e-10)


def test_oracle_f32_close_to_f64_on_golden(oracle):
    c = _case("c1_smoke")
    r64 = oracle.stack_forward_backward(c["x"], c["h0"], _params(c, 1), c["dy"], c["dhn"], dtype=np.float64)
    r32 = oracle.stack_forward_backward(c["x"], c["h0"], _params(c, 1), c["dy"], c["dhn"], dtype=np.float32)
    np.testing.assert_allclose(r32.y, r64.y, atol=1e-6)
    np.testing.assert_allclose(r32.dx, r64.dx, atol=1e-5)


def test_planted_gate_swap_is_caught_by_fixtures(oracle):
    """Swapping the r and z row blocks (a plausible indexing mistake) must fail."""
    c = _case("odd_h33")
    p = _params(c, 1)
    H = int(c["dims"][2])
    bad = {k: v.copy() for k, v in p[0].items()}
    for k in bad:
        v = bad[k]
        v[:H], v[H:2 * H] = p[0][k][H:2 * H].copy(), p[0][k][:H].copy()
    res = oracle.stack_forward_backward(c["x"], c["h0"], [bad], c["dy"], c["dhn"])
    assert np.abs(res.y - c["y"]).max() > 1e-3


@pytest.mark.parametrize("L,I,H,B,T", [(1, 4, 129, 2, 3), (1, 5, 130, 2, 3), (3, 6, 9, 2, 4), (1, 1, 1, 1, 3)])
def test_oracle_matches_live_torch_gru_f64(oracle, L, I, H, B, T):
    torch.manual_seed(7 + L + I + H)
    gru = torch.nn.GRU(I, H, num_layers=L, batch_first=True).double()
    x = torch.randn(B, T, I, dtype=torch.float64, requires_grad=True)
    h0 = torch.randn(L, B, H, dtype=torch.float64, requires_grad=True)
    y, hn = gru(x, h0)
    dy = torch.randn_like(y)
    dhn = torch.randn_like(hn)
    (y * dy).sum().add((hn * dhn).sum()).backward()
    params = [{n: getattr(gru, f"{n}_l{l}").detach().numpy() for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")}
              for l in range(L)]
    res = oracle.stack_forward_backward(x.detach().numpy(), h0.detach().numpy(), params, dy.numpy(), dhn.numpy())
    np.testing.assert_allclose(res.y, y.detach().numpy(), atol=1e-12)
    np.testing.assert_allclose(res.hn, hn.detach().numpy(), atol=1e-12)
    np.testing.assert_allclose(res.dx, x.grad.numpy(), atol=1e-11)
    np.testing.assert_allclose(res.dhx, h0.grad.numpy(), atol=1e-11)
    for l in range(L):
        for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh"):
            np.testing.assert_allclose(res.grads[l][n], getattr(gru, f"{n}_l{l}").grad.numpy(), atol=1e-10)


def _rand_layer(rng, I, H, scale=0.5):
    return {
        "weight_ih": rng.uniform(-scale, scale, (3 * H, I)),
        "weight_hh": rng.uniform(-scale, scale, (3 * H, H)),
        "bias_ih": rng.uniform(-scale, scale, 3 * H),
        "bias_hh": rng.uniform(-scale, scale, 3 * H),
    }


def test_oracle_backward_matches_finite_differences(oracle):
    """Brute force: d/dθ of L = <dy, y> + <dhn, h_n> by central differences."""
    rng = np.random.default_rng(11)
    B, T, I, H = 2, 4, 3, 5
    p = _rand_layer(rng, I, H)
    x = rng.standard_normal((B, T, I))
    h0 = rng.standard_normal((B, H))
    dy = rng.standard_normal((B, T, H))
    dhn = rng.standard_normal((B, H))

    def loss(x_, h0_, p_):
        f = oracle.forward(x_, h0_, p_["weight_ih"], p_["weight_hh"], p_["bias_ih"], p_["bias_hh"], with_cache=False)
        return float((f.y * dy).sum() + (f.hn * dhn).sum())

    f = oracle.forward(x, h0, p["weight_ih"], p["weight_hh"], p["bias_ih"], p["bias_hh"])
    g = oracle.backward(x, h0, p["weight_ih"], p["weight_hh"], f.y, f.cache, dy, dhn)
    eps = 1e-6
    checks = [("x", x, g.dx), ("h0", h0, g.dh0)] + [
        (k, p[k], v) for k, v in (("weight_ih", g.dw_ih), ("weight_hh", g.dw_hh), ("bias_ih", g.db_ih),
                                  ("bias_hh", g.db_hh))]
    for name, arr, analytic in checks:
        num = np.zeros_like(arr)
        it = np.nditer(arr, flags=["multi_index"])
        for _ in it:
            idx = it.multi_index
            orig = arr[idx]
            arr[idx] = orig + eps
            lp = loss(x, h0, p)
            arr[idx] = orig - eps
            lm = loss(x, h0, p)
            arr[idx] = orig
            num[idx] = (lp - lm) / (2 * eps)
        np.testing.assert_allclose(analytic, num, atol=1e-7, err_msg=name)


def test_oracle_single_step_closed_form(oracle):
    """T = 1, h0 = 0: h = (1 - z) n, z = s(W_iz x + b_iz + b_hz), n = tanh(W_in x + b_in + r b_hn)."""
    rng = np.random.default_rng(3)
    B, I, H = 3, 4, 6
    p = _rand_layer(rng, I, H)
    x = rng.standard_normal((B, 1, I))
    f = oracle.forward(x, np.zeros((B, H)), p["weight_ih"], p["weight_hh"], p["bias_ih"], p["bias_hh"])
    s = lambda v: 1.0 / (1.0 + np.exp(-v))
    gi = x[:, 0] @ p["weight_ih"].T + p["bias_ih"]
    bh = p["bias_hh"]
    r = s(gi[:, :H] + bh[:H])
    z = s(gi[:, H:2 * H] + bh[H:2 * H])
    n = np.tanh(gi[:, 2 * H:] + r * bh[2 * H:])
    np.testing.assert_allclose(f.y[:, 0], (1 - z) * n, atol=1e-14)
    np.testing.assert_allclose(f.cache[:, 0, 3 * H:], np.broadcast_to(bh[2 * H:], (B, H)), atol=1e-15)


def test_oracle_zero_recurrent_weights_is_pointwise(oracle):
    """W_hh = 0: a = b_hh each step, so the recurrence is an elementwise map."""
    rng = np.random.default_rng(5)
    B, T, I, H = 2, 6, 3, 4
    p = _rand_layer(rng, I, H)
    p["weight_hh"][:] = 0.0
    x = rng.standard_normal((B, T, I))
    h = rng.standard_normal((B, H))
    f = oracle.forward(x, h, p["weight_ih"], p["weight_hh"], p["bias_ih"], p["bias_hh"])
    s = lambda v: 1.0 / (1.0 + np.exp(-v))
    bh = p["bias_hh"]
    for t in range(T):
        gi = x[:, t] @ p["weight_ih"].T + p["bias_ih"]
        r = s(gi[:, :H] + bh[:H])
        z = s(gi[:, H:2 * H] + bh[H:2 * H])
        n = np.tanh(gi[:, 2 * H:] + r * bh[2 * H:])
        h = n + z * (h - n)
        np.testing.assert_allclose(f.y[:, t], h, atol=1e-14)


def test_oracle_none_gradients_mean_zero(oracle):
    """dy = None and dhn = None behave as zeros (reference gru.py:534-554)."""
    rng = np.random.default_rng(9)
    B, T, I, H = 2, 3, 2, 4
    p = _rand_layer(rng, I, H)
    x = rng.standard_normal((B, T, I))
    h0 = rng.standard_normal((B, H))
    f = oracle.forward(x, h0, p["weight_ih"], p["weight_hh"], p["bias_ih"], p["bias_hh"])
    dhn = rng.standard_normal((B, H))
    a = oracle.backward(x, h0, p["weight_ih"], p["weight_hh"], f.y, f.cache, None, dhn)
    b = oracle.backward(x, h0, p["weight_ih"], p["weight_hh"], f.y, f.cache, np.zeros((B, T, H)), dhn)
    np.testing.assert_array_equal(a.dx, b.dx)
    np.testing.assert_array_equal(a.dw_hh, b.dw_hh)


def test_row_parallel_oracle_equals_the_single_call():
    """The batch-row-parallel wrappers (used for the full-size parity check)
    give the single call's per-row results exactly and its weight gradients
    up to the grouping of the batch sum."""
    from oracle import gru_oracle

    rng = np.random.default_rng(11)
    B, T, I, H = 7, 5, 4, 6
    k = H ** -0.5
    w_ih, w_hh = rng.uniform(-k, k, (3 * H, I)), rng.uniform(-k, k, (3 * H, H))
    b_ih, b_hh = rng.uniform(-k, k, 3 * H), rng.uniform(-k, k, 3 * H)
    x, h0 = rng.standard_normal((B, T, I)), rng.standard_normal((B, H))
    dy, dhn = rng.standard_normal((B, T, H)), rng.standard_normal((B, H))
    f = gru_oracle.forward(x, h0, w_ih, w_hh, b_ih, b_hh)
    fp = gru_oracle.forward_rows_parallel(x, h0, w_ih, w_hh, b_ih, b_hh, threads=3)
    assert np.array_equal(f.y, fp.y) and np.array_equal(f.hn, fp.hn) and np.array_equal(f.cache, fp.cache)
    b = gru_oracle.backward(x, h0, w_ih, w_hh, f.y, f.cache, dy, dhn)
    bp = gru_oracle.backward_rows_parallel(x, h0, w_ih, w_hh, f.y, f.cache, dy, dhn, threads=3)
    assert np.array_equal(b.dx, bp.dx) and np.array_equal(b.dh0, bp.dh0)
    for name in ("dw_ih", "dw_hh", "db_ih", "db_hh"):
        np.testing.assert_allclose(getattr(bp, name), getattr(b, name), rtol=1e-13, atol=1e-13)


def test_row_parallel_stack_equals_the_single_stack_call():
    """The row-parallel stack (used for the full-size two-layer check) gives
    stack_forward_backward's per-row results exactly and its weight gradients
    up to the grouping of the batch sum, with the output gradient formed from
    each chunk's own forward result (here the MSE gradient against a target),
    and matches the committed two-layer torch.nn.GRU fixture."""
    from oracle import gru_oracle

    c = _case("two_layer")
    L = int(c["dims"][0])
    params = _params(c, L)
    dy = c["dy"]
    ref = gru_oracle.stack_forward_backward(c["x"], c["h0"], params, dy, c["dhn"])
    par = gru_oracle.stack_rows_parallel(c["x"], c["h0"], params, lambda y, a, b: dy[a:b], threads=2,
                                         dhn=c["dhn"])
    assert np.array_equal(ref.y, par.y) and np.array_equal(ref.hn, par.hn)
    assert np.array_equal(ref.dx, par.dx) and np.array_equal(ref.dhx, par.dhx)
    for l in range(L):
        for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh"):
            np.testing.assert_allclose(par.grads[l][n], ref.grads[l][n], rtol=1e-13, atol=1e-13)
            np.testing.assert_allclose(par.grads[l][n], c[f"grad_{n}_l{l}"], rtol=0, atol=1e-11)
    np.testing.assert_allclose(par.y, c["y"], rtol=0, atol=1e-12)
    # an output gradient that depends on the chunk's forward output
    rng = np.random.default_rng(3)
    target = rng.standard_normal(ref.y.shape)
    scale = 2.0 / target.size
    mse = gru_oracle.stack_rows_parallel(c["x"], c["h0"], params, lambda y, a, b: scale * (y - target[a:b]),
                                         threads=3)
    full = gru_oracle.stack_forward_backward(c["x"], c["h0"], params, scale * (mse.y - target))
    assert np.array_equal(full.dx, mse.dx) and np.array_equal(full.dhx, mse.dhx)
