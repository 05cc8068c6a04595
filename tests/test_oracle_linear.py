"""Pins of the CPU oracle's linear/LoRA code (oracle/linear.py) and SwiGLU code (oracle/mlp.py)
against float64 autograd of the forward expressions: the oracle's hand-written backward formulas
(transposes, the LoRA scale s, the dropout keep-scale, the mask) must agree with the derivatives
torch computes itself, to within the fp16 roundings the reference inserts."""

import numpy as np
import torch

from oracle import linear, mlp

F16, F32 = np.float16, np.float32


def _data(m=64, k=128, n=96, r=16, seed=0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(F16)
    w = (rng.standard_normal((n, k)) * 0.05).astype(F16)
    bias = (rng.standard_normal(n) * 0.1).astype(F16)
    a = rng.uniform(-1, 1, (r, k)).astype(F16) / F16(np.sqrt(k))
    b = (rng.standard_normal((n, r)) * 0.2).astype(F16)
    mask = (rng.random((m, k)) >= 0.05).astype(np.uint8)
    dy = (rng.standard_normal((m, n)) * 0.1).astype(F16)
    return x, w, bias, a, b, mask, dy


def _ref64(x, w, bias, a, b, mask, dy, s, ks):
    t = lambda v: torch.tensor(np.asarray(v, dtype=np.float64), requires_grad=True)  # noqa: E731
    X, W, A, B = t(x), t(w), t(a), t(b)
    M = torch.tensor(mask.astype(np.float64))
    y = X @ W.T + torch.tensor(bias.astype(np.float64)) + s * ((M * X * ks) @ A.T) @ B.T
    y.backward(torch.tensor(dy.astype(np.float64)))
    return y.detach().numpy(), X.grad.numpy(), A.grad.numpy(), B.grad.numpy()


def _close(got, want, rtol, atol):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert np.all(np.abs(got - want) <= atol + rtol * np.abs(want)), np.abs(got - want).max()


def test_linear_forward_and_backward_match_autograd():
    s, ks = 2.0, linear.keep_scale(0.05)
    x, w, bias, a, b, mask, dy = _data()
    y_ref, dx_ref, da_ref, db_ref = _ref64(x, w, bias, a, b, mask, dy, s, ks)
    y, z = linear.linear_fwd(x, w, bias, mask, ks, a, b, s)
    _close(y, y_ref, 1e-2, 2e-2)
    g = linear.linear_bwd(dy, w, z, x, mask, ks, a, b, s)
    scale = lambda v: np.abs(v).max()  # noqa: E731
    _close(g["dx"], dx_ref, 1e-2, 1e-2 * scale(dx_ref))
    _close(g["dA"], da_ref, 1e-2, 1e-2 * scale(da_ref))
    _close(g["dB"], db_ref, 1e-2, 1e-2 * scale(db_ref))


def test_linear_backward_detects_a_missing_keep_scale():
    # the autograd comparison above has the power to see a dropped factor of 1/0.95
    s, ks = 2.0, linear.keep_scale(0.05)
    x, w, bias, a, b, mask, dy = _data(seed=1)
    _, _, da_ref, _ = _ref64(x, w, bias, a, b, mask, dy, s, ks)
    y, z = linear.linear_fwd(x, w, bias, mask, 1.0, a, b, s)
    g = linear.linear_bwd(dy, w, z, x, mask, 1.0, a, b, s)
    err = np.abs(g["dA"] - da_ref).max() / np.abs(da_ref).max()
    assert err > 2e-2


def test_keep_scale_is_pytorch_dropout_scale():
    assert linear.keep_scale(0.05) == float(F32(1.0) / F32(0.95))
    assert linear.keep_scale(0.05) != 1.0 / 0.95


def test_lora_down_is_the_dropped_input_times_a():
    x, w, bias, a, b, mask, dy = _data(seed=2)
    ks = linear.keep_scale(0.05)
    z = linear.lora_down(x, mask, ks, a)
    want = (mask * x.astype(np.float64) * ks) @ a.astype(np.float64).T
    _close(z, want, 1e-2, 1e-2)


def test_gated_silu_matches_autograd():
    rng = np.random.default_rng(4)
    n, inter = 33, 1100
    gu = (rng.standard_normal((n, 2 * inter)) * 2).astype(F16)
    g = torch.tensor(gu[:, :inter].astype(np.float64), requires_grad=True)
    u = torch.tensor(gu[:, inter:].astype(np.float64), requires_grad=True)
    ref = torch.nn.functional.silu(g) * u
    _close(mlp.gated_silu_fwd(gu), ref.detach().numpy(), 2e-3, 2e-3)
    da = rng.standard_normal((n, inter)).astype(F16)
    ref.backward(torch.tensor(da.astype(np.float64)))
    out = mlp.gated_silu_bwd(gu, da)
    _close(out[:, :inter], g.grad.numpy(), 3e-3, 3e-3)
    _close(out[:, inter:], u.grad.numpy(), 3e-3, 3e-3)


def test_example_swiglu_matches_autograd():
    rng = np.random.default_rng(5)
    gate = (rng.standard_normal(4000) * 2).astype(F16)
    up = rng.standard_normal(4000).astype(F16)
    G = torch.tensor(gate.astype(np.float64), requires_grad=True)
    U = torch.tensor(up.astype(np.float64), requires_grad=True)
    ref = G * torch.sigmoid(G) * U
    _close(mlp.swiglu_fwd(gate, up), ref.detach().numpy(), 2e-3, 2e-3)
    grad = rng.standard_normal(4000).astype(F16)
    ref.backward(torch.tensor(grad.astype(np.float64)))
    dg, du = mlp.swiglu_bwd(grad, gate, up)
    _close(dg, G.grad.numpy(), 3e-3, 3e-3)
    _close(du, U.grad.numpy(), 3e-3, 3e-3)


def test_mlp_backward_chain_matches_autograd():
    rng = np.random.default_rng(6)
    m, d, inter = 32, 64, 96
    x = rng.standard_normal((m, d)).astype(F16)
    wgu = (rng.standard_normal((2 * inter, d)) * 0.1).astype(F16)
    wd = (rng.standard_normal((d, inter)) * 0.1).astype(F16)
    dy = rng.standard_normal((m, d)).astype(F16)
    X = torch.tensor(x.astype(np.float64), requires_grad=True)
    gu = X @ torch.tensor(wgu.astype(np.float64)).T
    h = torch.nn.functional.silu(gu[:, :inter]) * gu[:, inter:]
    y = h @ torch.tensor(wd.astype(np.float64)).T
    y.backward(torch.tensor(dy.astype(np.float64)))
    gu16, h16, y16 = mlp.mlp_fwd(x, wgu, wd)
    _close(y16, y.detach().numpy(), 1e-2, 2e-2)
    _, dx = mlp.mlp_bwd(dy, gu16, wgu, wd)
    _close(dx, X.grad.numpy(), 2e-2, 2e-2 * np.abs(X.grad.numpy()).max())
