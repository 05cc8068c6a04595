"""Pins of the RMSNorm + dropout and QKV-epilogue oracles (oracle/norm.py, oracle/rope.py) against
formulations that do not share their code: float64 closed forms, torch float64 autograd, a finite
difference and the adjoint identity, with the checks and tolerances of the reference's own tests
(solution/test_kernels.py:139-257, dev/test_emu.py:74-219)."""

import numpy as np
import torch

from oracle import norm, rope

F32, F16 = np.float32, np.float16


def _close(got, want, rtol, atol, what):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    bad = np.abs(got - want) > atol + rtol * np.abs(want)
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} beyond tolerance, max err " \
                          f"{np.abs(got - want).max():.3g}"


def _norm_inputs(n=7, d=1536, seed=0, p=0.05):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, d)).astype(F32)
    delta = (rng.standard_normal((n, d)) * 0.5).astype(F16)
    w = rng.uniform(0.5, 1.5, d).astype(F32)
    mq = (rng.uniform(size=(n, d)) >= p).astype(np.uint8)
    mv = (rng.uniform(size=(n, d)) >= p).astype(np.uint8)
    ks = 1.0 / float(F32(1.0 - p))
    return x, delta, w, mq, mv, ks


def test_rms_forward_closed_form():
    x, delta, w, mq, mv, ks = _norm_inputs()
    eps = 1e-6
    h, rstd, y, xq, xv = norm.rms_fwd(x, w, eps, delta, mq, mv, ks)
    href = x.astype(np.float64) + delta.astype(np.float64)
    assert np.array_equal(h, (x + delta.astype(F32)).astype(F32))        # x + delta exactly in fp32
    r = 1.0 / np.sqrt((href ** 2).mean(1) + eps)
    yr = w.astype(np.float64) * href * r[:, None]
    _close(rstd, r, 1e-6, 0, "rstd")
    _close(y, yr, 1e-3, 2e-3, "y fp16")
    _close(xq, np.where(mq != 0, yr * ks, 0), 1e-3, 2e-3, "dropout q")
    _close(xv, np.where(mv != 0, yr * ks, 0), 1e-3, 2e-3, "dropout v")
    assert not np.any(xq[mq == 0]) and not np.any(xv[mv == 0])
    # no delta: the norm of x itself
    _, r2, y2, _, _ = norm.rms_fwd(x, w, eps)
    _close(y2, w * x * (1.0 / np.sqrt((x.astype(np.float64) ** 2).mean(1) + eps))[:, None], 1e-3,
           2e-3, "y (no delta)")


def test_rms_backward_autograd_and_finite_difference():
    x, delta, w, mq, mv, ks = _norm_inputs(n=5, seed=1)
    eps = 1e-6
    h, rstd, _, _, _ = norm.rms_fwd(x, w, eps, delta)
    rng = np.random.default_rng(2)
    dy16 = rng.standard_normal(h.shape).astype(F16)
    lq = (rng.standard_normal(h.shape) * 0.3).astype(F16)
    lv = (rng.standard_normal(h.shape) * 0.3).astype(F16)
    dres = rng.standard_normal(h.shape).astype(F32)
    gs = 0.75
    out, out16 = norm.rms_bwd(dy16, gs, h, w, rstd, dres, lq, lv, mq, mv, ks)
    # torch float64 autograd of sum(upstream * y(h))
    hh = torch.from_numpy(h.astype(np.float64)).requires_grad_(True)
    wt = torch.from_numpy(w.astype(np.float64))
    yy = wt * (hh * torch.rsqrt(hh.pow(2).mean(-1, keepdim=True) + eps))
    up = (torch.from_numpy(dy16.astype(np.float64)) * gs
          + torch.from_numpy(mq.astype(np.float64)) * torch.from_numpy(lq.astype(np.float64)) * ks
          + torch.from_numpy(mv.astype(np.float64)) * torch.from_numpy(lv.astype(np.float64)) * ks)
    (yy * up).sum().backward()
    _close(out, hh.grad.numpy() + dres, 1e-4, 1e-4, "rms bwd vs autograd")
    assert np.array_equal(out16, out.astype(F16))
    # the float64 closed form agrees with autograd, and a central difference pins one element
    ref = norm.rms_bwd_float64(up.numpy(), h, w, eps)
    _close(ref, hh.grad.numpy(), 1e-9, 1e-9, "closed form vs autograd")
    i, j = 2, 77

    def f(row):
        return np.sum(up.numpy()[i] * w * row / np.sqrt((row ** 2).mean() + eps))
    e = np.zeros(h.shape[1])
    e[j] = 1e-5
    hd = h[i].astype(np.float64)
    fd = (f(hd + e) - f(hd - e)) / 2e-5
    _close(out[i, j] - dres[i, j], fd, 1e-5, 1e-6, "rms bwd vs finite difference")


def _rope_inputs(n=7, nq=12, nkv=2, hd=128, seed=3, positions=64):
    rng = np.random.default_rng(seed)
    cos, sin = rope.rope_tables(positions, hd)
    pos = rng.integers(0, positions, n).astype(np.int32)
    qkv = rng.standard_normal((n, (nq + 2 * nkv) * hd)).astype(F16)
    lq = (rng.standard_normal((n, nq * hd)) * 0.1).astype(F16)
    lv = (rng.standard_normal((n, nkv * hd)) * 0.1).astype(F16)
    return qkv, lq, lv, pos, cos, sin


def _rope_t(x, c, s):
    """x * cos + rotate_half(x) * sin over the full-width tables (torch, any dtype)."""
    half = x.shape[-1] // 2
    return x * c + torch.cat((-x[..., half:], x[..., :half]), -1) * s


def test_rope_forward_rotate_half_form():
    nq, nkv, hd = 12, 2, 128
    qkv, lq, lv, pos, cos, sin = _rope_inputs()
    n = qkv.shape[0]
    out = rope.qkv_epilogue_fwd(qkv, lq, lv, pos, cos, sin, 2.0, nq, nkv, hd)
    c = torch.from_numpy(cos[pos].astype(np.float64))[:, None, :]
    s = torch.from_numpy(sin[pos].astype(np.float64))[:, None, :]
    o = torch.from_numpy(qkv.astype(np.float64))
    q = o[:, :nq * hd].view(n, nq, hd) + torch.from_numpy(lq.astype(np.float64)).view(n, nq, hd) * 2
    k = o[:, nq * hd:(nq + nkv) * hd].view(n, nkv, hd)
    v = o[:, (nq + nkv) * hd:] + torch.from_numpy(lv.astype(np.float64)) * 2
    _close(out[:, :nq * hd], _rope_t(q, c, s).reshape(n, -1).numpy(), 2e-3, 2e-3, "q rope+lora")
    _close(out[:, nq * hd:(nq + nkv) * hd], _rope_t(k, c, s).reshape(n, -1).numpy(), 2e-3, 2e-3,
           "k rope")
    _close(out[:, (nq + nkv) * hd:], v.numpy(), 2e-3, 2e-3, "v lora")
    # position 0 is the identity rotation on q and k
    z = np.zeros_like(pos)
    zero_lora = rope.qkv_epilogue_fwd(qkv, np.zeros_like(lq), np.zeros_like(lv), z, cos, sin, 2.0,
                                      nq, nkv, hd)
    assert np.array_equal(zero_lora, qkv)


def test_rope_backward_autograd_adjoint_and_gqa():
    nq, nkv, hd = 12, 2, 128
    g = nq // nkv
    qkv, lq, lv, pos, cos, sin = _rope_inputs(seed=4)
    n = qkv.shape[0]
    rng = np.random.default_rng(5)
    dq = rng.standard_normal((n, nq * hd)).astype(F32)
    dkp = rng.standard_normal((n, nq * hd)).astype(F32)
    dvp = rng.standard_normal((n, nq * hd)).astype(F32)
    out = rope.qkv_epilogue_bwd(dq, dkp, dvp, pos, cos, sin, nq, nkv, hd, g)
    c = torch.from_numpy(cos[pos].astype(np.float64))[:, None, :]
    s = torch.from_numpy(sin[pos].astype(np.float64))[:, None, :]
    qr = torch.zeros(n, nq, hd, dtype=torch.float64, requires_grad=True)
    kr = torch.zeros(n, nkv, hd, dtype=torch.float64, requires_grad=True)
    vr = torch.zeros(n, nkv, hd, dtype=torch.float64, requires_grad=True)
    t = lambda a: torch.from_numpy(a.astype(np.float64))  # noqa: E731
    loss = (_rope_t(qr, c, s) * t(dq).view(n, nq, hd)).sum()
    loss = loss + (_rope_t(kr, c, s).repeat_interleave(g, 1) * t(dkp).view(n, nq, hd)).sum()
    loss = loss + (vr.repeat_interleave(g, 1) * t(dvp).view(n, nq, hd)).sum()
    loss.backward()
    _close(out[:, :nq * hd], qr.grad.reshape(n, -1).numpy(), 3e-3, 2e-3, "dq")
    _close(out[:, nq * hd:(nq + nkv) * hd], kr.grad.reshape(n, -1).numpy(), 1e-2, 2e-3, "dk")
    _close(out[:, (nq + nkv) * hd:], vr.grad.reshape(n, -1).numpy(), 1e-2, 2e-3, "dv")
    # GIN = 1 (grads already reduced per KV head, fp16) gives the same within fp16 rounding
    dk16 = dkp.reshape(n, nkv, g, hd).sum(2).reshape(n, -1).astype(F16)
    dv16 = dvp.reshape(n, nkv, g, hd).sum(2).reshape(n, -1).astype(F16)
    out1 = rope.qkv_epilogue_bwd(dq.astype(F16), dk16, dv16, pos, cos, sin, nq, nkv, hd, 1)
    _close(out1[:, nq * hd:(nq + nkv) * hd], kr.grad.reshape(n, -1).numpy(), 3e-2, 3e-3, "dk (GIN 1)")
    # adjoint: <rope(x), d> == <x, rope^T(d)> for one head of every row, in float64
    x = rng.standard_normal((n, 1, hd))
    dd = rng.standard_normal((n, 1, hd))
    lhs = float((_rope_t(t(x), c, s) * t(dd)).sum())
    back = rope.qkv_epilogue_bwd(np.tile(dd.reshape(n, hd), (1, nq)).astype(F32),
                                 np.zeros((n, nkv * hd), F32), np.zeros((n, nkv * hd), F32), pos,
                                 cos, sin, nq, nkv, hd, 1)
    rhs = float(np.sum(x.reshape(n, hd) * back[:, :hd].astype(np.float64)))
    assert abs(lhs - rhs) <= 2e-3 * (abs(lhs) + np.abs(x).sum()), (lhs, rhs)
