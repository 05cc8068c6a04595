"""GPU parity of the RMSNorm + dropout and QKV-epilogue kernels (dk_rms_fwd/bwd,
dk_qkv_epilogue_fwd/bwd) with the oracle, following the reference's own tests
(solution/test_kernels.py:139-257, dev/test_emu.py:74-219): the norm to the reference tests'
tolerances (its row sums reduce in another order than the oracle's), the QKV epilogue bit for bit
(the same fp32 operations in the same order), every output the reference checks exactly (x +
delta, dropped elements, out16 = fp16(out), the forward without y, the backward from x + delta)
checked exactly here too, on ragged row counts and several hidden sizes."""

import numpy as np
import pytest

from tests.helpers import host, log

pytestmark = pytest.mark.gpu
F32, F16 = np.float32, np.float16


@pytest.fixture(scope="module")
def torch():
    import torch as t
    return t


def _close(got, want, rtol, atol, what):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    bad = np.abs(got - want) > atol + rtol * np.abs(want)
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} beyond tolerance, max err " \
                          f"{np.abs(got - want).max():.3g}"


def _exact(got, want, what):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape and np.array_equal(got.view(np.uint8), want.view(np.uint8)), \
        f"{what}: {np.count_nonzero(got != want)} of {got.size} differ"


@pytest.mark.parametrize("n,d", [(300, 1536), (5, 1536), (7, 896), (33, 2048), (4, 4096)])
def test_rmsnorm_forward_backward_and_dropout(torch, n, d):
    from decentrik_prime_amd import k_norm
    from oracle import norm
    log(f"rmsnorm fwd/bwd + dropout, n={n} d={d}")
    dev = "cuda"
    g = torch.Generator(device=dev)
    g.manual_seed(n * 7 + d)
    eps, p = 1e-6, 0.05
    ks = 1.0 / float(torch.tensor(1.0 - p, dtype=torch.float32))
    x = torch.randn(n, d, device=dev, generator=g)
    delta = (torch.randn(n, d, device=dev, generator=g) * 0.5).half()
    w = torch.rand(d, device=dev, generator=g) + 0.5
    mq = (torch.rand(n, d, device=dev, generator=g) >= p).to(torch.uint8)
    mv = (torch.rand(n, d, device=dev, generator=g) >= p).to(torch.uint8)
    y = torch.empty(n, d, dtype=torch.float16, device=dev)
    xq, xv = torch.empty_like(y), torch.empty_like(y)
    xout = torch.empty(n, d, device=dev)
    rstd = torch.empty(n, device=dev)
    k_norm.rms_forward(x, w, y, rstd, eps, delta=delta, xout=xout, xq=xq, xv=xv, mq=mq, mv=mv,
                       keep_scale=ks)
    torch.cuda.synchronize()
    h, r_o, y_o, xq_o, xv_o = norm.rms_fwd(host(x), host(w), eps, host(delta), host(mq), host(mv),
                                           ks)
    _exact(host(xout), h, "xout = x + delta")
    _close(host(rstd), r_o, 1e-6, 0, "rstd")
    _close(host(y), y_o, 2e-3, 2e-3, "y")
    _close(host(xq), xq_o, 2e-3, 2e-3, "dropout q")
    _close(host(xv), xv_o, 2e-3, 2e-3, "dropout v")
    assert not np.any(host(xq)[host(mq) == 0]) and not np.any(host(xv)[host(mv) == 0])
    # the float64 closed form (the reference test's own check)
    hh = h.astype(np.float64)
    ref = host(w).astype(np.float64) * hh / np.sqrt((hh ** 2).mean(1, keepdims=True) + eps)
    _close(host(y), ref, 2e-3, 2e-3, "y vs float64")

    # the forward without y: rstd and the dropout inputs identical, y untouched
    y_keep = torch.full_like(y, 3.0)
    rstd3, xq3, xv3 = torch.empty_like(rstd), torch.empty_like(y), torch.empty_like(y)
    k_norm.rms_forward(x, w, None, rstd3, eps, delta=delta, xq=xq3, xv=xv3, mq=mq, mv=mv,
                       keep_scale=ks)
    torch.cuda.synchronize()
    _exact(host(rstd3), host(rstd), "rstd without y")
    _exact(host(xq3), host(xq), "xq without y")
    _exact(host(xv3), host(xv), "xv without y")
    assert torch.equal(y_keep, torch.full_like(y, 3.0))

    # backward: in place on the residual gradient, both LoRA input grads, fp16 copy
    dy16 = torch.randn(n, d, device=dev, generator=g).half()
    lq = (torch.randn(n, d, device=dev, generator=g) * 0.3).half()
    lv = (torch.randn(n, d, device=dev, generator=g) * 0.3).half()
    dres = torch.randn(n, d, device=dev, generator=g)
    gscale = torch.tensor([0.5], device=dev)
    hdev = torch.from_numpy(h).to(dev)
    out = dres.clone()
    out16 = torch.empty(n, d, dtype=torch.float16, device=dev)
    k_norm.rms_backward(dy16, gscale, hdev, w, rstd, out, dres=out, lq=lq, lv=lv, mq=mq, mv=mv,
                        keep_scale=ks, out16=out16)
    torch.cuda.synchronize()
    o_ref, _ = norm.rms_bwd(host(dy16), 0.5, h, host(w), host(rstd), host(dres), host(lq), host(lv),
                            host(mq), host(mv), ks)
    _close(host(out), o_ref, 1e-4, 1e-4, "rms backward vs oracle")
    up = (host(dy16).astype(np.float64) * 0.5 + host(mq) * host(lq).astype(np.float64) * ks
          + host(mv) * host(lv).astype(np.float64) * ks)
    _close(host(out), norm.rms_bwd_float64(up, h, host(w), eps) + host(dres), 1e-4, 1e-4,
           "rms backward vs float64")
    _exact(host(out16), host(out).astype(F16), "out16 = fp16(out)")
    # the backward given the norm input as x + delta: bit-identical
    out_d = dres.clone()
    out16_d = torch.empty_like(out16)
    k_norm.rms_backward(dy16, gscale, x, w, rstd, out_d, dres=out_d, lq=lq, lv=lv, mq=mq, mv=mv,
                        keep_scale=ks, out16=out16_d, delta=delta)
    torch.cuda.synchronize()
    _exact(host(out_d), host(out), "backward from x + delta")
    _exact(host(out16_d), host(out16), "backward from x + delta, fp16")
    # no LoRA, no residual, no fp16 copy
    out_p = torch.empty_like(out)
    k_norm.rms_backward(dy16, gscale, hdev, w, rstd, out_p)
    torch.cuda.synchronize()
    p_ref, _ = norm.rms_bwd(host(dy16), 0.5, h, host(w), host(rstd))
    _close(host(out_p), p_ref, 1e-4, 1e-4, "plain backward")


@pytest.mark.parametrize("n,nq,nkv,hd", [(257, 12, 2, 128), (7, 12, 2, 128), (64, 14, 2, 64)])
def test_qkv_epilogue_forward_backward(torch, n, nq, nkv, hd):
    from decentrik_prime_amd import k_rope
    from oracle import rope
    log(f"qkv epilogue fwd/bwd, n={n} heads {nq}/{nkv} hd={hd}")
    dev = "cuda"
    rng = np.random.default_rng(n + hd)
    cos, sin = rope.rope_tables(512, hd)
    pos = rng.integers(0, 512, n).astype(np.int32)
    qkv = rng.standard_normal((n, (nq + 2 * nkv) * hd)).astype(F16)
    lq = (rng.standard_normal((n, nq * hd)) * 0.1).astype(F16)
    lv = (rng.standard_normal((n, nkv * hd)) * 0.1).astype(F16)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    tq, tc, ts, tp = t(qkv), t(cos), t(sin), t(pos)
    k_rope.qkv_epilogue_forward(tq, t(lq), t(lv), tp, tc, ts, 2.0, nq, nkv, hd)
    torch.cuda.synchronize()
    _exact(host(tq), rope.qkv_epilogue_fwd(qkv, lq, lv, pos, cos, sin, 2.0, nq, nkv, hd),
           "qkv forward vs oracle")
    # backward: per-query-head fp32 partials (gin = nq / nkv), and fp16 grads already reduced
    gin = nq // nkv
    dq = rng.standard_normal((n, nq * hd)).astype(F32)
    dkp = rng.standard_normal((n, nkv * gin * hd)).astype(F32)
    dvp = rng.standard_normal((n, nkv * gin * hd)).astype(F32)
    out = torch.empty(n, (nq + 2 * nkv) * hd, dtype=torch.float16, device=dev)
    k_rope.qkv_epilogue_backward(t(dq), t(dkp), t(dvp), tp, tc, ts, out, nq, nkv, hd, gin)
    torch.cuda.synchronize()
    _exact(host(out), rope.qkv_epilogue_bwd(dq, dkp, dvp, pos, cos, sin, nq, nkv, hd, gin),
           "qkv backward (fp32, partials) vs oracle")
    dk16 = dkp.reshape(n, nkv, gin, hd).sum(2).reshape(n, -1).astype(F16)
    dv16 = dvp.reshape(n, nkv, gin, hd).sum(2).reshape(n, -1).astype(F16)
    out1 = torch.empty_like(out)
    k_rope.qkv_epilogue_backward(t(dq.astype(F16)), t(dk16), t(dv16), tp, tc, ts, out1, nq, nkv, hd, 1)
    torch.cuda.synchronize()
    _exact(host(out1), rope.qkv_epilogue_bwd(dq.astype(F16), dk16, dv16, pos, cos, sin, nq, nkv, hd,
                                             1), "qkv backward (fp16, reduced) vs oracle")


@pytest.mark.parametrize("m", [2048, 200])
def test_qkv_gemm_with_rotary_epilogue(torch, m):
    """The fused QKV projection with the rotary embedding in the GEMM epilogue against the
    unfused chain (GEMM + bias, LoRA up, then the standalone QKV epilogue kernel, whose order of
    operations it follows): bit-identical when the chain's lq16 / lv16 are the epilogue's own
    LoRA products (a GEMM with a zero weight gives fp16(s lo16) = s lo16 exactly); within the
    GEMM tolerance of the oracle; the v columns equal dk_h16_linear_fwd_lora's."""
    from decentrik_prime_amd import k_rope, w4linear
    from oracle import linear, rope
    from tests.helpers import cuda16, lora_inputs, nf4_weight, to_w4
    log(f"qkv GEMM + rotary epilogue, M={m}")
    D, KV, nq, nkv, hd = 1536, 256, 12, 2, 128
    q = nf4_weight(D + 2 * KV, D, seed=217)
    x, aq, bq, mq, _ = lora_inputs(m, D, D, seed=31)
    _, av, bv, mv, _ = lora_inputs(m, D, KV, seed=32)
    rng = np.random.default_rng(33)
    bias = (rng.standard_normal(D + 2 * KV) * 0.1).astype(F16)
    cos, sin = rope.rope_tables(4096, hd)
    pos = rng.integers(0, 4096, m).astype(np.int32)
    w = to_w4(q)
    w16 = w.dequantize()
    ks = linear.keep_scale(0.05)
    zq = w4linear.lora_down(cuda16(x), cuda16(aq), torch.from_numpy(mq).cuda(), ks)
    zv = w4linear.lora_down(cuda16(x), cuda16(av), torch.from_numpy(mv).cuda(), ks)
    terms = [(zq, cuda16(bq), 0, D, 2.0), (zv, cuda16(bv), D + KV, D + 2 * KV, 2.0)]
    tp = torch.from_numpy(pos).cuda()
    tc, ts = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    fused = w4linear.linear_forward_rope(cuda16(x), w, cuda16(bias), terms, tp, tc, ts,
                                         (nq + nkv) * hd, w16=w16)
    # unfused: q16/k16/v16 = GEMM + bias; lq16, lv16 = fp16(z B^T); then the epilogue kernel
    chain = w4linear.linear_forward_lora(cuda16(x), w, cuda16(bias), [], w16=w16)
    lora2 = w4linear.linear_forward_lora(cuda16(x), w, None, terms, w16=torch.zeros_like(w16))
    lq16 = (lora2[:, :D] * 0.5).contiguous()
    lv16 = (lora2[:, D + KV:] * 0.5).contiguous()
    k_rope.qkv_epilogue_forward(chain, lq16, lv16, tp, tc, ts, 2.0, nq, nkv, hd)
    plain = w4linear.linear_forward_lora(cuda16(x), w, cuda16(bias), terms, w16=w16)
    torch.cuda.synchronize()
    a = host(fused)
    if m == 2048:   # the chain's GEMMs run the same kernel and tile plan
        _exact(a, host(chain), "rotary GEMM vs GEMM + LoRA up + QKV epilogue")
        _exact(a[:, (nq + nkv) * hd:], host(plain)[:, (nq + nkv) * hd:], "v columns")
    else:           # the chain's plain GEMMs split K on the NF4-form kernel: summation order only
        b = host(chain).astype(np.float64)
        tol = 2 * 2.0 ** -10 * np.abs(b) + 2.0 ** -11 * np.abs(b).max()
        assert not (np.abs(a.astype(np.float64) - b) > tol).any(), "rotary GEMM vs chain"
    # oracle: fp16 GEMM + bias, LoRA up, rotary (oracle.rope), at the GEMM tolerance
    base = linear.mm16(x, q["deq"].T)
    base = (base.astype(np.float32) + bias.astype(np.float32)).astype(F16)
    lq_o = linear.mm16(host(zq), bq.T)
    lv_o = linear.mm16(host(zv), bv.T)
    ref = rope.qkv_epilogue_fwd(base, lq_o, lv_o, pos, cos, sin, 2.0, nq, nkv, hd)
    _close(a, ref, 1e-2, 2e-2, "rotary qkv vs oracle")
    with pytest.raises(ValueError):
        w4linear.linear_forward_rope(cuda16(x), w, cuda16(bias), terms, tp, tc[:, :64].contiguous(),
                                     ts[:, :64].contiguous(), (nq + nkv) * hd, w16=w16, hd=64)
