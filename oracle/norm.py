"""CPU restatement of the fused residual add + RMSNorm with the two LoRA dropout masks, forward
and backward.  TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product path.

forward (solution/k_norm.py:38-58), per token row of hidden D, fp32 arithmetic:
    x    = x_prev [+ fp32(delta16)]
    rstd = 1 / sqrt(sum(x * x) * (1 / D) + eps)
    y    = w * (x * rstd)
    y16 = fp16(y);  xq16 = fp16(keep_q ? y * ks : 0);  xv16 = fp16(keep_v ? y * ks : 0)
backward (solution/k_norm.py:61-88):
    dy  = fp32(dy16) * gscale [+ (keep_q ? fp32(lq16) * ks : 0)] [+ (keep_v ? fp32(lv16) * ks : 0)]
    xh  = x * rstd;  g = dy * w;  c = sum(g * xh) * (1 / D)
    dx  = (g - xh * c) * rstd [+ dres];  out16 = fp16(dx)

Sums are taken in float64 here and rounded once (the GPU reduces in another order: the two
agree to the tolerances of solution/test_kernels.py:139-208).
"""

import numpy as np

F32, F16 = np.float32, np.float16


def rms_fwd(x, w, eps, delta=None, mq=None, mv=None, keep_scale=1.0):
    """Returns (h, rstd, y16, xq16, xv16); h = the norm input x [+ delta] (fp32), xq16 / xv16 None
    without masks."""
    h = np.asarray(x, F32)
    if delta is not None:
        h = (h + np.asarray(delta, F16).astype(F32)).astype(F32)
    d = h.shape[-1]
    ms = (np.sum(h.astype(np.float64) ** 2, axis=-1) * (1.0 / d)).astype(F32)
    rstd = (1.0 / np.sqrt(ms.astype(np.float64) + eps)).astype(F32)
    y = (np.asarray(w, F32) * (h * rstd[..., None]).astype(F32)).astype(F32)
    ks = F32(keep_scale)
    xq = xv = None
    if mq is not None:
        xq = np.where(np.asarray(mq) != 0, (y * ks).astype(F32), F32(0)).astype(F16)
    if mv is not None:
        xv = np.where(np.asarray(mv) != 0, (y * ks).astype(F32), F32(0)).astype(F16)
    return h, rstd, y.astype(F16), xq, xv


def rms_bwd(dy16, gscale, h, w, rstd, dres=None, lq=None, lv=None, mq=None, mv=None,
            keep_scale=1.0):
    """Returns (out fp32, out16); h is the norm input (x + delta)."""
    dy = (np.asarray(dy16, F16).astype(F32) * F32(gscale)).astype(F32)
    ks = F32(keep_scale)
    if lq is not None:
        dy = (dy + np.where(np.asarray(mq) != 0, (np.asarray(lq, F16).astype(F32) * ks).astype(F32),
                            F32(0))).astype(F32)
    if lv is not None:
        dy = (dy + np.where(np.asarray(mv) != 0, (np.asarray(lv, F16).astype(F32) * ks).astype(F32),
                            F32(0))).astype(F32)
    h = np.asarray(h, F32)
    r = np.asarray(rstd, F32)[..., None]
    xh = (h * r).astype(F32)
    g = (dy * np.asarray(w, F32)).astype(F32)
    d = h.shape[-1]
    c = (np.sum(g.astype(np.float64) * xh.astype(np.float64), axis=-1) * (1.0 / d)).astype(F32)
    dx = ((g - (xh * c[..., None]).astype(F32)).astype(F32) * r).astype(F32)
    if dres is not None:
        dx = (dx + np.asarray(dres, F32)).astype(F32)
    return dx, dx.astype(F16)


def rms_bwd_float64(dy_total, h, w, eps):
    """The analytic gradient of L = sum(dy_total * w * h * rstd(h)) in float64 (no rounding), the
    form solution/test_kernels.py and dev/test_emu.py:122-133 compare against."""
    hh = np.asarray(h, np.float64)
    d = hh.shape[-1]
    rr = 1.0 / np.sqrt((hh ** 2).mean(-1) + eps)
    xh = hh * rr[..., None]
    g = np.asarray(dy_total, np.float64) * np.asarray(w, np.float64)
    return rr[..., None] * (g - xh * (g * xh).sum(-1, keepdims=True) / d)
