"""Fused residual add + RMSNorm with the two LoRA dropout inputs, forward and backward.

Drop-in for the reference's solution/k_norm.py (same function names and arguments), running the
gfx950 kernels ``dk_rms_fwd`` / ``dk_rms_bwd`` of libdk.so, one token row per wave:

forward   h = x (fp32) [+ delta (fp16 GEMM output)]              written to xout if given
          rstd = rsqrt(mean(h^2) + eps);  y = w * (h * rstd)          Qwen2RMSNorm in fp32
          y16 = fp16(y);  xq16 = fp16(dropout_q(y)), xv16 = fp16(dropout_v(y))
backward  dy = fp16 grad * gscale + [mask_q] keep_scale lq16 + [mask_v] keep_scale lv16
          dx = rstd (w dy - xhat mean(w dy xhat)),  out = dres + dx   (out may alias dres)

The keep-masks are inputs (uint8 or bool [n, d], nonzero = keep), as in the reference (v15).
``dummy16`` / ``dummy32`` are accepted for signature compatibility and unused: an output that is
not wanted is passed as NULL to the kernel.
"""

import torch

from . import _lib


def _mask(m, shape, what):
    if m is None:
        return None
    if m.dtype == torch.bool:
        m = m.view(torch.uint8)
    if m.dtype != torch.uint8 or tuple(m.shape) != tuple(shape) or not m.is_contiguous():
        raise ValueError(f"{what} must be a contiguous uint8 [n, d] keep-mask")
    return m


def _t(t, dtype, shape, what):
    if t is None:
        return None
    if t.dtype != dtype or not t.is_cuda or not t.is_contiguous() or tuple(t.shape) != tuple(shape):
        raise ValueError(f"{what} must be a contiguous CUDA {dtype} tensor of shape {tuple(shape)}")
    return t


def rms_forward(x, w, y, rstd, eps, *, delta=None, xout=None, xq=None, xv=None, mq=None, mv=None,
                keep_scale=1.0, dummy16=None, dummy32=None):
    """y=None: rstd and the dropout-masked LoRA inputs only (the backward's norm recompute when
    the attention activations were kept).  xq/xv need the uint8 keep-masks mq/mv."""
    if x.dim() != 2:
        raise ValueError("x must be [n, d]")
    n, d = x.shape
    dropout = xq is not None or xv is not None
    if dropout and (xq is None or xv is None or mq is None or mv is None):
        raise ValueError("the LoRA dropout outputs need their keep-masks")
    _t(x, torch.float32, (n, d), "x")
    _t(w, torch.float32, (d,), "w")
    _t(rstd, torch.float32, (n,), "rstd")
    for t, dt, nm in ((y, torch.float16, "y"), (delta, torch.float16, "delta"),
                      (xout, torch.float32, "xout"), (xq, torch.float16, "xq"),
                      (xv, torch.float16, "xv")):
        _t(t, dt, (n, d), nm)
    mq = _mask(mq, (n, d), "mq") if dropout else None
    mv = _mask(mv, (n, d), "mv") if dropout else None
    rc = _lib.lib().dk_rms_fwd(_lib.ptr(x), _lib.ptr(delta), _lib.ptr(xout), _lib.ptr(w),
                               _lib.ptr(y), _lib.ptr(rstd), _lib.ptr(xq), _lib.ptr(xv),
                               _lib.ptr(mq), _lib.ptr(mv), n, d, float(eps), float(keep_scale),
                               _lib.stream_handle(x.device))
    _lib.check(rc, "dk_rms_fwd")


def rms_backward(dy16, gscale, x, w, rstd, out, *, dres=None, lq=None, lv=None, mq=None, mv=None,
                 keep_scale=1.0, out16=None, delta=None, dummy16=None, dummy32=None):
    """delta: the norm's input is x + delta (fp16), added in registers as in the forward, so the
    backward needs no recomputed copy of it.  lq/lv (LoRA-A input grads) need the keep-masks.
    gscale: a CUDA fp32 tensor whose first element scales dy16.  dy16 may also be fp32 (the fused
    q|k|v dX GEMM's output, which already holds the masked LoRA input gradients)."""
    if x.dim() != 2:
        raise ValueError("x must be [n, d]")
    n, d = x.shape
    use_lora = lq is not None or lv is not None
    if use_lora and (lq is None or lv is None or mq is None or mv is None):
        raise ValueError("the LoRA input gradients need their keep-masks")
    _t(x, torch.float32, (n, d), "x")
    _t(w, torch.float32, (d,), "w")
    _t(rstd, torch.float32, (n,), "rstd")
    _t(out, torch.float32, (n, d), "out")
    if gscale.dtype != torch.float32 or not gscale.is_cuda or gscale.numel() < 1:
        raise ValueError("gscale must be a CUDA fp32 tensor")
    dy32 = dy16.dtype == torch.float32
    for t, dt, nm in ((dy16, dy16.dtype if dy32 else torch.float16, "dy16"),
                      (delta, torch.float16, "delta"),
                      (dres, torch.float32, "dres"), (lq, torch.float16, "lq"),
                      (lv, torch.float16, "lv"), (out16, torch.float16, "out16")):
        _t(t, dt, (n, d), nm)
    mq = _mask(mq, (n, d), "mq") if use_lora else None
    mv = _mask(mv, (n, d), "mv") if use_lora else None
    rc = _lib.lib().dk_rms_bwd(_lib.ptr(dy16), int(dy32), _lib.ptr(gscale), _lib.ptr(x),
                               _lib.ptr(delta),
                               _lib.ptr(w), _lib.ptr(rstd), _lib.ptr(dres), _lib.ptr(out),
                               _lib.ptr(lq), _lib.ptr(lv), _lib.ptr(out16), _lib.ptr(mq),
                               _lib.ptr(mv), n, d, float(keep_scale), _lib.stream_handle(x.device))
    _lib.check(rc, "dk_rms_bwd")


def warmup_specs(hidden):
    """Nothing to warm up: the kernels are compiled ahead of time into libdk.so."""
    return []
