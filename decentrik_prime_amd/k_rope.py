"""QKV epilogue: LoRA add + rotary embedding, in place on the fused [N, (nq + 2 nkv) hd] QKV
buffer, and its backward.

Drop-in for the reference's solution/k_rope.py (same function names and arguments), running the
gfx950 kernels ``dk_qkv_epilogue_fwd`` / ``dk_qkv_epilogue_bwd`` of libdk.so, one token row per
wave, every product and sum rounded to fp32 on its own:

forward   q = f32(q16) + scale f32(lq16), k = f32(k16), v = f32(v16) + scale f32(lv16)
          q/k <- [x1 c - x2 s | x2 c + x1 s]  (c, s = cos/sin[pos, :hd/2]); stored fp16
backward  dk/dv rows hold gin partials per KV head (gin = nq/nkv for per-query-head partials,
          1 for grads already reduced), summed in order; [d1 c + d2 s | d2 c - d1 s]; fp16 out
"""

import torch

from . import _lib


def _t(t, dtypes, what, shape=None):
    if t.dtype not in dtypes or not t.is_cuda or not t.is_contiguous():
        raise ValueError(f"{what} must be a contiguous CUDA tensor of {dtypes}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{what} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    return t


def _tables(pos, cos, sin, n, hd):
    _t(pos, (torch.int32,), "pos", (n,))
    _t(cos, (torch.float32,), "cos")
    _t(sin, (torch.float32,), "sin", tuple(cos.shape))
    if cos.dim() != 2 or cos.shape[1] != hd:
        raise ValueError(f"cos/sin must be [positions, {hd}]")


def qkv_epilogue_forward(qkv, lq, lv, pos, cos, sin, lora_scale, nq, nkv, hd):
    n = qkv.shape[0]
    _t(qkv, (torch.float16,), "qkv", (n, (nq + 2 * nkv) * hd))
    _t(lq, (torch.float16,), "lq", (n, nq * hd))
    _t(lv, (torch.float16,), "lv", (n, nkv * hd))
    _tables(pos, cos, sin, n, hd)
    rc = _lib.lib().dk_qkv_epilogue_fwd(_lib.ptr(qkv), _lib.ptr(lq), _lib.ptr(lv), _lib.ptr(pos),
                                        _lib.ptr(cos), _lib.ptr(sin), n, float(lora_scale), nq,
                                        nkv, hd, _lib.stream_handle(qkv.device))
    _lib.check(rc, "dk_qkv_epilogue_fwd")


def qkv_epilogue_backward(dq, dk, dv, pos, cos, sin, out, nq, nkv, hd, gin):
    n = out.shape[0]
    _t(out, (torch.float16,), "out", (n, (nq + 2 * nkv) * hd))
    grads = (torch.float32, torch.float16)
    _t(dq, grads, "dq", (n, nq * hd))
    _t(dk, (dq.dtype,), "dk", (n, nkv * gin * hd))
    _t(dv, (dq.dtype,), "dv", (n, nkv * gin * hd))
    _tables(pos, cos, sin, n, hd)
    rc = _lib.lib().dk_qkv_epilogue_bwd(_lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv),
                                        int(dq.dtype == torch.float32), _lib.ptr(pos),
                                        _lib.ptr(cos), _lib.ptr(sin), _lib.ptr(out), n, nq, nkv,
                                        hd, gin, _lib.stream_handle(out.device))
    _lib.check(rc, "dk_qkv_epilogue_bwd")


def warmup_specs(nq, nkv, hd, gin, grad_dtype):
    """Nothing to warm up: the kernels are compiled ahead of time into libdk.so."""
    return []
