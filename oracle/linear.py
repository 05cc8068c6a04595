"""CPU restatement of the projection GEMMs with the LoRA/dropout term.  TEST INFRASTRUCTURE ONLY.

Every GEMM is an fp32 torch-CPU product of fp16-valued operands, rounded to fp16 where the
reference's fp16 ``torch.mm`` rounds (cuBLAS fp16 GEMMs accumulate in fp32 and round once).
The rounding points follow the reference line by line:

forward  (solution/fast_qwen.py:943-947, solution/k_norm.py:49-53, solution/k_rope.py:39-43):
    Xd  = fp16(keep ? fp32(X) * ks : 0)          dropout input of lora_A
    Y16 = fp16(X W^T + bias)                      torch.addmm, one rounding
    Z   = fp16(Xd A^T)                            aq = mm(xq, A^T)
    L   = fp16(Z B^T)                             lq = mm(aq, B^T)
    Y   = fp16(fp32(Y16) + s * fp32(L))           epilogue q32 = q16 + scale * lq16

backward (solution/fast_qwen.py:1364-1377, solution/k_norm.py:65-71):
    dXb = fp16(dY W)                              dy1 = mm(dqkv, W_qkv)
    dB  = fp32(fp16(dY^T Z)) * s                  d_bq = mm(gq^T, aq).float() * s
    dZ  = fp16(fp16(dY B) * s)                    daq = mm(gq, B).mul_(s), an fp16 tensor
    dA  = fp32(fp16(dZ^T Xd))                     d_aq = mm(daq^T, xq).float()
    Lx  = fp16(dZ A)                              lqx = mm(daq, A)
    dX  = fp32(dXb) + (keep ? fp32(Lx) * ks : 0)  the rms backward's dy += mask * ks * lq (fp32)

The input X of this build's boundary is fp16 (the reference drops out the fp32 norm output; the
linear layer on its own only sees fp16 activations), so Xd is formed from fp16 X.
"""

import numpy as np
import torch

F32, F16 = np.float32, np.float16


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(np.asarray(a).astype(F32)))


def mm16(a16, b16):
    """fp16(fp32(a) @ fp32(b)) for fp16-valued operands (a [m,k], b [k,n])."""
    return (_t(a16) @ _t(b16)).numpy().astype(F16)


def mm32(a16, b16):
    return (_t(a16) @ _t(b16)).numpy().astype(F32)


def keep_scale(p):
    """PyTorch's dropout scale 1 / fp32(1 - p) (solution/fast_qwen.py:368-370)."""
    return float(F32(1.0) / F32(1.0 - p))


def dropout_input(x16, mask, ks):
    """fp16(keep ? fp32(x) * ks : 0)  (solution/k_norm.py:49-53)."""
    x = np.asarray(x16, dtype=F16).astype(F32)
    return np.where(np.asarray(mask) != 0, (x * F32(ks)).astype(F32), F32(0)).astype(F16)


def linear_fwd(x16, w16, bias16=None, mask=None, ks=1.0, a16=None, b16=None, s=2.0):
    """Y = X W^T (+ bias) (+ s * (drop(X) A^T) B^T).  Returns (Y fp16, Z fp16 or None)."""
    acc = mm32(x16, np.asarray(w16).T)
    if bias16 is not None:
        acc = (acc + np.asarray(bias16, dtype=F16).astype(F32)[None, :]).astype(F32)
    y16 = acc.astype(F16)
    if a16 is None:
        return y16, None
    xd = dropout_input(x16, mask, ks)
    z = mm16(xd, np.asarray(a16).T)
    lo = mm16(z, np.asarray(b16).T)
    y = (y16.astype(F32) + F32(s) * lo.astype(F32)).astype(F32).astype(F16)
    return y, z


def lora_down(x16, mask, ks, a16):
    """Z = fp16(drop(X) A^T)."""
    return mm16(dropout_input(x16, mask, ks), np.asarray(a16).T)


def linear_bwd(dy16, w16, z16=None, x16=None, mask=None, ks=1.0, a16=None, b16=None, s=2.0):
    """Returns dict(dx fp32, dx_base fp16, and with LoRA: dA fp32 [r,K], dB fp32 [N,r], dZ fp16)."""
    dxb = mm16(dy16, w16)
    out = dict(dx_base=dxb, dx=dxb.astype(F32))
    if a16 is None:
        return out
    dB = (mm16(np.asarray(dy16).T, z16).astype(F32) * F32(s)).astype(F32)
    dZ = (mm16(dy16, b16).astype(F32) * F32(s)).astype(F16)
    xd = dropout_input(x16, mask, ks)
    dA = mm16(dZ.T, xd).astype(F32)
    lx = mm16(dZ, a16)
    term = np.where(np.asarray(mask) != 0, (lx.astype(F32) * F32(ks)).astype(F32), F32(0))
    out.update(dx=(dxb.astype(F32) + term).astype(F32), dA=dA, dB=dB, dZ=dZ, lx=lx)
    return out
