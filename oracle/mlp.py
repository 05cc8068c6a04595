"""CPU restatement of the gated SiLU (SwiGLU) of the Qwen2 MLP.  TEST INFRASTRUCTURE ONLY.

gu = [gate | up] is one fp16 row of 2*I per token (the fused gate|up GEMM output).
forward  (solution/k_mlp.py:20-29):  act = fp16(g / (1 + exp(-g)) * u), fp32 math
backward (solution/k_mlp.py:32-47):  e = 1 + exp(-g), sig = 1/e, silu = g/e
                                      d up   = da * silu
                                      d gate = (da * u) * sig * (1 + g * (1 - sig))
                                      written in place into gu as [d gate | d up] (fp16)
Example SwiGLU (solution/swiglu.py:15-37): out = gate * sigmoid(gate) * up, and its backward
dup = grad * gate * sig, dgate = grad * up * sig * (1 + gate * (1 - sig)).
"""

import numpy as np

from . import linear

F32, F16 = np.float32, np.float16


def _split(gu16):
    gu = np.asarray(gu16, dtype=F16)
    inter = gu.shape[-1] // 2
    return gu[..., :inter].astype(F32), gu[..., inter:].astype(F32)


def gated_silu_fwd(gu16):
    g, u = _split(gu16)
    silu = (g / (F32(1) + np.exp(-g))).astype(F32)
    return (silu * u).astype(F32).astype(F16)


def gated_silu_bwd(gu16, dact16):
    """Returns the new gu buffer [d gate | d up] (fp16)."""
    g, u = _split(gu16)
    da = np.asarray(dact16, dtype=F16).astype(F32)
    e = (F32(1) + np.exp(-g)).astype(F32)
    sig = (F32(1) / e).astype(F32)
    silu = (g / e).astype(F32)
    d_up = (da * silu).astype(F32)
    d_gate = ((da * u) * sig * (F32(1) + g * (F32(1) - sig))).astype(F32)
    return np.concatenate([d_gate.astype(F16), d_up.astype(F16)], axis=-1)


def swiglu_fwd(gate16, up16):
    g = np.asarray(gate16, dtype=F16).astype(F32)
    u = np.asarray(up16, dtype=F16).astype(F32)
    sig = (F32(1) / (F32(1) + np.exp(-g))).astype(F32)
    return (g * sig * u).astype(F32).astype(F16)


def swiglu_bwd(grad16, gate16, up16):
    gr = np.asarray(grad16, dtype=F16).astype(F32)
    g = np.asarray(gate16, dtype=F16).astype(F32)
    u = np.asarray(up16, dtype=F16).astype(F32)
    sig = (F32(1) / (F32(1) + np.exp(-g))).astype(F32)
    dup = (gr * g * sig).astype(F32)
    dgate = (gr * u * sig * (F32(1) + g * (F32(1) - sig))).astype(F32)
    return dgate.astype(F16), dup.astype(F16)


def mlp_fwd(x16, wgu16, wd16):
    """gu = fp16(X Wgu^T) [M, 2I]; H = gated_silu(gu); Y = fp16(H Wd^T).  Returns (gu, H, Y)."""
    gu = linear.mm16(x16, np.asarray(wgu16).T)
    h = gated_silu_fwd(gu)
    y = linear.mm16(h, np.asarray(wd16).T)
    return gu, h, y


def mlp_bwd(dy16, gu16, wgu16, wd16):
    """dact = fp16(dY Wd); gu <- [dgate|dup]; dX = fp16(dgu Wgu).  Returns (dgu, dX fp16)."""
    dact = linear.mm16(dy16, wd16)
    dgu = gated_silu_bwd(gu16, dact)
    dx = linear.mm16(dgu, wgu16)
    return dgu, dx
