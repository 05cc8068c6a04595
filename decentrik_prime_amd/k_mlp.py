"""Gated SiLU of the Qwen2 MLP on the fused gate|up output, forward and in-place backward.

Drop-in for the reference's solution/k_mlp.py (same function names and arguments), running the
gfx950 kernels ``dk_gated_silu_fwd/bwd`` of libdk.so.  gu = [gate | up] is one fp16 row of
2 * I per token:
    act    = fp16(silu(gate) * up)                                   fp32 math
    d up   = dact * silu(gate)
    d gate = dact * up * sig * (1 + gate * (1 - sig))                written in place into gu
The fused forward (gate|up GEMM + this epilogue) and the fused backward (down^T GEMM + this
backward) are ``w4linear.gateup_swiglu_forward`` / ``down_swiglu_backward``.
"""

import torch

from . import _lib


def _check(gu, other, name):
    if gu.dtype != torch.float16 or other.dtype != torch.float16 or not gu.is_cuda:
        raise ValueError("gated SiLU operands must be CUDA fp16 tensors")
    if not gu.is_contiguous() or not other.is_contiguous():
        raise ValueError("gated SiLU operands must be contiguous")
    n, two_i = gu.shape
    if two_i % 2 or tuple(other.shape) != (n, two_i // 2):
        raise ValueError(f"{name} must be [n, inter] for gu [n, 2 * inter]")
    return n, two_i // 2


def gated_silu_forward(gu, act):
    n, inter = _check(gu, act, "act")
    rc = _lib.lib().dk_gated_silu_fwd(_lib.ptr(gu), _lib.ptr(act), n, inter,
                                      _lib.stream_handle(gu.device))
    _lib.check(rc, "dk_gated_silu_fwd")
    return act


def gated_silu_backward(gu, dact):
    n, inter = _check(gu, dact, "dact")
    rc = _lib.lib().dk_gated_silu_bwd(_lib.ptr(gu), _lib.ptr(dact), n, inter,
                                      _lib.stream_handle(gu.device))
    _lib.check(rc, "dk_gated_silu_bwd")
    return gu


def warmup_specs(inter):
    """Nothing to warm up: the kernels are compiled ahead of time into libdk.so."""
    return []
