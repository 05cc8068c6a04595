"""Out-of-place SwiGLU, silu(gate) * up, with its autograd Function and the Qwen2MLP patch.

Counterpart of the reference's example solution/swiglu.py (the stock, non-fused path):
forward ``out = gate * sigmoid(gate) * up``, backward ``dup = grad * gate * sig``,
``dgate = grad * up * sig * (1 + gate * (1 - sig))``, fp32 math, in the gfx950 kernels
``dk_swiglu_fwd/bwd``.  fp16 operands only.
"""

import torch

from . import _lib


def _launch(name, *tensors, n):
    rc = getattr(_lib.lib(), name)(*[_lib.ptr(t) for t in tensors], n,
                                   _lib.stream_handle(tensors[0].device))
    _lib.check(rc, name)


class SwiGLU(torch.autograd.Function):
    """silu(gate) * up in one launch each way."""

    @staticmethod
    def forward(ctx, gate, up):
        if gate.dtype != torch.float16 or not gate.is_cuda:
            raise ValueError("SwiGLU expects CUDA fp16 inputs")
        gate = gate.contiguous()
        up = up.to(gate.dtype).contiguous()
        out = torch.empty_like(gate)
        _launch("dk_swiglu_fwd", gate, up, out, n=gate.numel())
        ctx.save_for_backward(gate, up)
        return out

    @staticmethod
    def backward(ctx, grad):
        gate, up = ctx.saved_tensors
        grad = grad.to(gate.dtype).contiguous()
        dgate, dup = torch.empty_like(gate), torch.empty_like(up)
        _launch("dk_swiglu_bwd", grad, gate, up, dgate, dup, n=gate.numel())
        return dgate, dup


def swiglu(gate, up):
    return SwiGLU.apply(gate, up)


def patch_qwen2_mlp():
    """Send Qwen2MLP.forward through the SwiGLU kernels for CUDA fp16 inputs."""
    from transformers.models.qwen2 import modeling_qwen2

    original = modeling_qwen2.Qwen2MLP.forward

    def forward(self, x):
        act = getattr(getattr(self, "config", None), "hidden_act", "silu")
        if act != "silu" or not x.is_cuda or x.dtype != torch.float16:
            return original(self, x)
        return self.down_proj(swiglu(self.gate_proj(x), self.up_proj(x)))

    modeling_qwen2.Qwen2MLP.forward = forward
