"""decentrik_prime_amd: the NF4 QLoRA linear path of a Qwen2.5 training step on MI355X (gfx950).

Hand-written HIP kernels (``csrc/``, built into ``libdk.so`` with a C ABI declared in
``include/dk.h``) behind Python operators with the reference's call signatures:

  k_nf4      NF4 double-quant layer format and dequant (dequant_tensors / _layer / _range)
  k_mlp      gated SiLU forward / in-place backward
  swiglu     the stock path's out-of-place SwiGLU autograd Function
  w4linear   fused NF4 GEMMs: linear forward with LoRA, dX backward with the LoRA term, LoRA
             gradients, gate|up with the SwiGLU epilogue, down backward with the SwiGLU backward
  quant      GPU NF4 quantiser producing bitsandbytes-shaped weights
  stack      the 28-layer NF4 linear stack of Qwen2.5-1.5B, forward + backward
"""

from . import _lib  # noqa: F401

__all__ = ["k_nf4", "k_mlp", "swiglu", "w4linear", "quant", "stack"]
