"""CPU oracle for the NF4 QLoRA linear path.  TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU (numpy, and torch-CPU for fp32 GEMMs), what the reference
computes on its hot path, so that the HIP kernels of ``decentrik_prime_amd`` can be checked
against it on identical inputs.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker or the timed CPU
baseline; the product path never calls into it and fails loudly when its HIP library is missing.

Modules:
  nf4     NF4 double-quantised format: quantiser (bitsandbytes-style, parity unpinned against
          bitsandbytes itself, which is absent here) and the dequant closed form
          (solution/k_nf4.py:16-21, 40-57).
  linear  projection GEMMs with the LoRA/dropout term, forward and backward
          (solution/fast_qwen.py:943-947, 1366-1383; solution/k_norm.py:49-53, 65-71;
          solution/k_rope.py:39-43, 54-58).
  mlp     gated SiLU forward/backward (solution/k_mlp.py:20-47) and the example SwiGLU
          (solution/swiglu.py:15-37).
"""
