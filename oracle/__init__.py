"""CPU oracle for the fused QLoRA training-step kernels.

TEST INFRASTRUCTURE ONLY. This package restates, on the CPU, the arithmetic of the reference's
Triton kernels (solution/kernels.py) and of the step engine around them (solution/engine.py),
so that the HIP kernels can be checked against it. Only `tests/`, `__graft_entry__.smoke()` and
`bench.py`'s `cpu_baseline` leg may import it, and only as the checker or as the timed CPU
baseline. The product (the `hack-fe30cb28-opus-5-5-ultracode_amd` package and its C-ABI
library) never imports or calls anything here, and has no CPU fallback.

Modules:
  nf4      bitsandbytes-format NF4 double quantisation (input generation) and the bit-exact
           dequantisation of kernels.py:68-105
  philox   Philox4x32-10 (Random123) + rocRAND's init/uniform map, PyTorch's dropout grid and
           counter formula: the LoRA-dropout keep masks of kernels.py:117-126
  ops      RMSNorm fwd/bwd, qkv+RoPE fwd/bwd, SwiGLU fwd/bwd, the three cross-entropy kernels,
           as plain PyTorch on the CPU
  step     one full Qwen2 NF4 + LoRA training step (engine.py:1054-1400) on the CPU

Pinning (what fixes each function independently of its own formula) is listed in each module's
docstring; functions with no independent pin say "parity unpinned".
"""
