"""MI355X-native (gfx950) fused QLoRA training-step kernels for a Qwen2 NF4 + LoRA step.

A drop-in for the kernel layer of the reference's fused step (solution/kernels.py, called
through solution/engine.py's op wrappers): the same Python call signatures, each launching a
hand-written HIP kernel of libqlora_amd.so (C-ABI: include/qlora_amd.h) on torch's current HIP
stream. There is no Triton and no CPU fallback: without the built library every op raises.

  engine   the training step: Packed, _Layer, _Head, FusedQwen2, random_qwen2
  linear   the step's GEMMs (NF4 projections forward/backward, lm_head) on the package's MFMA
           GEMM
  head     the LM head over vocabulary pieces with the hidden and embedding gradients
  trainer  the HF / TRL Trainer drop-in: compute_loss replaced by the fused step (install)
  ops      the engine's op wrappers (_rms_fwd, _rms_bwd, _rope_fwd, _rope_bwd, _glu_fwd,
           _glu_bwd, _attn_fwd, _attn_bwd, _ce, _ce_piece, _ce_finish, _ce_grad, dequant,
           dequant_many, NF4Weight, NF4Group, TorchDropout)
  quant    bitsandbytes-format NF4 double quantisation on the GPU (builds the frozen weights)
  _lib     the ctypes binding of the C-ABI
  build    hipcc build of the library
"""

from . import _lib, ops, quant, linear, engine, head, profiling, trainer  # noqa: F401
from .ops import (NF4Group, NF4Weight, TorchDropout, _attn_bwd, _attn_fwd, _ce,  # noqa: F401
                  _ce_finish, _ce_grad, _ce_piece, _glu_bwd, _glu_fwd, _rms_bwd, _rms_fwd,
                  _rope_bwd, _rope_fwd, dequant, dequant_many)
