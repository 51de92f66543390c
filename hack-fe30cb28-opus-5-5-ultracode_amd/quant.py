"""bitsandbytes-format NF4 double quantisation on the GPU (csrc/nf4_quant.hip).

Builds the frozen weights of the step in the exact in-memory format the path reads from a
bitsandbytes Params4bit (engine.py:77-101; hostload.py:66-79): packed uint8 [numel/2, 1] (element
i = high nibble of byte i/2 for even i), absmax uint8 codes per 64-value block, state2.absmax fp32
per 256 blocks, state2.code fp32 [256] (bitsandbytes' signed dynamic map), offset fp32 = the mean
of the block absmax. The kernels restate bitsandbytes 0.50.2's published quantiser
(functional.quantize_4bit with compress_statistics=True: the NF4 decision tree on fp32
midpoints, the 8-bit binary search); bitsandbytes itself is not installable here, so byte
equality with its output is not claimed (the mean is summed in fp64 over a fixed tree, where
bitsandbytes takes torch's fp32 mean).
"""

import ctypes

import numpy as np
import torch

from . import _lib
from .ops import NF4_LEVELS, _ptr, _stream


def _dynamic_map():
    """bitsandbytes' signed dynamic 8-bit code (create_dynamic_map(signed=True)): 256 sorted
    fp32 values."""
    data = []
    for i in range(7):
        items = 2 ** i + 1
        bounds = np.linspace(0.1, 1, items, dtype=np.float32)
        means = (bounds[:-1] + bounds[1:]) / np.float32(2.0)
        scale = 10.0 ** (-6 + i)
        data += (scale * means.astype(np.float64)).tolist()
        data += (-scale * means.astype(np.float64)).tolist()
    data += [0.0, 1.0]
    data.sort()
    assert len(data) == 256
    return torch.tensor(data, dtype=torch.float32)


class QuantState2:
    def __init__(self, absmax, code, blocksize):
        self.absmax, self.code, self.blocksize = absmax, code, blocksize


class QuantState:
    """The QuantState fields the path reads."""

    def __init__(self, absmax, shape, code, blocksize, dtype, offset=None, state2=None):
        self.absmax = absmax
        self.shape = torch.Size(shape)
        self.code = code
        self.blocksize = blocksize
        self.quant_type = "nf4"
        self.dtype = dtype
        self.offset = offset
        self.state2 = state2
        self.nested = state2 is not None


class Params4bit:
    """Holder with a Params4bit's `.data` (packed bytes) and `.quant_state`."""

    def __init__(self, data, quant_state):
        self.data = data
        self.quant_state = quant_state


_TABLES = {}  # device -> (NF4 levels, dynamic map), copied to the device once


def _tables(dev):
    t = _TABLES.get(dev)
    if t is None:
        t = _TABLES[dev] = (torch.tensor(NF4_LEVELS, dtype=torch.float32, device=dev),
                            _dynamic_map().to(dev))
    return t


@torch.no_grad()
def quantize_nf4(w, blocksize=64, compress_statistics=True, blocksize2=256):
    """NF4-quantise a [N, K] fp16 / fp32 / bf16 weight on its GPU (bf16 is widened to fp32
    first); returns a Params4bit-like holder on w's device."""
    if blocksize != 64 or blocksize2 != 256:
        raise ValueError("the GPU quantiser takes blocksize 64 and blocksize2 256 "
                         "(bitsandbytes' defaults for NF4)")
    dev = w.device
    if dev.type != "cuda":
        raise ValueError("quantize_nf4 runs on the GPU: w must be a device tensor")
    shape = w.shape
    flat = w.reshape(-1)
    if flat.dtype not in (torch.float16, torch.float32):
        flat = flat.float()
    flat = flat.contiguous()
    if flat.numel() % blocksize:
        raise ValueError("weight size is not a whole number of quantization blocks")
    n_blocks = flat.numel() // blocksize
    packed = torch.empty((flat.numel() // 2,), device=dev, dtype=torch.uint8)
    absmax = torch.empty((n_blocks,), device=dev, dtype=torch.float32)
    levels, code2 = _tables(dev)
    _lib.call("qlora_nf4_quantize", _ptr(flat), int(flat.dtype == torch.float32), n_blocks,
              _ptr(packed), _ptr(absmax), _stream(dev))
    packed = packed.view(-1, 1)
    if not compress_statistics:
        return Params4bit(packed, QuantState(absmax, shape, levels, blocksize, w.dtype))
    elems = ctypes.c_int64(0)
    _lib.call("qlora_nf4_quantize_stats_workspace", n_blocks, ctypes.byref(elems))
    work = torch.empty((elems.value,), device=dev, dtype=torch.float64)
    q = torch.empty((n_blocks,), device=dev, dtype=torch.uint8)
    absmax2 = torch.empty(((n_blocks + blocksize2 - 1) // blocksize2,), device=dev,
                          dtype=torch.float32)
    offset = torch.empty((), device=dev, dtype=torch.float32)
    _lib.call("qlora_nf4_quantize_stats", _ptr(absmax), n_blocks, _ptr(code2), _ptr(work),
              work.numel(), _ptr(q), _ptr(absmax2), _ptr(offset), _stream(dev))
    state2 = QuantState2(absmax2, code2, blocksize2)
    state = QuantState(q, shape, levels, blocksize, w.dtype, offset=offset, state2=state2)
    return Params4bit(packed, state)
