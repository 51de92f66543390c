"""bitsandbytes-format NF4 double quantisation with torch ops (on any device).

Builds the frozen weights of the step in the exact in-memory format the path reads from a
bitsandbytes Params4bit (engine.py:77-101; hostload.py:66-79): packed uint8 [numel/2, 1] (element
i = high nibble of byte i/2 for even i), absmax uint8 codes per 64-value block, state2.absmax fp32
per 256 blocks, state2.code fp32 [256] (bitsandbytes' signed dynamic map), offset fp32 = mean of
the block absmax. The quantiser restates bitsandbytes 0.50.2's published algorithm
(functional.quantize_4bit with compress_statistics=True); bitsandbytes itself is not installable
here, so byte equality with its output is not claimed.
"""

import numpy as np
import torch

from .ops import NF4_LEVELS


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


def _nearest(x, code):
    """Index of the nearest entry of the sorted code (ties to the lower entry)."""
    mids = (code[:-1].double() + code[1:].double()) / 2.0
    return torch.bucketize(x.double(), mids.to(x.device), right=False)


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


@torch.no_grad()
def quantize_nf4(w, blocksize=64, compress_statistics=True, blocksize2=256):
    """NF4-quantise a [N, K] weight; returns a Params4bit-like holder on w's device."""
    dev = w.device
    shape = w.shape
    flat = w.reshape(-1).float()
    if flat.numel() % blocksize:
        raise ValueError("weight size is not a whole number of quantization blocks")
    blocks = flat.view(-1, blocksize)
    absmax = blocks.abs().amax(dim=1)
    inv = torch.where(absmax > 0, 1.0 / torch.where(absmax > 0, absmax, torch.ones_like(absmax)),
                      torch.zeros_like(absmax))
    normed = (blocks * inv[:, None]).reshape(-1)
    levels = torch.tensor(NF4_LEVELS, dtype=torch.float32, device=dev)
    codes = _nearest(normed, levels).to(torch.uint8)
    packed = ((codes[0::2] << 4) | codes[1::2]).contiguous().view(-1, 1)
    if not compress_statistics:
        state = QuantState(absmax.contiguous(), shape, levels, blocksize, w.dtype)
        return Params4bit(packed, state)
    offset = absmax.double().mean().float()
    centred = absmax - offset
    nb2 = (centred.numel() + blocksize2 - 1) // blocksize2
    pad = torch.zeros(nb2 * blocksize2, dtype=torch.float32, device=dev)
    pad[:centred.numel()] = centred
    absmax2 = pad.view(nb2, blocksize2).abs().amax(dim=1)
    inv2 = torch.where(absmax2 > 0,
                       1.0 / torch.where(absmax2 > 0, absmax2, torch.ones_like(absmax2)),
                       torch.zeros_like(absmax2))
    code2 = _dynamic_map().to(dev)
    q = _nearest((pad.view(nb2, blocksize2) * inv2[:, None]).reshape(-1), code2)
    q = q[:centred.numel()].to(torch.uint8).contiguous()
    state2 = QuantState2(absmax2.contiguous(), code2, blocksize2)
    state = QuantState(q, shape, levels, blocksize, w.dtype, offset=offset.reshape(()),
                       state2=state2)
    return Params4bit(packed, state)
