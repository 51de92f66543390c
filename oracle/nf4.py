"""NF4 double quantisation (bitsandbytes format) and bit-exact dequantisation, on the CPU.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Storage format (as the reference reads it from a bitsandbytes QuantState, engine.py:74-101, and
as solution/hostload.py:66-79 sizes it):
  packed   uint8 [numel/2]: element i of the row-major [N, K] weight is the high nibble of byte
           i//2 for even i, the low nibble for odd i (kernels.py:34-35, 103)
  absmax   one scale per block of BS1 = 64 consecutive elements; fp32 without double quant,
           uint8 codes into `code2` with double quant
  code2    fp32 [256], absmax2 fp32 [ceil(blocks/BS2)], BS2 = 256, offset fp32 scalar
Dequantisation (kernels.py:85-105):
  scale_b = fp32( fp32(code2[absmax[b]] * absmax2[b // BS2]) + offset )   (two roundings)
  out_i   = fp16_rne( fp32(level[code_i] * scale_b) )

Pins:
  * dequantize: closed form above, brute force over all 16 codes x 256 absmax codes, the
    special values (code 7 -> +0, codes 0/15 -> -/+scale exactly, absmax 0 -> zeros), and
    fp64 cross-check of every product (tests/test_oracle_nf4.py).
  * NF4_LEVELS: the table held by the reference (kernels.py:38-41), which is also the published
    QLoRA NF4 code (Dettmers et al. 2023) - checked for symmetry/ordering properties in tests.
  * quantize_*: restates bitsandbytes' published quantiser (bitsandbytes 0.50.2,
    functional.quantize_4bit / quantize_blockwise / create_dynamic_map and its CUDA
    dQuantizeNF4 / dQuantize; not vendored in the reference and not installable here): the
    NF4 decision tree on fp32 midpoints, the 8-bit binary search with its midpoint rule. It is
    the checker of the HIP quantiser (csrc/nf4_quant.hip, bit for bit) and generates the other
    tests' inputs (both the HIP kernels and this oracle dequantise the same bytes, so dequant
    parity does not depend on it). Pinned by: the tie rules at every threshold, exact levels
    and code entries mapping to themselves, the nearest-entry property away from midpoints,
    round-trip error bounds (tests/test_oracle_nf4.py). Byte equality with bitsandbytes' own
    output: parity unpinned; the mean of the absmax is defined here as an fp64 sum over a
    binary tree of adjacent pairs (bitsandbytes takes torch's fp32 mean, whose summation order
    is the device library's), so the offset can differ from bitsandbytes' in its last bit.
"""

import numpy as np

# kernels.py:38-41 (bitsandbytes' quant_state.code for quant_type="nf4"), as fp32
NF4_LEVELS = np.array(
    (-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
     -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
     0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
     0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0), dtype=np.float32)


def create_dynamic_map(signed=True, max_exponent_bits=7, total_bits=8):
    """bitsandbytes' dynamic 8-bit code (functional.create_dynamic_map): for each exponent
    level i, the midpoints of a linear grid on [0.1, 1] scaled by 10^(i - (E-1)), both signs,
    plus 0 and 1, sorted. 256 fp32 values. (parity unpinned vs bitsandbytes' bytes)"""
    data = []
    non_sign_bits = total_bits - (1 if signed else 0)
    additional_items = 2 ** (non_sign_bits - max_exponent_bits) - 1
    for i in range(max_exponent_bits):
        fraction_items = int(2 ** (i + non_sign_bits - max_exponent_bits) + 1 if signed
                             else 2 ** (i + non_sign_bits - max_exponent_bits + 1) + 1)
        boundaries = np.linspace(0.1, 1, fraction_items, dtype=np.float32)
        means = (boundaries[:-1] + boundaries[1:]) / np.float32(2.0)
        scale = 10.0 ** (-(max_exponent_bits - 1) + i)
        data += (scale * means.astype(np.float64)).tolist()
        if signed:
            data += (-scale * means.astype(np.float64)).tolist()
    if additional_items > 0:
        boundaries = np.linspace(0.1, 1, additional_items + 1, dtype=np.float32)
        means = (boundaries[:-1] + boundaries[1:]) / np.float32(2.0)
        scale = 10.0 ** (-(max_exponent_bits - 1) + max_exponent_bits - 1)
        data += (scale * means.astype(np.float64)).tolist()
        if signed:
            data += (-scale * means.astype(np.float64)).tolist()
    data.append(0.0)
    data.append(1.0)
    data += [0.0] * (2 ** total_bits - len(data))
    data.sort()
    return np.array(data, dtype=np.float32)


# midpoints of neighbouring NF4 levels rounded to fp32: bitsandbytes' dQuantizeNF4 thresholds
NF4_MIDS = ((NF4_LEVELS[:-1].astype(np.float64) + NF4_LEVELS[1:].astype(np.float64))
            / 2.0).astype(np.float32)


def nf4_codes(x):
    """dQuantizeNF4: the NF4 code of each fp32 x, the number of fp32 midpoints strictly below x
    (its decision tree compares x > threshold at every node; ties go to the lower level)."""
    return np.searchsorted(NF4_MIDS, np.asarray(x, np.float32), side="left").astype(np.uint8)


def dquantize(code, x):
    """bitsandbytes' dQuantize (deterministic) over a sorted 256-entry fp32 code: seven halving
    steps of a binary search from pivot 127, then the nearer of the last pivot and the pivot
    bracketing it on x's side, by an fp32 midpoint (x == midpoint keeps the last pivot)."""
    code = np.asarray(code, np.float32)
    x = np.asarray(x, np.float32)
    pivot = np.full(x.shape, 127, np.int64)
    upper_p = np.full(x.shape, 255, np.int64)
    lower_p = np.zeros(x.shape, np.int64)
    lower = np.full(x.shape, -1.0, np.float32)
    upper = np.full(x.shape, 1.0, np.float32)
    val = code[pivot]
    i = 64
    while i > 0:
        gt = x > val
        lower_p, lower = np.where(gt, pivot, lower_p), np.where(gt, val, lower)
        upper_p, upper = np.where(gt, upper_p, pivot), np.where(gt, upper, val)
        pivot = np.where(gt, pivot + i, pivot - i)
        val = code[pivot]
        i >>= 1
    upper = np.where(upper_p == 255, code[255], upper).astype(np.float32)
    lower = np.where(lower_p == 0, code[0], lower).astype(np.float32)
    mid_u = ((upper + val) * np.float32(0.5)).astype(np.float32)
    mid_l = ((lower + val) * np.float32(0.5)).astype(np.float32)
    out = np.where(x > val, np.where(x > mid_u, upper_p, pivot),
                   np.where(x < mid_l, lower_p, pivot))
    return out.astype(np.uint8)


def tree_sum(values, chunk=1024):
    """fp64 sum over a binary tree of adjacent pairs, the values zero-padded to a power of
    `chunk` (summed `chunk` at a time, level by level)."""
    x = np.asarray(values, np.float64).reshape(-1)
    levels = int(np.log2(chunk))
    while True:
        x = np.concatenate([x, np.zeros((-x.size) % chunk)]).reshape(-1, chunk)
        for _ in range(levels):
            x = x[:, 0::2] + x[:, 1::2]
        x = x.reshape(-1)
        if x.size == 1:
            return x[0]


def quantize_blockwise(a, blocksize=256, code=None):
    """8-bit blockwise quantisation of fp32 values: absmax per block (zero-padded), the code
    index of a * (1 / absmax) by dQuantize. Returns (uint8 codes, fp32 absmax per block, code)."""
    if code is None:
        code = create_dynamic_map(signed=True)
    a = np.asarray(a, dtype=np.float32).reshape(-1)
    n = a.size
    nb = (n + blocksize - 1) // blocksize
    pad = np.zeros(nb * blocksize, dtype=np.float32)
    pad[:n] = a
    blocks = pad.reshape(nb, blocksize)
    absmax = np.abs(blocks).max(axis=1).astype(np.float32)
    inv = np.where(absmax > 0, np.float32(1.0) / np.where(absmax > 0, absmax, 1), 0)
    normed = (blocks * inv.astype(np.float32)[:, None]).astype(np.float32)
    q = dquantize(code, normed.reshape(-1))[:n]
    return q, absmax, code


class QuantState:
    """The fields of a bitsandbytes QuantState that the NF4 path reads (engine.py:77-101)."""

    def __init__(self, absmax, shape, code, blocksize, quant_type="nf4", offset=None,
                 state2=None):
        self.absmax = absmax
        self.shape = tuple(shape)
        self.code = code
        self.blocksize = blocksize
        self.quant_type = quant_type
        self.offset = offset
        self.state2 = state2
        self.nested = state2 is not None


class QuantState2:
    def __init__(self, absmax, code, blocksize):
        self.absmax = absmax
        self.code = code
        self.blocksize = blocksize


def quantize_nf4(w, blocksize=64, compress_statistics=True, blocksize2=256):
    """bitsandbytes-style NF4 quantisation of a [N, K] weight (numpy, any float dtype).

    Per block of `blocksize` consecutive elements: absmax = max |w|; code = nf4_codes of
    w * (1 / absmax) (0 for an all-zero block). With compress_statistics the fp32 absmax are
    double-quantised: offset = fp32(tree_sum(absmax) / count), then 8-bit blockwise
    quantisation of (absmax - offset) in blocks of `blocksize2`. Returns (packed uint8 [numel/2], QuantState with numpy arrays)."""
    w = np.asarray(w)
    shape = w.shape
    flat = w.astype(np.float32).reshape(-1)
    n = flat.size
    if n % blocksize or blocksize % 2:
        raise ValueError("weight size is not a whole number of quantization blocks")
    blocks = flat.reshape(-1, blocksize)
    absmax = np.abs(blocks).max(axis=1).astype(np.float32)
    inv = np.where(absmax > 0, np.float32(1.0) / np.where(absmax > 0, absmax, 1),
                   np.float32(0)).astype(np.float32)
    normed = (blocks * inv[:, None]).astype(np.float32).reshape(-1)
    codes = nf4_codes(normed)
    packed = ((codes[0::2] << 4) | codes[1::2]).astype(np.uint8)
    if compress_statistics:
        offset = np.float32(tree_sum(absmax) / np.float64(absmax.size))
        q, absmax2, code2 = quantize_blockwise(absmax - offset, blocksize=blocksize2)
        state = QuantState(q, shape, NF4_LEVELS.copy(), blocksize, offset=offset,
                           state2=QuantState2(absmax2, code2, blocksize2))
    else:
        state = QuantState(absmax, shape, NF4_LEVELS.copy(), blocksize)
    return packed, state


def block_scales(state, n_blocks=None, seg_offsets=None, seg_bounds=None):
    """Per-block fp32 scale as kernels.py:85-94 forms it. For a group of weights stacked back to
    back (engine.py:118-157), `seg_offsets` holds each weight's offset and `seg_bounds` the first
    block of each weight after the first."""
    if not state.nested:
        return np.asarray(state.absmax, dtype=np.float32)
    q = np.asarray(state.absmax, dtype=np.int64)
    nb = q.size if n_blocks is None else n_blocks
    b = np.arange(nb)
    code2 = np.asarray(state.state2.code, dtype=np.float32)
    absmax2 = np.asarray(state.state2.absmax, dtype=np.float32)
    prod = np.multiply(code2[q], absmax2[b // state.state2.blocksize], dtype=np.float32)
    if seg_offsets is None:
        off = np.float32(state.offset)
        return np.add(prod, off, dtype=np.float32)
    seg = np.zeros(nb, dtype=np.int64)
    for bound in seg_bounds:
        seg += (b >= bound)
    return np.add(prod, np.asarray(seg_offsets, dtype=np.float32)[seg], dtype=np.float32)


def dequantize_nf4(packed, state, levels=None, scales=None):
    """Bit-exact fp16 dequantisation (kernels.py:68-105). Returns float16 [N, K]."""
    packed = np.asarray(packed, dtype=np.uint8).reshape(-1)
    levels = NF4_LEVELS if levels is None else np.asarray(levels, dtype=np.float32)
    bs = state.blocksize
    if scales is None:
        scales = block_scales(state)
    codes = np.empty(packed.size * 2, dtype=np.uint8)
    codes[0::2] = packed >> 4
    codes[1::2] = packed & 15
    vals = levels[codes].reshape(-1, bs)
    out = np.multiply(vals, scales[:, None].astype(np.float32), dtype=np.float32)
    return out.astype(np.float16).reshape(state.shape)
