"""Pins of the NF4 oracle (oracle/nf4.py) that do not restate its own formula."""

import struct

import numpy as np
import pytest
from scipy.stats import norm

from oracle import nf4 as N


def test_levels_are_the_normal_float4_code():
    """NF4 (QLoRA, Dettmers et al. 2023): 8 positive levels from the normal quantiles of
    linspace(0.9677083, 0.5, 9)[:-1], 7 negative from linspace(0.9677083, 0.5, 8)[:-1], plus 0,
    normalised by the largest. The reference's table (kernels.py:38-41) must be that code."""
    off = 0.9677083
    pos = norm.ppf(np.linspace(off, 0.5, 9)[:-1])
    neg = -norm.ppf(np.linspace(off, 0.5, 8)[:-1])
    vals = np.sort(np.concatenate([pos, neg, [0.0]]))
    vals = vals / vals.max()
    assert len(vals) == 16
    np.testing.assert_allclose(N.NF4_LEVELS.astype(np.float64), vals, rtol=0, atol=3e-7)
    assert N.NF4_LEVELS[7] == 0.0 and N.NF4_LEVELS[0] == -1.0 and N.NF4_LEVELS[15] == 1.0
    assert np.all(np.diff(N.NF4_LEVELS) > 0)


def _f32(x):
    return struct.unpack("f", struct.pack("f", x))[0]


def _f16(x):
    return float(np.float16(np.float32(x)))


def _state(absmax_q, absmax2, offset, code2, n_blocks):
    return N.QuantState(absmax_q, (n_blocks, 64), N.NF4_LEVELS, 64, offset=np.float32(offset),
                        state2=N.QuantState2(absmax2, code2, 256))


def test_dequant_every_code_and_absmax_code_fp64_stepwise():
    """All 16 NF4 codes x all 256 absmax codes: each output equals the value built one IEEE
    rounding at a time in fp64 (exact product, then round to fp32; exact sum, round to fp32;
    exact product, round to fp32, then to fp16) - no fused multiply-add anywhere."""
    rng = np.random.default_rng(1)
    code2 = N.create_dynamic_map()
    n_blocks = 256
    absmax_q = np.arange(256, dtype=np.uint8)
    absmax2 = np.array([0.0173], dtype=np.float32)
    offset = np.float32(0.0412)
    codes = np.tile(np.arange(16, dtype=np.uint8), n_blocks * 4)
    rng.shuffle(codes)
    packed = (codes[0::2] << 4) | codes[1::2]
    out = N.dequantize_nf4(packed, _state(absmax_q, absmax2, offset, code2, n_blocks))
    out = out.reshape(-1)
    for b in range(n_blocks):
        scale = _f32(_f32(float(code2[b]) * float(absmax2[0])) + float(offset))
        for j in range(64):
            i = b * 64 + j
            want = _f16(_f32(float(N.NF4_LEVELS[codes[i]]) * scale))
            got = float(out[i])
            assert got == want or (np.isnan(got) and np.isnan(want)), (b, j, got, want)


def test_dequant_special_values_and_nibble_order():
    code2 = N.create_dynamic_map()
    absmax2 = np.array([0.5, 0.25], dtype=np.float32)
    q = np.array([255, 200, 17, 255, 0, 128, 255, 255] * 40, dtype=np.uint8)[:300]
    st = _state(q, absmax2, 0.1, code2, 300)
    scales = N.block_scales(st)
    # element 2k is the HIGH nibble of byte k: codes (15, 0) in byte 0xF0 -> (+scale, -scale)
    packed = np.zeros(300 * 32, dtype=np.uint8)
    packed[0::32] = 0xF0
    packed[1::32] = 0x77  # code 7 twice -> zeros
    out = N.dequantize_nf4(packed, st).reshape(300, 64)
    np.testing.assert_array_equal(out[:, 0], scales.astype(np.float16))
    np.testing.assert_array_equal(out[:, 1], (-scales).astype(np.float16))
    assert np.all(out[:, 2:4] == 0)
    # codes 0 elsewhere -> -scale
    np.testing.assert_array_equal(out[:, 5], (-scales).astype(np.float16))
    # plain (not double-quantised) fp32 absmax, absmax 0 -> zeros
    plain = N.QuantState(np.zeros(4, np.float32), (4, 64), N.NF4_LEVELS, 64)
    assert np.all(N.dequantize_nf4(np.full(128, 0xAB, np.uint8), plain) == 0)


@pytest.mark.parametrize("shape", [(256, 1536), (1536, 512), (64, 64)])
@pytest.mark.parametrize("nested", [True, False])
def test_quantize_round_trip_error(shape, nested):
    """Dequantised value within half the widest NF4 gap of the block scale, plus the 8-bit
    double-quantisation error of the scale itself."""
    rng = np.random.default_rng(0)
    w = (rng.standard_normal(shape) * 0.05).astype(np.float16)
    packed, st = N.quantize_nf4(w, compress_statistics=nested)
    assert packed.size * 2 == w.size
    out = N.dequantize_nf4(packed, st).astype(np.float64)
    blocks = np.abs(w.astype(np.float64)).reshape(-1, 64).max(1)
    gap = np.max(np.diff(N.NF4_LEVELS.astype(np.float64))) / 2
    scales = N.block_scales(st).astype(np.float64)
    # scale error of the double quantisation: at most half a step of the dynamic code at
    # its coarsest (0.1 relative) times the block's absmax2
    serr = np.abs(scales - blocks)
    if nested:
        a2 = np.repeat(st.state2.absmax.astype(np.float64), 256)[:blocks.size]
        assert np.all(serr <= 0.06 * a2 + 1e-7)
    else:
        assert np.all(serr == 0)
    err = np.abs(out.reshape(-1, 64) - w.astype(np.float64).reshape(-1, 64))
    bound = gap * np.maximum(blocks, scales) + serr + 1e-3 * blocks + 1e-7
    assert np.all(err <= bound[:, None])


def test_dynamic_map_shape():
    code = N.create_dynamic_map()
    assert code.shape == (256,) and code.dtype == np.float32
    assert np.all(np.diff(code) >= 0)
    assert code[-1] == 1.0 and 0.0 in code
    assert np.sum(code > 0) == 128 and np.sum(code < 0) == 127


def test_nf4_tree_thresholds_and_ties():
    """dQuantizeNF4's thresholds are the fp32 midpoints of neighbouring levels (the published
    tree's root and right-spine constants), a midpoint itself goes to the lower level, the next
    float above it to the upper; every level maps to its own code."""
    mids = N.NF4_MIDS
    assert mids.dtype == np.float32 and np.all(np.diff(mids) > 0)
    for i, c in ((7, 0.03979014977812767), (11, 0.3893125355243683), (13, 0.6427869200706482),
                 (14, 0.8614784181118011)):
        assert mids[i] == np.float32(c)
    for i, m in enumerate(mids):
        assert N.nf4_codes(m) == i
        assert N.nf4_codes(np.nextafter(m, np.float32(np.inf))) == i + 1
    assert np.array_equal(N.nf4_codes(N.NF4_LEVELS), np.arange(16))
    assert N.nf4_codes(np.float32(-2.0)) == 0 and N.nf4_codes(np.float32(2.0)) == 15


def test_dquantize_binary_search():
    """Every entry of the dynamic map maps to its own index; away from the midpoints the result
    is the nearest entry (brute force); at a midpoint it is one of its two entries."""
    code = N.create_dynamic_map()
    assert np.array_equal(N.dquantize(code, code), np.arange(256))
    rng = np.random.default_rng(3)
    x = rng.uniform(-1.0, 1.0, 200000).astype(np.float32)
    x = np.concatenate([x, (rng.standard_normal(50000) * 1e-3).astype(np.float32)])
    mids = (code[:-1].astype(np.float64) + code[1:].astype(np.float64)) / 2
    gaps = np.diff(code.astype(np.float64))
    near = np.abs(x.astype(np.float64)[:, None] - mids[None, :]) < 1e-3 * gaps[None, :]
    keep = ~near.any(axis=1)
    want = np.abs(x[keep, None].astype(np.float64) - code[None, :].astype(np.float64)).argmin(1)
    assert np.array_equal(N.dquantize(code, x[keep]), want)
    m32 = ((code[:-1] + code[1:]) * np.float32(0.5)).astype(np.float32)
    got = N.dquantize(code, m32).astype(np.int64)
    assert np.all((got == np.arange(255)) | (got == np.arange(1, 256)))


@pytest.mark.parametrize("n", [1, 5, 1024, 1025, 70000])
def test_tree_sum(n):
    """Exact on small integers (any order is exact there), and within fp64 rounding of fsum."""
    import math
    ints = np.arange(n, dtype=np.float64) % 97
    assert N.tree_sum(ints) == ints.sum()
    rng = np.random.default_rng(n)
    v = rng.uniform(0.0, 1.0, n)
    assert abs(N.tree_sum(v) - math.fsum(v)) <= 1e-13 * max(1.0, math.fsum(v))


def test_product_dynamic_map_equals_oracle(pkg):
    """The code the GPU quantiser is handed is the oracle's create_dynamic_map, bit for bit."""
    assert np.array_equal(pkg.quant._dynamic_map().numpy(), N.create_dynamic_map())
