"""Pins of the dropout-mask oracle (oracle/philox.py)."""

import json
import os

import numpy as np
import pytest

from oracle import philox as P

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "rocrand_uniform4.json")


@pytest.mark.parametrize("ctr,key,want", [
    # Random123 known-answer vectors for philox4x32_10 (kat_vectors, Salmon et al. SC'11)
    ((0, 0, 0, 0), (0, 0), (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
    ((0xffffffff,) * 4, (0xffffffff,) * 2, (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
    ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
     (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
])
def test_philox_random123_kat(ctr, key, want):
    got = P.philox4x32_10(*[np.array([c], np.uint32) for c in ctr],
                          np.uint32(key[0]), np.uint32(key[1]))
    assert tuple(int(w[0]) for w in got) == want


def test_matches_rocrand_headers():
    """rocrand_init(seed, subsequence, offset) + rocrand4 / rocrand_uniform4, from rocRAND's own
    headers compiled for the host (tests/golden/make_rocrand_vectors.py)."""
    data = json.load(open(GOLDEN))
    assert len(data["cases"]) >= 5
    for case in data["cases"]:
        k0, k1 = P._seed_words(case["seed"])
        sub, ctr = case["subsequence"], case["offset"] // 4
        for j, draw in enumerate(case["draws"]):
            c = ctr + j
            words = P.philox4x32_10(np.uint32(c & 0xFFFFFFFF), np.uint32(c >> 32),
                                    np.uint32(sub & 0xFFFFFFFF), np.uint32(sub >> 32), k0, k1)
            assert [int(w) for w in words] == draw["u32"], (case, j)
            bits = P.uniform(np.array(draw["u32"], np.uint32)).view(np.uint32).tolist()
            assert bits == draw["f32_bits"], (case, j)


def test_keep_mask_is_thread_draw_layout():
    """Element e of a VEC=8 call is word e%4 of draw (e//8 // G)*2 + (e%8)//4 of thread
    (e//8) % G: check against a direct per-thread simulation of the grid-stride loop."""
    G, vec, seed, ctr, p_keep = 48, 8, 99, 12, np.float32(0.9)
    nelem = G * vec * 3 + 40
    mask = P.keep_mask_call(nelem, seed, ctr, G, p_keep, vec)
    k0, k1 = P._seed_words(seed)
    want = np.zeros(nelem, bool)
    for t in range(G):
        draws = 0
        for start in range(t * vec, nelem, G * vec):
            for ii in range(0, vec, 4):
                c = ctr + draws
                draws += 1
                w = P.philox4x32_10(np.uint32(c), np.uint32(0), np.uint32(t), np.uint32(0),
                                    k0, k1)
                for jj in range(4):
                    e = start + ii + jj
                    if e < nelem:
                        want[e] = P.uniform(np.array([int(w[jj])], np.uint32))[0] < p_keep
    np.testing.assert_array_equal(mask, want)


@pytest.mark.parametrize("p", [0.05, 0.25])
def test_keep_rate(p):
    mask = P.keep_mask_call(4 * 37 * 1536, 1234, 17, 524288, np.float32(1 - p), 4)
    rate = 1 - mask.mean()
    assert abs(rate - p) < 4 * np.sqrt(p * (1 - p) / mask.size)


def test_generator_offsets_of_reference_run():
    """The reference's T4 run left the CUDA generator at offsets 2016, 4928, 9408 after steps
    1-3 (README.md:676-677): 56 dropout calls per step (28 layers x q, v), T4 grid G = 40960
    threads (test_kernels.py:105). Each step's advance must be 56 equal increments the launch
    formula can produce for a [4, T, 1536] fp32 LoRA input."""
    max_blocks = 40960 // 256
    advances = [2016, 4928 - 2016, 9408 - 4928]
    reachable = {}
    for T in range(1, 1025):
        _, G, inc = P.draw(4 * T * 1536, 0, max_blocks)
        assert G == 40960 or 4 * T * 1536 < 40960
        reachable.setdefault(inc, T)
    for adv in advances:
        assert adv % 56 == 0
        inc = adv // 56
        assert inc % 4 == 0 and inc in reachable, (adv, inc)


def test_p0_keeps_everything():
    """p = 0: every element kept, whatever the draw (PyTorch's dropout is the identity then);
    the oracle's normed LoRA inputs equal the normed rows."""
    assert P.keep_mask(np.arange(1 << 16), 5, 7, 4096, np.float32(1.0), 4).all()
    import torch
    from oracle import ops as O
    x = torch.randn(6, 40, generator=torch.Generator().manual_seed(0))
    w = torch.rand(40, generator=torch.Generator().manual_seed(1)) + 0.5
    o = O.rms_fwd(x, w, 1e-6, tok=torch.arange(6), p=0.0, seed=9, ctrs=(3, 4), G=64,
                  drop_q=True, drop_v=True)
    assert torch.equal(o[2], o[1]) and torch.equal(o[3], o[1])
