"""LoRA-dropout keep masks on the CPU: Philox4x32-10 with rocRAND's state layout and uniform map,
over PyTorch's vectorized dropout grid.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

What the reference computes (kernels.py:108-126, engine.py:767-805) is the keep mask that
PyTorch's own `fused_dropout_kernel_vec` draws for element e of a contiguous tensor:
  g      = e // VEC                    (VEC elements per vector load; 4 for fp32, 8 for fp16)
  thread = g mod G                     (G = blocks * 256 threads of the launch)
  j      = (g // G) * (VEC / 4) + (e mod VEC) // 4      (the thread's j-th uniform4 draw)
  r      = Philox4x32-10(key = seed, counter = (ctr + j, thread))[e mod 4]
  keep   = U(r) < 1 - p                (fp32 compare)
with ctr = the generator's offset / 4 (engine.py:796-805). On ROCm, PyTorch's curand calls are
hipRAND -> rocRAND: rocrand_init(seed, subsequence=thread, offset) puts the key = (seed lo, seed
hi), counter.xy = offset / 4, counter.zw = subsequence (rocrand_philox4x32_10.h, restart /
discard_impl / discard_subsequence_impl), and rocrand_uniform4 maps each 32-bit output to
U = 2^-32 + float(r) * 2^-32 in fp32 (rocrand_uniform.h, uniform_distribution4).

Philox4x32-10 itself is the published Random123 generator (Salmon, Moraes, Dror, Shaw, SC'11):
ten rounds of (c0, c1, c2, c3) -> (hi(M1*c2) ^ c1 ^ k0, lo(M1*c2), hi(M0*c0) ^ c3 ^ k1,
lo(M0*c0)), with the key bumped by the Weyl constants (W0, W1) between rounds.

Pins (tests/test_oracle_philox.py):
  * Random123's published known-answer vectors for philox4x32_10;
  * tests/golden/rocrand_uniform4.json, written by tests/golden/make_rocrand_vectors.py, which
    compiles a host-only program against rocRAND's own headers (rocrand_init +
    rocrand_uniform4) - pins the init layout, draw order and uniform map;
  * on the GPU box, the HIP kernel's mask against torch.nn.functional.dropout on the same
    generator state (tests/test_gpu_dropout.py), the reference's own check (engine.py:807-828).
"""

import numpy as np

M0 = np.uint64(0xD2511F53)
M1 = np.uint64(0xCD9E8D57)
W0 = np.uint32(0x9E3779B9)
W1 = np.uint32(0xBB67AE85)
TWO_POW_M32 = np.float32(2.0 ** -32)
MASK32 = np.uint64(0xFFFFFFFF)


def philox4x32_10(c0, c1, c2, c3, k0, k1):
    """Vectorised Philox4x32-10. All arguments uint32 arrays (broadcastable). Returns 4 uint32
    arrays (the four output words, in counter-word order)."""
    c0, c1, c2, c3 = (np.asarray(c, dtype=np.uint32) for c in (c0, c1, c2, c3))
    k0 = np.asarray(k0, dtype=np.uint32) + np.zeros_like(c0)
    k1 = np.asarray(k1, dtype=np.uint32) + np.zeros_like(c0)
    with np.errstate(over="ignore"):
        for rnd in range(10):
            p0 = c0.astype(np.uint64) * M0
            p1 = c2.astype(np.uint64) * M1
            hi0 = (p0 >> np.uint64(32)).astype(np.uint32)
            lo0 = (p0 & MASK32).astype(np.uint32)
            hi1 = (p1 >> np.uint64(32)).astype(np.uint32)
            lo1 = (p1 & MASK32).astype(np.uint32)
            c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
            if rnd < 9:
                k0 = k0 + W0
                k1 = k1 + W1
    return c0, c1, c2, c3


def uniform(r):
    """rocRAND's uint32 -> fp32 map, (0, 1]: 2^-32 + float(r) * 2^-32, rounded as fp32."""
    f = np.asarray(r, dtype=np.uint32).astype(np.float32)
    return (TWO_POW_M32 + f * TWO_POW_M32).astype(np.float32)


def _seed_words(seed):
    s = int(seed) & 0xFFFFFFFFFFFFFFFF  # int64 seeds carry the uint64 bits (engine.py:803-804)
    return np.uint32(s & 0xFFFFFFFF), np.uint32(s >> 32)


def keep_mask(elems, seed, ctr, G, p_keep, vec):
    """Keep mask (bool) of the given element indices of one dropout call. p_keep >= 1 (p = 0)
    keeps everything: PyTorch's dropout returns its input unchanged for p = 0 (ATen
    Dropout.cpp, _dropout_impl), PEFT puts nn.Identity there."""
    e = np.asarray(elems, dtype=np.int64)
    if vec not in (4, 8):
        raise ValueError("vec must be 4 or 8")
    if np.float32(p_keep) >= np.float32(1.0):
        return np.ones(e.shape, dtype=bool)
    g = e // vec
    thread = (g % G).astype(np.uint64)
    j = (g // G) * (vec // 4) + (e % vec) // 4
    c = (np.uint64(int(ctr) & 0xFFFFFFFFFFFFFFFF) + j.astype(np.uint64))
    k0, k1 = _seed_words(seed)
    r = philox4x32_10((c & MASK32).astype(np.uint32), (c >> np.uint64(32)).astype(np.uint32),
                      (thread & MASK32).astype(np.uint32),
                      (thread >> np.uint64(32)).astype(np.uint32), k0, k1)
    comp = e % 4
    word = np.choose(comp, r)
    return uniform(word) < np.float32(p_keep)


def keep_mask_call(nelem, seed, ctr, G, p_keep, vec):
    """Keep mask of elements 0..nelem of one dropout call (the test hook of kernels.py:129-135)."""
    return keep_mask(np.arange(nelem, dtype=np.int64), seed, ctr, G, p_keep, vec)


BLOCK, UNROLL = 256, 4  # PyTorch's dropout launch: block size, counter unroll (engine.py:779)


def draw(nelem, offset, max_blocks):
    """PyTorch's dropout launch for nelem elements at generator offset `offset` (engine.py:796-805):
    returns (counter = offset // 4, threads G, the generator's offset increment)."""
    blocks = min(max_blocks, (nelem + BLOCK - 1) // BLOCK)
    increment = ((nelem - 1) // (BLOCK * blocks * UNROLL) + 1) * UNROLL
    return offset // 4, blocks * BLOCK, increment
