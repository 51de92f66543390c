"""The C-ABI library: loads, exports every entry point include/qlora_amd.h declares, and the
Python binding covers the same set with the same arity. No device call is made here."""

import ctypes
import os
import re

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    decls = {}
    for name in os.listdir(os.path.join(ROOT, "include")):
        if not name.endswith(".h"):
            continue
        text = open(os.path.join(ROOT, "include", name)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(?:int|const char\*)\s+(qlora_\w+)\s*\(([^;]*?)\)\s*;", text,
                             flags=re.S):
            args = m.group(2).strip()
            decls[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return decls


def test_header_declares_entry_points():
    decls = _declared()
    assert len(decls) >= 13
    assert "qlora_nf4_dequant" in decls and "qlora_ce_piece" in decls


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg._lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.qlora_abi_version() == 1


def test_binding_matches_header(pkg):
    decls = _declared()
    sigs = pkg._lib.SIGNATURES
    for name, nargs in decls.items():
        if name in ("qlora_error_string", "qlora_abi_version"):
            continue
        assert name in sigs, name
        assert len(sigs[name]) == nargs, (name, len(sigs[name]), nargs)
    assert set(sigs) <= set(decls)


def test_error_string(pkg):
    lib = pkg._lib.load()
    assert lib.qlora_error_string(1)  # hipErrorInvalidValue has a message


class _Spec:
    eps = 1e-6
    HQ, HKV, D = 12, 2, 128


def test_ops_refuse_cpu_tensors(pkg):
    """No CPU path: host tensors are rejected before any launch."""
    x = torch.zeros(4, 64)
    w = torch.ones(64)
    with pytest.raises(ValueError, match="GPU"):
        pkg.ops._rms_fwd(_Spec, x, w, None)
    with pytest.raises(ValueError, match="GPU"):
        pkg.ops._glu_fwd(torch.zeros(2, 16, dtype=torch.float16), 8)
    with pytest.raises(ValueError, match="GPU"):
        pkg.ops._ce(torch.zeros(2, 16, dtype=torch.float16), torch.zeros(2, dtype=torch.long),
                    torch.zeros(2), torch.zeros(2), torch.zeros(2, dtype=torch.int32))


def test_zero_rows_is_noop_without_launch(pkg):
    """n == 0 returns 0 from the C-ABI without touching the device (reference: launches are
    skipped for empty inputs, engine.py:958, 973, 991)."""
    lib = pkg._lib.load()
    assert lib.qlora_glu_fwd(None, None, 0, 8960, None) == 0
    assert lib.qlora_nf4_dequant(None, None, None, None, None, None, None, 0, 1, 1, 64, 256,
                                 0, 0, None) == 0
    assert lib.qlora_ce(None, 16, None, None, None, None, 0, 16, 1, None) == 0


def test_invalid_arguments_rejected_before_launch(pkg):
    lib = pkg._lib.load()
    # D not a multiple of 16, negative sizes, bad block size: hipErrorInvalidValue (1)
    assert lib.qlora_rope_fwd(None, None, None, None, None, 512, None, None, None, None, 5, 12,
                              2, 100, 12, 1.0, None) == 1
    assert lib.qlora_glu_fwd(None, None, -1, 8, None) == 1
    assert lib.qlora_nf4_dequant(None, None, None, None, None, None, None, 4, 0, 1, 6, 256,
                                 0, 0, None) == 1


def test_gemm16_rejects_bad_problems_before_any_device_call(pkg):
    """qlora_gemm16 checks mode, sizes, leading dimensions, tile/stage pairs and the epilogue's
    operands on the host (hipErrorInvalidValue, nothing launched): null pointers stand in for
    the buffers, which the checks never read."""
    lib = pkg._lib.load()
    P = 16  # a non-null, 16-byte aligned stand-in address: the checks fail before any access

    def gemm(M=256, N=256, K=256, mode=0, ldc=256, epi=0, tile=256, stages=2, splits=1,
             lda=256, ldb=256, bias=None, resid=None, ldr=0, gu=None, ldgu=0, swiglu_I=0):
        return lib.qlora_gemm16(P, lda, P, ldb, M, N, K, mode, P, ldc, bias, resid, ldr, epi,
                                swiglu_I, gu, ldgu, tile, stages, splits, None, 0, None)

    assert gemm(mode=2) == 1                       # no such mode
    assert gemm(K=192) == 1                        # reduction not in blocks of 128
    assert gemm(mode=1, N=200, ldb=256) == 1       # NN: N not a multiple of the tile
    assert gemm(N=12, ldb=256, ldc=16) == 1        # NT: N % 8
    assert gemm(tile=256, stages=4) == 1           # four stages need 128 x 128 tiles
    assert gemm(tile=64) == 1                      # no such tile
    assert gemm(tile=0, splits=1) == 1             # the automatic plan takes tile 0 and splits 0
    assert gemm(lda=200) == 1                      # lda < K
    assert gemm(epi=1) == 1                        # bias epilogue without a bias
    assert gemm(epi=2) == 1                        # residual epilogue without a residual
    assert gemm(epi=5, N=128, swiglu_I=128) == 1   # SwiGLU keep without gu
    assert gemm(epi=3, mode=1) == 1                # SwiGLU is NT only
    assert gemm(epi=3, splits=2) == 1              # SwiGLU takes no split-K
    assert gemm(splits=2) == 1                     # split-K without a workspace
    assert gemm(epi=4) == 1                        # the partials form is internal
    assert gemm(M=-1) == 1
    assert gemm(M=0) == 0                          # no rows: nothing to do


def test_gemm16_f32_rejects_bad_problems_before_any_device_call(pkg):
    """qlora_gemm16_f32 checks its mode, the transposed-A shape (whole tiles of M), the
    reduction blocks, leading dimensions and the row scale's residual on the host."""
    lib = pkg._lib.load()
    P = 16  # non-null, 16-byte aligned stand-in: the checks fail before any access

    def f32(M=256, N=256, K=256, mode=1, lda=256, ldb=256, ldc=256, tile=256, stages=2,
            splits=1, row_scale=None, resid=None, ldr=0):
        return lib.qlora_gemm16_f32(P, lda, P, ldb, M, N, K, mode, P, ldc, 1.0, row_scale,
                                    resid, ldr, tile, stages, splits, None, 0, None)

    assert f32(mode=0) == 1                    # the fp32 form is NN or transposed-A
    assert f32(mode=3) == 1
    assert f32(mode=2, M=200, lda=256) == 1    # transposed A: whole tiles of M
    assert f32(mode=2, M=256, lda=200) == 1    # lda >= M
    assert f32(K=192) == 1                     # reduction in blocks of 128
    assert f32(N=200) == 1                     # N % tile
    assert f32(row_scale=P) == 1               # a row scale without a residual
    assert f32(resid=P, ldr=100) == 1          # ldr >= N
    assert f32(splits=2) == 1                  # split-K without a workspace
    assert f32(tile=256, stages=4) == 1
    assert f32(M=0) == 0


def test_gemm16_workspace_sizes(pkg):
    """qlora_gemm16_workspace (host only) at 256 x 256 tiles: splits x M x N with split-K; with
    one slice the K-sliced last round's partials when at most 64 tiles are left past the last
    full round of 256 (the largest slice count that fits that round with no empty slice), else
    0."""
    import ctypes
    lib = pkg._lib.load()

    def ws(M, N, K, epi, splits):
        n = ctypes.c_int64(-1)
        assert lib.qlora_gemm16_workspace(M, N, K, 0, epi, 256, 2, splits, ctypes.byref(n)) == 0
        return n.value

    tile = 256 * 256
    assert ws(700, 2048, 1536, 0, 4) == 4 * 700 * 2048
    # SwiGLU, I = 8960 (70 tiles per 256 rows): 2,600 rows -> 770 tiles, 2 past 768; 24 k-tiles
    # of 64: 12 slices of 2 (16 slices would leave some empty)
    assert ws(2600, 8960, 1536, 3, 1) == 2 * 12 * tile
    assert ws(2600, 8960, 1536, 5, 1) == 2 * 12 * tile  # the keep form: the same tail
    assert ws(2560, 8960, 1536, 3, 1) == 0  # 700 tiles: 188 past 512, more than a quarter
    assert ws(300, 8960, 1536, 3, 1) == 0   # 140 tiles: no full round
    # 2,048 columns (8 tiles per 256 rows), 33 row tiles -> 264 tiles, 8 past 256: 16 slices
    # would leave empty ones with 24 k-tiles, 12 of 2 fit (8 x 12 <= 256)
    assert ws(8348, 2048, 1536, 0, 1) == 8 * 12 * tile
    assert ws(8348, 2048, 16384, 0, 1) == 8 * 16 * tile  # 256 k-tiles: 16 slices of 16
    assert ws(0, 2048, 1536, 0, 1) == 0
    n = ctypes.c_int64()
    assert lib.qlora_gemm16_workspace(4, 8, 128, 0, 0, 256, 2, 0, ctypes.byref(n)) == 1
    assert lib.qlora_gemm16_workspace(4, 8, 128, 0, 0, 256, 2, 1, None) == 1
    assert lib.qlora_gemm16_workspace(4, 8, 128, 0, 4, 256, 2, 1, ctypes.byref(n)) == 1


def _uniform32(r):
    """rocRAND's fp32 uniform of Philox words r (uint32 array): 2^-32 + r 2^-32, in numpy fp32."""
    inv = np.float32(2.0**-32)
    return inv + r.astype(np.float32) * inv


@pytest.mark.parametrize("p_keep", [0.95, 0.9, 0.75, 0.5, 0.25, 0.05, 1e-3, 0.999999,
                                    np.nextafter(np.float32(1), np.float32(0)), 2.0**-32,
                                    3.0 * 2.0**-32, 0.0, 1.0])
def test_dropout_keep_below_is_the_fp32_compare(pkg, p_keep):
    """The integer keep test r < keep_below of every dropout kernel equals the fp32 compare
    2^-32 + r 2^-32 < p_keep: the words just below and at the threshold, the whole word range's
    ends, and a spread of words, evaluated in numpy fp32 (not through the library)."""
    lib = pkg._lib.load()
    out = ctypes.c_uint32()
    assert lib.qlora_dropout_keep_below(ctypes.c_float(p_keep), ctypes.byref(out)) == 0
    T = int(out.value)
    p = np.float32(p_keep)
    if p >= 1:
        return  # every word is kept by the kernels' own p_keep >= 1 test
    words = np.unique(np.concatenate([
        np.arange(max(T - 300, 0), min(T + 300, 2**32), dtype=np.int64),
        np.array([0, 1, 2**32 - 1], dtype=np.int64),
        np.linspace(0, 2**32 - 1, 4097).astype(np.int64)])).astype(np.uint32)
    want = _uniform32(words) < p
    assert np.array_equal(words.astype(np.int64) < T, want), (p_keep, T)


def test_gemm16_plan_is_fixed_and_valid(pkg):
    """qlora_gemm16's automatic plan (host only, no device call): the same answer every time
    for a problem, and always a variant the library accepts (its workspace query succeeds with
    that explicit variant, and asks the same workspace as the automatic form) - over the step's
    products at token counts from 1 to 8,192 and other Qwen2 widths."""
    L = pkg.linear
    shapes = [(0, 2048, 1536, 1), (0, 1536, 1536, 2), (0, 17920, 1536, 0), (0, 8960, 1536, 3),
              (0, 1536, 8960, 2), (1, 1536, 2048, 0), (1, 1536, 1536, 0), (1, 1536, 17920, 0),
              (1, 8960, 1536, 0), (0, 151936, 1536, 0), (1, 1536, 151936, 0),
              (0, 1152, 896, 1), (1, 896, 4864, 0), (0, 4864, 896, 3), (1, 3584, 18944, 0)]
    for M in (1, 37, 300, 1875, 2325, 2560, 2949, 4096, 8192):
        for mode, N, K, epi in shapes:
            plan = L.gemm_plan(M, N, K, mode, epi)
            assert plan == L.gemm_plan(M, N, K, mode, epi)
            tile, stages, splits = plan
            assert (tile, stages) in ((256, 2), (128, 2), (128, 4)) and 1 <= splits <= 8
            assert (K // 64) % stages == 0 and (mode == 0 or N % tile == 0)
            assert epi != 3 or splits == 1
            auto = L.hgemm_workspace(M, N, K, epi, 0, 0, 0, mode)
            full = L.gemm_plan_split(M, N, K, mode, epi)
            assert full[:3] == plan
            rest, n_first = full[3:]
            if rest:  # leading columns on whole rounds of 256 x 256 tiles, the rest on 128 x 128
                assert tile == 256 and splits == 1 and rest in (2, 4) and auto == 0
                assert 0 < n_first < N and n_first % (128 if epi in (3, 5) else 256) == 0
                assert (K // 64) % rest == 0 and (mode == 0 or (N - n_first) % 128 == 0)
                continue
            assert n_first == 0
            assert auto == L.hgemm_workspace(M, N, K, epi, splits, tile, stages, mode)
            if splits > 1:
                assert auto == splits * M * N


def test_gemm16_plan_at_the_step_shapes(pkg):
    """The plan's choices at config-5 token counts, each the variant measured fastest there on
    MI355X (HIP graphs, warm caches): 128 x 128 tiles for the narrow products (four stages while
    one round of 256 CUs holds them, else two workgroups per CU), 256 x 256 tiles split along K
    for the longest reductions, and 256 x 256 tiles in one slice for gate|up and the lm_head."""
    L = pkg.linear
    assert L.gemm_plan(2560, 1536, 1536, 1, 0) == (128, 4, 1)  # o dX: 240 tiles
    assert L.gemm_plan(2560, 1536, 2048, 1, 0) == (128, 4, 1)  # qkv dX
    assert L.gemm_plan(2949, 1536, 1536, 1, 0) == (128, 2, 1)  # 288 tiles: two per CU
    assert L.gemm_plan(2560, 2048, 1536, 0, 1) == (128, 2, 1)  # qkv + bias: 320 tiles
    assert L.gemm_plan(2560, 8960, 1536, 0, 3) == (256, 2, 1)  # gate|up with SwiGLU
    assert L.gemm_plan(2560, 151936, 1536, 0, 0) == (256, 2, 1)  # lm_head
    assert L.gemm_plan(2560, 1536, 8960, 0, 2) == (128, 4, 1)  # down + residual: 84 us
    assert L.gemm_plan(2949, 1536, 8960, 0, 2) == (256, 2, 3)  # (288 tiles of 128)
    assert L.gemm_plan(2560, 1536, 17920, 1, 0) == (256, 2, 4)  # gate|up dX
    # down dX: two whole rounds of 256 x 256 tiles over the first 6,400 columns, the other
    # 2,560 on 128 x 128 tiles (two workgroups per CU), instead of 1,400 tiles of 128 x 128
    assert L.gemm_plan_split(2560, 8960, 1536, 1, 0) == (256, 2, 1, 2, 6400)
    # gate|up with SwiGLU at 2,113 tokens: 9 x 70 tiles; 56 whole N tiles in two rounds
    assert L.gemm_plan_split(2113, 8960, 1536, 0, 5) == (256, 2, 1, 2, 7168)
    assert L.gemm_plan_split(2560, 8960, 1536, 0, 5) == (256, 2, 1, 0, 0)
