"""The step's GEMMs: frozen NF4 projections forward (Y = X W^T [+ bias]) and backward
(dX = dY W), and the plain fp16 lm_head products (engine.py:1082, 1112, 1163, 1179, 1239, 1293,
1301, 1316, 1376, 1381). Every product runs on this package's MFMA GEMM.

Backend "dequant" (default, the faster one): the layer-wide dequant kernel into fp16 buffers,
then the package's fp16-B GEMM (qlora_gemm16) with its fixed tile/split plan - the reference's
own structure (dequant, then cuBLAS) - with the epilogues the step needs (qkv bias, the SwiGLU of
gate|up with or without the product kept, the residual add after down_proj).
Backend "fused": qlora_nf4_gemm, the NF4 decode inside the MFMA GEMM's B-operand loader, with
the same epilogues.
"""

import ctypes

import torch

from . import _lib
from .ops import NF4Group, _need, _ptr, _stream, dequant, dequant_many, gemm_tiles

BACKEND = "dequant"


def _weights(w):
    return w.weights if isinstance(w, NF4Group) else [w]


_REUSE = None


class reuse_dequant:
    """Within this context each NF4 weight is dequantized once and its fp16 copy reused (a
    layer's backward multiplies by the same weights in its recompute and in its dY W products);
    `copies`: fp16 copies made earlier (a forward's, kept for its backward), used instead of
    dequantizing again. On exit the context's copies stay in `self.copies` for the caller to
    keep or drop."""

    def __init__(self, copies=None):
        self.copies = {} if copies is None else copies

    def __enter__(self):
        global _REUSE
        self.prev, _REUSE = _REUSE, self.copies
        return self

    def __exit__(self, *exc):
        global _REUSE
        _REUSE = self.prev
        return False


def dequant_layer(weights):
    """Dequantize the given weights (at most four: a layer's qkv, o, gate|up, down) in one
    launch into the active reuse_dequant context, where the layer's products then find them."""
    if _REUSE is None or BACKEND != "dequant":
        return
    todo = [w for w in weights if w not in _REUSE]
    if todo:
        for w, out in zip(todo, dequant_many(todo, todo[0].packed.device)):
            _REUSE[w] = out


def dequantize(w):
    """fp16 [N, K] of an NF4Weight or NF4Group (one launch for a group)."""
    if _REUSE is not None and w in _REUSE:
        return _REUSE[w]
    ws = _weights(w)
    out = dequant(ws, ws[0].packed.device)
    if _REUSE is not None:
        _REUSE[w] = out
    return out


def _shape(w):
    ws = _weights(w)
    return sum(x.shape[0] for x in ws), ws[0].shape[1]


def _nf4_args(w, tiled=False, swiglu_I=0):
    """(packed, scales, code, bs1, tiled) of an NF4Weight or NF4Group, as qlora_nf4_gemm takes
    them (code null for the NF4 table); tiled: the tile-major copy of codes and scales."""
    if tiled:
        codes, scales = gemm_tiles(w, swiglu_I)
    else:
        codes, scales = w.packed, w.block_scales()
    return (_ptr(codes), _ptr(scales), None if w.standard else _ptr(w.code), w.bs1, int(tiled))


TILE = 256  # output tile of the MFMA GEMM kernels (256 x 256; SwiGLU: 256 x 128 outputs)
SLOTS = 256  # workgroups resident at once (one per CU)


def split_k(M, N, Kr, epi):
    """Slices of the reduction for the MFMA GEMMs: doubled while the tiles alone leave CUs idle
    and every slice keeps at least 8 k-tiles of 64 (the partial sums cost an fp32 round trip
    of M N per slice)."""
    if epi in (3, 5):
        return 1
    tiles = -(-M // TILE) * (N // TILE)
    ktiles = Kr // 64
    s = 1
    while s < 8 and tiles * s < SLOTS and ktiles // (2 * s) >= 8:
        s *= 2
    return s


def _gemm_out(a, M, n_out, epi, resid, out, dev):
    odt = torch.float32 if epi == 2 else torch.float16
    if out is None:
        out = torch.empty((M, n_out), device=dev, dtype=odt)
    _need(out, "out", odt, dev, contiguous=False)
    if out.shape != (M, n_out) or out.stride(1) != 1:
        raise ValueError("out has the wrong shape")
    ldr = 0
    if epi == 2:
        _need(resid, "resid", torch.float32, dev, contiguous=False)
        if resid.shape != (M, n_out) or resid.stride(1) != 1:
            raise ValueError("resid must match the output")
        ldr = resid.stride(0)
    return out, ldr


def _a16(a):
    _need(a, "a", None, contiguous=False)
    if a.dim() != 2:
        raise ValueError("a must be 2-D")
    if a.dtype == torch.float32:
        a = a.to(torch.float16)  # the reference's dY.to(fp16) before the product
    if a.dtype != torch.float16:
        raise ValueError("a must be fp16 or fp32")
    if a.stride(1) != 1 or a.stride(0) % 8 or a.data_ptr() % 16:
        a = a.contiguous()
    return a


def nf4_gemm(a, w, mode, epi=0, bias=None, resid=None, out=None, swiglu_I=0, splits=None,
             tiled=True):
    """The fused NF4-decode GEMM (qlora_nf4_gemm). mode 0: A [M, K] x W^T; mode 1:
    A [M, N_w] x W. epi 0 fp16, 1 + bias, 2 fp32 residual (out = resid + fp16(acc)), 3 SwiGLU
    of [gate | up] (mode 0). tiled (mode 0): read the weight's tile-major copy (formed on first
    use) instead of the bitsandbytes order; the same results."""
    dev = a.device
    a = _a16(a)
    M = a.shape[0]
    w_rows, w_cols = _shape(w)
    if mode == 0:
        n_out, kr = (swiglu_I if epi == 3 else w_rows), w_cols
    else:
        n_out, kr = w_cols, w_rows
    if a.shape[1] != kr:
        raise ValueError(f"a has {a.shape[1]} columns, the product reduces over {kr}")
    if epi == 1:
        _need(bias, "bias", torch.float16, dev)
        if bias.numel() != n_out:
            raise ValueError("bias must have one entry per output column")
    out, ldr = _gemm_out(a, M, n_out, epi, resid, out, dev)
    if M == 0:
        return out
    splits = split_k(M, n_out, kr, epi) if splits is None else splits
    ws = torch.empty((splits * M * n_out,), device=dev, dtype=torch.float32) if splits > 1 \
        else None
    tiled = tiled and mode == 0
    _lib.call("qlora_nf4_gemm", _ptr(a), a.stride(0),
              *_nf4_args(w, tiled, swiglu_I if epi == 3 else 0), w_rows, w_cols, _ptr(out),
              out.stride(0), _ptr(bias), _ptr(resid), ldr, M, mode, epi, swiglu_I, splits,
              _ptr(ws), 0 if ws is None else ws.numel(), _stream(dev))
    return out


_HGEMM_WS = {}  # (M, N, K, epi, tile, splits) -> fp32 workspace elements qlora_gemm16 uses
# qlora_gemm16 in one slice runs a last, nearly empty round of tiles as K slices (default of
# hgemm's `tail`)
HGEMM_TAIL = True


def hgemm_workspace(M, N, K, epi, splits, tile=256, stages=2, mode=0):
    """fp32 elements of qlora_gemm16's workspace for this problem (qlora_gemm16_workspace;
    tile 0 / splits 0: the automatic plan's)."""
    key = (M, N, K, mode, epi, tile, stages, splits)
    n = _HGEMM_WS.get(key)
    if n is None:
        c = ctypes.c_int64(0)
        _lib.call("qlora_gemm16_workspace", M, N, K, mode, epi, tile, stages, splits,
                  ctypes.byref(c))
        n = _HGEMM_WS[key] = c.value
    return n


def gemm_plan(M, N, K, mode, epi=0):
    """(tile, stages, splits) of qlora_gemm16's automatic plan for this problem."""
    t, st, sp = ctypes.c_int32(0), ctypes.c_int32(0), ctypes.c_int32(0)
    _lib.call("qlora_gemm16_plan", M, N, K, mode, epi, ctypes.byref(t), ctypes.byref(st),
              ctypes.byref(sp))
    return t.value, st.value, sp.value


def gemm_plan_split(M, N, K, mode, epi=0):
    """qlora_gemm16's automatic plan in full: (tile, stages, splits, rest, n_first); rest > 0:
    the output columns past n_first run as a second launch on 128 x 128 tiles with `rest`
    stages."""
    t, st, sp, r = (ctypes.c_int32(0) for _ in range(4))
    nf = ctypes.c_int64(0)
    _lib.call("qlora_gemm16_plan_split", M, N, K, mode, epi, ctypes.byref(t), ctypes.byref(st),
              ctypes.byref(sp), ctypes.byref(r), ctypes.byref(nf))
    return t.value, st.value, sp.value, r.value, nf.value


def hgemm(a, b, mode, epi=0, bias=None, resid=None, out=None, swiglu_I=0, splits=None,
          tail=None, tile=256, stages=2, gu=None):
    """The MFMA GEMM with an fp16 B (qlora_gemm16): mode 0 C = A B^T (B [N, K]), mode 1 C = A B
    (B [K, N]); epilogues as nf4_gemm; tile: 256 or 128 (output tile edge), stages: 2, or 4 for
    128 x 128 tiles (one workgroup per CU, loads three k-tiles ahead). tail: with one slice, the
    tiles of a last, nearly empty round of the GPU run as K slices through a workspace (False:
    whole; None: HGEMM_TAIL). epi 5: SwiGLU as epi 3 and the product [g | u] itself written
    to `gu` (fp16 [M, 2 I])."""
    dev = a.device
    a = _a16(a)
    _need(b, "b", torch.float16, dev, contiguous=False)
    if b.dim() != 2 or b.stride(1) != 1:
        raise ValueError("b must be 2-D with unit column stride")
    M, K = a.shape
    if mode == 0:
        rows, kb = b.shape
        n_out = swiglu_I if epi in (3, 5) else rows
    else:
        kb, n_out = b.shape
    if kb != K:
        raise ValueError(f"inner dimensions differ: {K} vs {kb}")
    if epi == 1:
        _need(bias, "bias", torch.float16, dev)
        if bias.numel() != n_out:
            raise ValueError("bias must have one entry per output column")
    if epi == 5:
        _need(gu, "gu", torch.float16, dev, contiguous=False)
        if gu.shape != (M, 2 * n_out) or gu.stride(1) != 1:
            raise ValueError("gu must be [M, 2 I] with unit column stride")
    out, ldr = _gemm_out(a, M, n_out, epi, resid, out, dev)
    if M == 0:
        return out
    if tile == 0:  # the library's plan
        splits = 0
    elif splits is None:
        splits = split_k(M, n_out, K, epi)
    tail = HGEMM_TAIL if tail is None else tail
    n_ws = hgemm_workspace(M, n_out, K, epi, splits, tile, stages, mode) \
        if splits != 1 or tail or tile == 0 else 0
    ws = torch.empty((n_ws,), device=dev, dtype=torch.float32) if n_ws else None
    _lib.call("qlora_gemm16", _ptr(a), a.stride(0), _ptr(b), b.stride(0), M, n_out, K, mode,
              _ptr(out), out.stride(0), _ptr(bias), _ptr(resid), ldr, epi, swiglu_I, _ptr(gu),
              0 if gu is None else gu.stride(0), tile, stages, splits, _ptr(ws),
              0 if ws is None else ws.numel(), _stream(dev))
    return out


def gemm_f32(a, b, mode, alpha=1.0, row_scale=None, resid=None, out=None, tile=0, stages=2,
             splits=None):
    """The MFMA GEMM with an unrounded fp32 output (qlora_gemm16_f32): out = alpha A op(B)
    (+ row_scale[:, None] * resid). mode 1: A [M, K] x B [K, N]; mode 2: A^T B with A given as
    [K, M] (its columns are the output rows). resid may be out itself (then updated in place).
    tile 0: the automatic plan; else tile 256 or 128 with `stages` and `splits` (default 1)."""
    dev = a.device
    _need(a, "a", torch.float16, dev, contiguous=False)
    _need(b, "b", torch.float16, dev, contiguous=False)
    if a.dim() != 2 or b.dim() != 2 or a.stride(1) != 1 or b.stride(1) != 1:
        raise ValueError("a and b must be 2-D with unit column stride")
    if mode == 1:
        M, K = a.shape
    elif mode == 2:
        K, M = a.shape
    else:
        raise ValueError("mode must be 1 (A B) or 2 (A^T B)")
    kb, N = b.shape
    if kb != K:
        raise ValueError(f"inner dimensions differ: {K} vs {kb}")
    if out is None:
        out = torch.empty((M, N), device=dev, dtype=torch.float32)
    _need(out, "out", torch.float32, dev, contiguous=False)
    if out.shape != (M, N) or out.stride(1) != 1:
        raise ValueError("out must be [M, N] fp32 with unit column stride")
    ldr = 0
    if resid is not None:
        _need(resid, "resid", torch.float32, dev, contiguous=False)
        if resid.shape != (M, N) or resid.stride(1) != 1:
            raise ValueError("resid must match the output")
        ldr = resid.stride(0)
    if row_scale is not None:
        _need(row_scale, "row_scale", torch.float32, dev)
        if resid is None or row_scale.numel() != M:
            raise ValueError("row_scale needs resid and one entry per output row")
    if M == 0:
        return out
    if tile == 0 and mode == 2 and M > 256 and M % 256:
        # transposed A takes whole tiles of M only: the columns up to the last multiple of 256
        # on 256 x 256 tiles, the rest (128 of them for every Qwen2 vocabulary) on their own
        m1 = M // 256 * 256
        for lo, hi in ((0, m1), (m1, M)):
            gemm_f32(a[:, lo:hi], b, 2, alpha, None if row_scale is None else row_scale[lo:hi],
                     None if resid is None else resid[lo:hi], out[lo:hi])
        return out
    if tile == 0:
        splits = 0
    elif splits is None:
        splits = 1
    n_ws = hgemm_workspace(M, N, K, 6, splits, tile, stages, mode) if splits != 1 else 0
    ws = torch.empty((n_ws,), device=dev, dtype=torch.float32) if n_ws else None
    _lib.call("qlora_gemm16_f32", _ptr(a), a.stride(0), _ptr(b), b.stride(0), M, N, K, mode,
              _ptr(out), out.stride(0), float(alpha), _ptr(row_scale), _ptr(resid), ldr, tile,
              stages, splits, _ptr(ws), 0 if ws is None else ws.numel(), _stream(dev))
    return out


def tiles(K, N, mode):
    """Whether qlora_gemm16 takes a product with reduction K and N output columns: K in blocks
    of 128, N a multiple of 8 (NT) or of 128 (NN). Every Qwen2 size does (H, I, the q/k/v
    widths, the vocabularies 151,936 and 152,064)."""
    return K % 128 == 0 and (N % 8 == 0 if mode == 0 else N % 128 == 0)


def _check(K, N, mode, what):
    if not tiles(K, N, mode):
        raise ValueError(f"{what}: the package GEMM needs the reduction in blocks of 128 and "
                         f"{'N % 8' if mode == 0 else 'N % 128'} == 0 (got K = {K}, N = {N})")


def nf4_linear(x, w, bias=None):
    """Y = X W^T [+ bias], fp16 [M, N]."""
    if BACKEND == "fused":
        return nf4_gemm(x, w, 0, epi=1 if bias is not None else 0, bias=bias)
    _check(x.shape[1], _shape(w)[0], 0, "X W^T")
    return hgemm(x, dequantize(w), 0, epi=1 if bias is not None else 0, bias=bias, tile=0)


# The gate|up product with the NF4 weight decoded inside the GEMM (qlora_nf4_gemm over the
# weight's tile-major copy): the forward then dequantizes the layer's other three weights only.
# Off: alternating runs on one box gave 36.16 / 36.28 ms per step against 35.98 / 35.98 ms with
# the fp16 weight (the in-kernel decode costs about as much as the dequant it saves).
SWIGLU_NF4 = False


def swiglu_fused_nf4():
    """Whether the forward's gate|up product reads the NF4 weight itself (no fp16 copy)."""
    return BACKEND == "fused" or SWIGLU_NF4


def _gemm_fits(I, K):
    """The package's GEMM takes the SwiGLU output in 128-column tiles and the reduction in
    blocks of 128 (every Qwen2.5 size does: I = 4864 ... 29568, H = 896 ... 8192)."""
    return I % 128 == 0 and K % 128 == 0


def nf4_linear_swiglu(x, w, I):
    """m = fp16(silu(g) * u) of [g | u] = X W^T for the stacked gate|up weight, fp16 [M, I]:
    the SwiGLU in the GEMM's epilogue ([gate | up] never stored)."""
    if not _gemm_fits(I, x.shape[1]):
        raise ValueError(f"SwiGLU product: I = {I} and K = {x.shape[1]} must be multiples of 128")
    if swiglu_fused_nf4():
        return nf4_gemm(x, w, 0, epi=3, swiglu_I=I)
    return hgemm(x, dequantize(w), 0, epi=3, swiglu_I=I, tile=0)


def nf4_linear_swiglu_keep(x, w, I):
    """(m, [g | u]): the SwiGLU of the stacked gate|up product and the product itself, fp16
    [M, I] and [M, 2 I], from one GEMM (a recomputing layer keeps [g | u] for its backward, as
    the reference's step keeps it rather than multiplying again, engine.py:1204-1213); None
    with the NF4-decoding backend (which has no such epilogue)."""
    if BACKEND == "fused":
        return None
    if not _gemm_fits(I, x.shape[1]):
        raise ValueError(f"SwiGLU product: I = {I} and K = {x.shape[1]} must be multiples of 128")
    M = x.shape[0]
    gu = torch.empty((M, 2 * I), device=x.device, dtype=torch.float16)
    m = hgemm(x, dequantize(w), 0, epi=5, swiglu_I=I, tile=0, gu=gu)
    return m, gu


def nf4_linear_gu(x, w):
    """[g | u] = X W^T for the stacked gate|up weight, fp16 [M, 2 I] (kept for the backward)."""
    return nf4_linear(x, w)


def nf4_linear_resid(x, w, resid, out=None):
    """fp32 resid + fp16(X W^T) (the layer output h2 + d): the residual added in the GEMM's
    epilogue (or the split-K reduce's), no fp16 product in memory."""
    if BACKEND == "fused":
        return nf4_gemm(x, w, 0, epi=2, resid=resid, out=out)
    _check(x.shape[1], _shape(w)[0], 0, "X W^T + resid")
    return hgemm(x, dequantize(w), 0, epi=2, resid=resid, out=out, tile=0)


def nf4_linear_t(dy, w):
    """dX = fp16(dY) W, fp16 [M, K]; dY may be fp32 (rounded to fp16 first, as the reference's
    dY.to(fp16) @ W)."""
    if BACKEND == "fused":
        return nf4_gemm(dy, w, 1)
    if dy.dtype != torch.float16:
        dy = dy.to(torch.float16)
    _check(dy.shape[1], _shape(w)[1], 1, "dY W")
    return hgemm(dy, dequantize(w), 1, tile=0)


def hgemm_parts(a, b, mode):
    """qlora_gemm16 under its automatic plan, but a split-K plan's K slices are returned unsummed
    (fp32 [S, M, N], for a consumer that sums them in slice order: _rms_bwd dy_parts); a plan in
    one slice returns the fp16 product itself. Returns (product or None, slices or None)."""
    M, K = a.shape
    N = b.shape[0] if mode == 0 else b.shape[1]
    tile, stages, splits, rest, _ = gemm_plan_split(M, N, K, mode, 0)
    if splits == 1 or M == 0:
        return hgemm(a, b, mode, tile=0), None
    a = _a16(a)
    _need(b, "b", torch.float16, a.device, contiguous=False)
    ws = torch.empty((splits, M, N), device=a.device, dtype=torch.float32)
    _lib.call("qlora_gemm16_parts", _ptr(a), a.stride(0), _ptr(b), b.stride(0), M, N, K, mode,
              tile, stages, splits, _ptr(ws), ws.numel(), _stream(a.device))
    return None, ws


def nf4_linear_t_parts(dy, w):
    """nf4_linear_t, but a split-K plan's slices returned unsummed (hgemm_parts)."""
    if BACKEND == "fused" or dy.dtype != torch.float16:
        return nf4_linear_t(dy, w), None
    _check(dy.shape[1], _shape(w)[1], 1, "dY W")
    return hgemm_parts(dy, dequantize(w), 1)


def linear(x, w):
    """x W^T for an fp16 weight [V, H] (the lm_head)."""
    _check(x.shape[1], w.shape[0], 0, "lm_head x E^T")
    return hgemm(x, w, 0, tile=0)


def linear_t(g, w):
    """g W for an fp16 weight [V, H] (the lm_head's input gradient)."""
    _check(g.shape[1], w.shape[1], 1, "lm_head G E")
    return hgemm(g, w, 1, tile=0)
