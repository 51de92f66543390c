"""GPU parity of every HIP kernel against the CPU oracle on the same seeded inputs (bit-exact for
NF4 dequant and dropout masks; the reference's tolerances elsewhere, test_kernels.py)."""

import math

import numpy as np
import pytest
import torch

from oracle import nf4 as ON
from oracle import ops as O
from oracle import philox as OP

pytestmark = pytest.mark.gpu

DEV = "cuda"


def close(a, b, tol):
    torch.testing.assert_close(a.detach().cpu().double(), b.detach().cpu().double(),
                               rtol=tol, atol=tol)


def bits16(t):
    return t.detach().cpu().contiguous().view(torch.int16)


class _Param:
    def __init__(self, packed, state):
        self.data, self.quant_state = packed, state


def _device_state(packed, st):
    """The numpy QuantState of the oracle as torch tensors on the GPU (bitsandbytes layout)."""
    qs = ON.QuantState(None, st.shape, None, st.blocksize)
    qs.code = torch.from_numpy(st.code).to(DEV)
    if st.nested:
        qs.absmax = torch.from_numpy(np.asarray(st.absmax)).to(DEV)
        qs.offset = torch.tensor(float(st.offset), dtype=torch.float32, device=DEV)
        qs.state2 = ON.QuantState2(torch.from_numpy(st.state2.absmax).to(DEV),
                                   torch.from_numpy(st.state2.code).to(DEV), st.state2.blocksize)
        qs.nested = True
    else:
        qs.absmax = torch.from_numpy(np.asarray(st.absmax, np.float32)).to(DEV)
        qs.nested = False
    return _Param(torch.from_numpy(packed).to(DEV).view(-1, 1), qs)


@pytest.mark.parametrize("nested", [True, False])
@pytest.mark.parametrize("shape", [(1536, 1536), (256, 1536), (1536, 512), (17920, 1536)])
def test_nf4_dequant_bit_exact(pkg, nested, shape):
    rng = np.random.default_rng(0)
    w = (rng.standard_normal(shape) * 0.02).astype(np.float16)
    packed, st = ON.quantize_nf4(w, compress_statistics=nested)
    want = torch.from_numpy(ON.dequantize_nf4(packed, st))
    weight = pkg.ops.NF4Weight(_device_state(packed, st))
    out = torch.empty(shape, device=DEV, dtype=torch.float16)
    weight.dequant_into(out)
    assert torch.equal(bits16(out), bits16(want))


def test_nf4_dequant_non_standard_code(pkg):
    rng = np.random.default_rng(3)
    packed = rng.integers(0, 256, 64 * 32, dtype=np.uint8)
    code = np.sort(rng.standard_normal(16).astype(np.float32))
    st = ON.QuantState(rng.random(64).astype(np.float32), (64, 64), code, 64)
    want = torch.from_numpy(ON.dequantize_nf4(packed, st, levels=code))
    weight = pkg.ops.NF4Weight(_device_state(packed, st))
    assert not weight.standard
    out = torch.empty((64, 64), device=DEV, dtype=torch.float16)
    weight.dequant_into(out)
    assert torch.equal(bits16(out), bits16(want))


def test_nf4_group_dequant_equals_separate(pkg):
    """q, k, v stacked back to back in one launch (NF4Group, engine.py:112-157) equals three
    separate launches and the oracle with per-segment offsets."""
    rng = np.random.default_rng(1)
    ws = []
    for shape in ((1536, 1536), (256, 1536), (256, 1536)):
        w = (rng.standard_normal(shape) * 0.02).astype(np.float16)
        packed, st = ON.quantize_nf4(w)
        ws.append((packed, st, pkg.ops.NF4Weight(_device_state(packed, st))))
    group = pkg.ops.NF4Group.of([w for _, _, w in ws])
    assert group is not None and group.seg1 == 36864 and group.seg2 == 36864 + 6144
    out = pkg.ops.dequant([w for _, _, w in ws], torch.device(DEV))
    want = torch.cat([torch.from_numpy(ON.dequantize_nf4(p, s)) for p, s, _ in ws])
    assert torch.equal(bits16(out), bits16(want))


def test_nf4_block_scales_equal_oracle(pkg):
    """qlora_nf4_block_scales (the fused GEMM's scale operand) equals the oracle's per-block
    scale bit for bit: a q|k|v group with three double-quant offsets by segment, a single
    nested weight, and a plain fp32 absmax (returned as is)."""
    rng = np.random.default_rng(11)
    ws = []
    for shape in ((1536, 1536), (256, 1536), (256, 1536)):
        w = (rng.standard_normal(shape) * 0.02).astype(np.float16)
        packed, st = ON.quantize_nf4(w)
        ws.append((packed, st, pkg.ops.NF4Weight(_device_state(packed, st))))
    group = pkg.ops.NF4Group.of([w for _, _, w in ws])
    want = np.concatenate([ON.block_scales(st) for _, st, _ in ws])
    got = group.block_scales().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert group.block_scales() is group.block_scales()  # formed once
    single = ws[1][2].block_scales().cpu().numpy()
    assert np.array_equal(single.view(np.uint32), ON.block_scales(ws[1][1]).view(np.uint32))
    w = (rng.standard_normal((256, 512)) * 0.02).astype(np.float16)
    packed, st = ON.quantize_nf4(w, compress_statistics=False)
    plain = pkg.ops.NF4Weight(_device_state(packed, st))
    assert plain.block_scales() is plain.absmax


@pytest.mark.parametrize("mix", ["layer", "ragged", "32"])
def test_nf4_dequant_many_equals_oracle(pkg, mix):
    """One qlora_nf4_dequant_many launch over several weights (a layer's q|k|v group, o,
    gate|up group and down; or ragged sizes, plain absmax and a non-standard code mixed in)
    equals the oracle bit for bit for every weight."""
    rng = np.random.default_rng(7)

    def make(shape, nested=True, code=None):
        w = (rng.standard_normal(shape) * 0.02).astype(np.float16)
        if code is None:
            packed, st = ON.quantize_nf4(w, compress_statistics=nested)
            return packed, st, ON.dequantize_nf4(packed, st)
        packed = rng.integers(0, 256, shape[0] * shape[1] // 2, dtype=np.uint8)
        st = ON.QuantState(rng.random(shape[0] * shape[1] // 64).astype(np.float32), shape,
                           code, 64)
        return packed, st, ON.dequantize_nf4(packed, st, levels=code)

    if mix == "layer":
        parts = [[make((1536, 1536)), make((256, 1536)), make((256, 1536))], [make((1536, 1536))],
                 [make((8960, 1536)), make((8960, 1536))], [make((1536, 8960))]]
    elif mix == "ragged":
        code = np.sort(rng.standard_normal(16).astype(np.float32))
        parts = [[make((64, 64))], [make((300, 512), nested=False)], [make((8, 64), code=code)],
                 [make((64, 1536)), make((256, 1536))]]
    else:  # the most one launch takes (eight layers' weights), sizes and formats mixed
        code = np.sort(rng.standard_normal(16).astype(np.float32))
        parts = []
        for i in range(32):
            rows = int(rng.integers(1, 40)) * 8
            kind = i % 4
            parts.append([make((rows, 512), nested=kind != 1, code=code if kind == 2 else None)]
                         if kind != 3 else [make((64 * (1 + i % 3), 256)), make((64, 256))])
    items, wants = [], []
    for grp in parts:
        ws = [pkg.ops.NF4Weight(_device_state(p, st)) for p, st, _ in grp]
        items.append(ws[0] if len(ws) == 1 else pkg.ops.NF4Group.of(ws))
        assert items[-1] is not None
        wants.append(torch.from_numpy(np.concatenate([d for _, _, d in grp])))
    outs = pkg.ops.dequant_many(items, torch.device(DEV))
    assert len(outs) == len(items)
    if mix == "32":
        with pytest.raises(ValueError):
            pkg.ops.dequant_many(items + items[:1], torch.device(DEV))
    for out, want in zip(outs, wants):
        assert torch.equal(bits16(out), bits16(want))


def _oracle_state(qs):
    return ON.QuantState(qs.absmax.cpu().numpy(), tuple(qs.shape), qs.code.cpu().numpy(), 64,
                         offset=np.float32(qs.offset.item()),
                         state2=ON.QuantState2(qs.state2.absmax.cpu().numpy(),
                                               qs.state2.code.cpu().numpy(), 256))


@pytest.mark.parametrize("shape", [(3, 64), (64, 64), (1536, 1536), (1536, 8960)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("nested", [True, False])
def test_gpu_quantizer_matches_oracle(pkg, shape, dtype, nested):
    """qlora_nf4_quantize(_stats) against the oracle's restatement of bitsandbytes' quantiser,
    bit for bit: packed codes, absmax (or its 8-bit codes, absmax2 and the offset), over block
    counts below one workgroup, with partial 256-blocks and with a two-level offset sum; the
    first block all zeros, the second holding every NF4 threshold exactly."""
    g = torch.Generator().manual_seed(shape[0] + shape[1])
    w = (torch.randn(shape, generator=g) * 0.03).to(dtype)
    flat = w.view(-1)
    flat[:64] = 0
    if flat.numel() >= 128:
        flat[64] = 1.0
        flat[65:80] = torch.from_numpy(ON.NF4_MIDS.astype(np.float32)).to(dtype)
    print(f"quantize shape={shape} dtype={dtype} nested={nested}", flush=True)
    param = pkg.quant.quantize_nf4(w.to(DEV), compress_statistics=nested)
    torch.cuda.synchronize()
    packed, st = ON.quantize_nf4(w.numpy() if dtype == torch.float32 else w.numpy(),
                                 compress_statistics=nested)
    assert np.array_equal(param.data.view(-1).cpu().numpy(), packed)
    qs = param.quant_state
    if nested:
        assert np.array_equal(qs.absmax.cpu().numpy(), st.absmax)
        assert np.array_equal(qs.state2.absmax.cpu().numpy(), st.state2.absmax)
        assert np.float32(qs.offset.item()) == st.offset
        assert np.array_equal(qs.state2.code.cpu().numpy(), st.state2.code)
    else:
        assert np.array_equal(qs.absmax.cpu().numpy(), st.absmax)


def test_quantizer_bytes_dequantize_like_oracle(pkg):
    """The package's GPU quantiser produces bitsandbytes-layout bytes that the HIP dequant and
    the oracle dequant read identically."""
    torch.manual_seed(0)
    w = (torch.randn(512, 1536, device=DEV) * 0.02).half()
    param = pkg.quant.quantize_nf4(w)
    out = torch.empty_like(w)
    pkg.ops.NF4Weight(param).dequant_into(out)
    st = _oracle_state(param.quant_state)
    want = torch.from_numpy(ON.dequantize_nf4(param.data.cpu().numpy(), st))
    assert torch.equal(bits16(out), bits16(want))
    assert (out.float() - w.float()).abs().max() < 0.02


@pytest.mark.parametrize("nelem,G,vec,p", [(4 * 37 * 1536, 524288, 4, 0.05),
                                           (3 * 5 * 64, 1024, 8, 0.1),
                                           (2 * 300 * 1536, 40960, 4, 0.1)])
def test_dropout_keep_matches_oracle(pkg, nelem, G, vec, p):
    seed, ctr = -(2**63) + 12345, 2**32 + 7
    got = pkg.ops.keep_mask(nelem, seed, ctr, G, p, vec, DEV).cpu().numpy()
    want = OP.keep_mask_call(nelem, seed, ctr, G, np.float32(1 - p), vec)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("shape,dtype,p", [((4, 37, 1536), torch.float32, 0.05),
                                           ((2, 300, 1536), torch.float32, 0.1),
                                           ((1, 7, 1536), torch.float32, 0.25),
                                           ((3, 5, 64), torch.float16, 0.1),
                                           ((4, 512, 1536), torch.float16, 0.05)])
def test_dropout_masks_are_torchs(pkg, shape, dtype, p):
    """The LoRA dropout masks are PyTorch-ROCm's own: TorchDropout.draw takes the generator's
    state as nn.Dropout would and advances it the same way, and the kernel's mask from it is the
    one F.dropout draws, bit for bit (the reference's check, test_kernels.py:67-90)."""
    torch.cuda.manual_seed(1234)
    drop = pkg.ops.TorchDropout(torch.device(DEV), dtype)
    nelem = math.prod(shape)
    for _ in range(3):
        state = drop.gen.get_state()
        seed, ctr, threads = drop.draw(nelem)
        after = drop.gen.get_offset()
        drop.gen.set_state(state)
        ref = torch.nn.functional.dropout(torch.ones(shape, device=DEV, dtype=dtype), p,
                                          training=True) != 0
        assert drop.gen.get_offset() == after
        got = pkg.ops.keep_mask(nelem, seed, ctr, threads, p, drop.vec, DEV)
        assert torch.equal(got, ref.reshape(-1))


def test_dropout_self_check(pkg):
    """The first-step self-check of the engine (engine.py:807-828) passes on this GPU."""
    drop = pkg.ops.TorchDropout(torch.device(DEV), torch.float32)
    before = drop.gen.get_offset()
    assert drop.check(4, 64, 1536, 0.05)
    assert drop.gen.get_offset() == before  # the default generator is not touched


class _Spec:
    eps = 1e-6
    HQ, HKV, D = 12, 2, 128


class _Packed:
    def __init__(self, p):
        self.dropout_p = p


@pytest.mark.parametrize("nparts,n,H", [(1, 37, 1536), (2, 5, 100), (5, 2304, 1536),
                                         (16, 9, 896), (4, 0, 1536)])
def test_rms_bwd_sums_split_slices(pkg, nparts, n, H):
    """dy given as S split-K slices (fp32 [S, n, H]): the backward equals the one given fp16 of
    their sum in slice order, bit for bit, for every slice count the GEMM plan uses (and 1, 16
    and no rows), with and without the forward's sum formed in the kernel."""
    g = torch.Generator().manual_seed(nparts + n)
    x = torch.randn(n, H, generator=g) * 3
    delta = torch.randn(n, H, generator=g).half()
    w = (torch.rand(H, generator=g) + 0.5).half()
    packed = _Packed(0.0)
    xsum, _, _, _, rstd = pkg.ops._rms_fwd(_Spec, x.to(DEV), w.to(DEV), packed,
                                           delta=delta.to(DEV))
    parts = torch.randn(nparts, n, H, generator=g).to(DEV)
    s = parts[0].clone()
    for k in range(1, nparts):
        s = s + parts[k]
    dres = torch.randn(n, H, generator=g).to(DEV)
    want = pkg.ops._rms_bwd(_Spec, s.half(), xsum, rstd, w.to(DEV), packed, dres=dres)
    got = pkg.ops._rms_bwd(_Spec, None, xsum, rstd, w.to(DEV), packed, dres=dres,
                           dy_parts=parts)
    got2 = pkg.ops._rms_bwd(_Spec, None, x.to(DEV), None, w.to(DEV), packed, dres=dres,
                            xdelta=delta.to(DEV), dy_parts=parts)
    assert torch.equal(got, want) and torch.equal(got2, want)


@pytest.mark.parametrize("n,H,wdtype", [(37, 1536, torch.float32), (5, 100, torch.float32),
                                        (2304, 1536, torch.float16), (3, 50, torch.float16),
                                        (7, 3584, torch.float32), (9, 896, torch.float32),
                                        (4, 256, torch.float16)])
def test_rms_forward_backward(pkg, n, H, wdtype):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(n, H, generator=g) * 3
    delta = torch.randn(n, H, generator=g).half()
    w = (torch.rand(H, generator=g) + 0.5).to(wdtype)
    p = 0.25
    tok = torch.arange(n) * 3 + 1
    G, seed, ctrs = 40960, 77, (11, 12)
    packed = _Packed(p)
    packed.tok = tok.to(DEV)
    packed.drop_seed, packed.drop_threads, packed.drop_vec = seed, G, 4
    xsum, y, yq, yv, rstd = pkg.ops._rms_fwd(_Spec, x.to(DEV), w.to(DEV), packed,
                                             delta=delta.to(DEV), seeds=ctrs, drop_q=True,
                                             drop_v=True)
    o = O.rms_fwd(x, w, _Spec.eps, delta=delta, tok=tok, p=p, seed=seed, ctrs=ctrs, G=G,
                  vec=4, drop_q=True, drop_v=True)
    close(xsum, o[0], 1e-6)
    close(y, o[1], 2e-3)
    assert torch.equal((yq != 0).cpu(), o[2] != 0) and torch.equal((yv != 0).cpu(), o[3] != 0)
    close(yq, o[2], 2e-3)
    close(yv, o[3], 2e-3)
    close(rstd, o[4], 1e-5)
    # the same seeds regenerate the same masks
    _, _, yq2, yv2, _ = pkg.ops._rms_fwd(_Spec, xsum, w.to(DEV), packed, write_y=False,
                                         seeds=ctrs, drop_q=True, drop_v=True)
    assert torch.equal(yq, yq2) and torch.equal(yv, yv2)

    dy = torch.randn(n, H, generator=g).half()
    tq = torch.randn(n, H, generator=g).half()
    tv = torch.randn(n, H, generator=g).half()
    dres = torch.randn(n, H, generator=g)
    dx = pkg.ops._rms_bwd(_Spec, dy.to(DEV), xsum, rstd, w.to(DEV), packed, dres=dres.to(DEV),
                          tq=tq.to(DEV), tv=tv.to(DEV), seeds=ctrs, grad_scale=0.5)
    want = O.rms_bwd(dy, o[0], o[4], w, dres=dres, tq=tq, tv=tv, tok=tok, p=p, seed=seed,
                     ctrs=ctrs, G=G, vec=4, grad_scale=0.5)
    close(dx, want, 1e-4)
    # a row-strided dy (a column slice of a wider buffer, kernels.py:187)
    wide = torch.zeros(n, H + 8, dtype=torch.float16, device=DEV)
    wide[:, :H] = dy.to(DEV)
    dx2 = pkg.ops._rms_bwd(_Spec, wide[:, :H], xsum, rstd, w.to(DEV), packed, dres=dres.to(DEV),
                           tq=tq.to(DEV), tv=tv.to(DEV), seeds=ctrs, grad_scale=0.5)
    assert torch.equal(dx, dx2) or (dx - dx2).abs().max() < 1e-6
    # the optional fp16 copy is exactly fp16(dx) (RNE), dx itself unchanged
    dx16 = torch.empty(n, H, dtype=torch.float16, device=DEV)
    dx3 = pkg.ops._rms_bwd(_Spec, dy.to(DEV), xsum, rstd, w.to(DEV), packed, dres=dres.to(DEV),
                           tq=tq.to(DEV), tv=tv.to(DEV), seeds=ctrs, grad_scale=0.5, out16=dx16)
    assert torch.equal(dx3, dx)
    assert torch.equal(dx16.view(torch.int16), dx.half().view(torch.int16))
    # the input given as x + delta (the forward's sum and rstd formed in the backward kernel):
    # the same bits as from the forward's xsum and rstd
    dx8 = pkg.ops._rms_bwd(_Spec, dy.to(DEV), x.to(DEV), None, w.to(DEV), packed,
                           dres=dres.to(DEV), tq=tq.to(DEV), tv=tv.to(DEV), seeds=ctrs,
                           grad_scale=0.5, xdelta=delta.to(DEV))
    assert torch.equal(dx8, dx)
    dxn = pkg.ops._rms_bwd(_Spec, dy.to(DEV), xsum, rstd, w.to(DEV), packed, dres=dres.to(DEV))
    dxn2 = pkg.ops._rms_bwd(_Spec, dy.to(DEV), x.to(DEV), None, w.to(DEV), packed,
                            dres=dres.to(DEV), xdelta=delta.to(DEV))
    assert torch.equal(dxn, dxn2)
    # dy given as split-K slices: fp16 of their sum in slice order, the same bits as dy itself
    parts = torch.randn(3, n, H, generator=g).to(DEV)
    dy16 = ((parts[0] + parts[1]) + parts[2]).half()
    dxp = pkg.ops._rms_bwd(_Spec, dy16, xsum, rstd, w.to(DEV), packed, dres=dres.to(DEV))
    dxp2 = pkg.ops._rms_bwd(_Spec, None, x.to(DEV), None, w.to(DEV), packed, dres=dres.to(DEV),
                            xdelta=delta.to(DEV), dy_parts=parts)
    assert torch.equal(dxp, dxp2)
    # the masks stored as bits by the forward: the oracle's masks, the same outputs, and a
    # backward that reads them equals the one that draws them again, bit for bit
    kb = torch.full(pkg.ops.keep_bits_shape(n, H), 0xAA, dtype=torch.uint8, device=DEV)
    _, y4, yq4, yv4, _ = pkg.ops._rms_fwd(_Spec, x.to(DEV), w.to(DEV), packed,
                                          delta=delta.to(DEV), seeds=ctrs, drop_q=True,
                                          drop_v=True, keep=kb)
    assert torch.equal(y4, y) and torch.equal(yq4, yq) and torch.equal(yv4, yv)
    masks = [O._keep(tok, H, n, seed, c, G, np.float32(1 - p), 4) for c in ctrs]
    assert torch.equal(kb.cpu(), _pack_keep(masks, n, H))
    dx5 = pkg.ops._rms_bwd(_Spec, dy.to(DEV), xsum, rstd, w.to(DEV), packed, dres=dres.to(DEV),
                           tq=tq.to(DEV), tv=tv.to(DEV), seeds=ctrs, grad_scale=0.5, keep=kb)
    assert torch.equal(dx5, dx)
    # a recompute reads the stored bits instead of drawing the masks: the same outputs; bits
    # that differ from the draw show through (all zero: every dropped copy zero)
    _, y6, yq6, yv6, _ = pkg.ops._rms_fwd(_Spec, x.to(DEV), w.to(DEV), packed,
                                          delta=delta.to(DEV), seeds=ctrs, drop_q=True,
                                          drop_v=True, keep_in=kb)
    assert torch.equal(y6, y) and torch.equal(yq6, yq) and torch.equal(yv6, yv)
    _, _, yq7, yv7, _ = pkg.ops._rms_fwd(_Spec, x.to(DEV), w.to(DEV), packed,
                                         delta=delta.to(DEV), seeds=ctrs, drop_q=True,
                                         drop_v=True, keep_in=torch.zeros_like(kb))
    assert not yq7.any() and not yv7.any()


def _pack_keep(masks, n, H):
    """bool masks [n, H] (q, v) -> the keep-bit layout u8 [n, 2, ceil(H / 4)]."""
    kb = (H + 3) // 4
    out = torch.zeros(n, 2, kb, dtype=torch.int32)
    for m, mask in enumerate(masks):
        padded = torch.zeros(n, 4 * kb, dtype=torch.int32)
        padded[:, :H] = mask.to(torch.int32)
        q = padded.view(n, kb, 4)
        out[:, m] = q[..., 0] | (q[..., 1] << 1) | (q[..., 2] << 2) | (q[..., 3] << 3)
    return out.to(torch.uint8)


@pytest.mark.parametrize("n,H", [(37, 1536), (5, 100), (3, 50)])
def test_rms_dropout_p0_is_identity(pkg, n, H):
    """p = 0 keeps every element (PyTorch's dropout returns its input; PEFT: nn.Identity), in
    both directions and in the stored bits."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(n, H, generator=g)
    w = torch.rand(H, generator=g) + 0.5
    packed = _Packed(0.0)
    packed.tok = (torch.arange(n) * 5).to(DEV)
    packed.drop_seed, packed.drop_threads, packed.drop_vec = 3, 4096, 4
    kb = torch.zeros(pkg.ops.keep_bits_shape(n, H), dtype=torch.uint8, device=DEV)
    _, y, yq, yv, rstd = pkg.ops._rms_fwd(_Spec, x.to(DEV), w.to(DEV), packed, seeds=(1, 2),
                                          drop_q=True, drop_v=True, keep=kb)
    assert torch.equal(yq, y) and torch.equal(yv, y)
    assert torch.equal(kb.cpu(), _pack_keep([torch.ones(n, H, dtype=torch.bool)] * 2, n, H))
    dy, tq, tv = (torch.randn(n, H, generator=g).half() for _ in range(3))
    dx = pkg.ops._rms_bwd(_Spec, dy.to(DEV), x.to(DEV), rstd, w.to(DEV), packed, tq=tq.to(DEV),
                          tv=tv.to(DEV), seeds=(1, 2))
    want = O.rms_bwd(dy, x, rstd.cpu(), w, tq=tq, tv=tv, tok=packed.tok.cpu(), p=0.0, seed=3,
                     ctrs=(1, 2), G=4096, vec=4)
    close(dx, want, 1e-4)


@pytest.mark.parametrize("numel", [4, 1536 * 37, 2560 * 1536])
def test_resid_add(pkg, numel):
    """h3 = h2 + fp32(d) bit-exact (engine.py:1048-1051); in place too."""
    g = torch.Generator(device=DEV).manual_seed(numel)
    a = torch.randn(numel, generator=g, device=DEV)
    d = torch.randn(numel, generator=g, device=DEV).half()
    out = pkg.ops._resid_add(a, d)
    assert torch.equal(out, a + d.float())
    b = a.clone()
    pkg.ops._resid_add(b, d, out=b)
    assert torch.equal(b, out)


@pytest.mark.parametrize("kv_heads", [None, 2])
def test_qkv_rope_forward_backward(pkg, kv_heads):
    g = torch.Generator().manual_seed(0)
    n, HQ, HKV, D, s = 23, 12, 2, 128, 2.0
    C = (HQ + 2 * HKV) * D
    qkv = torch.randn(n, C, generator=g).half()
    lq = torch.randn(n, HQ * D, generator=g).half()
    lv = torch.randn(n, HKV * D, generator=g).half()
    pos = torch.randint(0, 500, (n,), generator=g, dtype=torch.int32)
    cos, sin = O.rope_tables(512, D, 1e6)

    class P:
        pass

    packed = P()
    packed.cos, packed.sin, packed.pos = cos.to(DEV), sin.to(DEV), pos.to(DEV)
    q, k, v = pkg.ops._rope_fwd(_Spec, qkv.to(DEV), lq.to(DEV), lv.to(DEV), packed, s,
                                kv_heads=kv_heads)
    qo, ko, vo = O.rope_fwd(qkv, lq, lv, cos, sin, pos, HQ, HKV, D, s, kv_heads=kv_heads)
    close(q, qo, 2e-3)
    close(k, ko, 2e-3)
    close(v, vo, 2e-3)
    kh = HQ if kv_heads is None else kv_heads
    dq = torch.randn(n, HQ, D, generator=g).half()
    dk = torch.randn(n, kh, D, generator=g).half()
    dv = torch.randn(n, kh, D, generator=g).half()
    dqkv = pkg.ops._rope_bwd(_Spec, dq.to(DEV), dk.to(DEV), dv.to(DEV), packed)
    want = O.rope_bwd(dq, dk, dv, cos, sin, pos, HQ, HKV, D)
    close(dqkv[:, :HQ * D], want[:, :HQ * D], 3e-3)
    close(dqkv[:, HQ * D:], want[:, HQ * D:], 1e-2)
    # no LoRA: q, v are the plain projections
    q2, _, v2 = pkg.ops._rope_fwd(_Spec, qkv.to(DEV), None, None, packed, s)
    qo2, _, vo2 = O.rope_fwd(qkv, None, None, cos, sin, pos, HQ, HKV, D, s)
    close(q2, qo2, 2e-3)
    close(v2, vo2, 2e-3)


@pytest.mark.parametrize("n,I", [(9, 8960), (3, 1000), (2, 37)])
def test_glu_forward_backward(pkg, n, I):
    g = torch.Generator().manual_seed(0)
    gu = (torch.randn(n, 2 * I, generator=g) * 3).half()
    m = pkg.ops._glu_fwd(gu.to(DEV), I)
    close(m, O.glu_fwd(gu, I), 2e-3)
    dm = torch.randn(n, I, generator=g).half()
    work = gu.to(DEV)
    pkg.ops._glu_bwd(dm.to(DEV), work, I)
    want = O.glu_bwd(dm, gu, I)
    close(work[:, :I], want[:, :I], 1e-2)
    close(work[:, I:], want[:, I:], 1e-2)


def _ulps(a, b):
    """Distance in fp16 units in the last place between two fp16 tensors (same sign order)."""
    def key(t):
        i = t.view(torch.int16).to(torch.int32)
        return torch.where(i < 0, -(i & 0x7FFF), i)
    return (key(a) - key(b)).abs()


def test_glu_forward_ulp_bound_config2(pkg):
    """SwiGLU at config 2's size ([2048, 8960] out of gu ~ N(0, 1) fp16) forms the sigmoid from
    the hardware exp2 and reciprocal: every output is within 1 fp16 ulp of the oracle's
    fp32 silu (accurate exp) rounded once, and under 0.1 % of outputs differ at all."""
    I = 8960
    g = torch.Generator().manual_seed(7)
    gu = torch.randn(2048, 2 * I, generator=g).half()
    m = pkg.ops._glu_fwd(gu.to(DEV), I).cpu()
    want = O.glu_fwd(gu, I)
    d = _ulps(m, want)
    assert int(d.max()) <= 1
    assert float((d > 0).float().mean()) < 1e-3


@pytest.mark.parametrize("V", [151936, 5000, 4093])
def test_lm_head_ce(pkg, V):
    g = torch.Generator().manual_seed(0)
    n = 37
    logits = (torch.randn(n, V, generator=g) * 4).half()
    target = torch.randint(0, V, (n,), generator=g)
    target[::5] = -100
    target[1] = logits[1].float().argmax()
    loss_o, ent_o, cor_o, grad_o = O.ce(logits, target)
    work = logits.to(DEV)
    loss = torch.empty(n, device=DEV)
    ent = torch.empty(n, device=DEV)
    correct = torch.empty(n, device=DEV, dtype=torch.int32)
    pkg.ops._ce(work, target.to(DEV), loss, ent, correct)
    close(loss, loss_o, 1e-4)
    close(ent, ent_o, 1e-3)
    assert torch.equal(correct.cpu(), cor_o)
    assert correct[1].item() == 1
    close(work, grad_o, 1e-3)


def _piece_run(pkg, logits, weight, targets, n_sup, H, piece=8192):
    n, V = logits.shape
    state = torch.tensor([float("-inf"), 0.0, 0.0, float("-inf")], device=DEV).repeat(n, 1)
    best_idx = torch.zeros(n, device=DEV, dtype=torch.int32)
    xt = torch.zeros(n, device=DEV)
    alpha = torch.empty(max(n_sup, 1), device=DEV)
    acc = torch.zeros((max(n_sup, 1), H), device=DEV)
    wt = torch.zeros((max(n_sup, 1), H), device=DEV, dtype=torch.float16)
    for v0 in range(0, V, piece):
        width = min(piece, V - v0)
        part = logits[:, v0:v0 + width].contiguous()
        w = weight[v0:v0 + width].contiguous()
        pkg.ops._ce_piece(part, w, targets, state, best_idx, xt, alpha, wt, v0, n_sup)
        acc[:n_sup] = acc[:n_sup] * alpha[:n_sup, None] + part[:n_sup].float() @ w.float()
    loss = torch.empty(n, device=DEV)
    ent = torch.empty(n, device=DEV)
    cor = torch.empty(n, device=DEV, dtype=torch.int32)
    dh = torch.empty((max(n_sup, 1), H), device=DEV, dtype=torch.float16)
    pkg.ops._ce_finish(state, best_idx, xt, targets, loss, ent, cor, acc, wt, dh, n_sup)
    return loss, ent, cor, dh


@pytest.mark.parametrize("n,n_prompt", [(300, 120), (37, 37), (5, 0)])
def test_piece_kernels_match_ce_kernel(pkg, n, n_prompt):
    """On the same logits the piece-by-piece kernels give the whole-row kernel's loss, entropy
    and accuracy to the bit, and dh within the one-GEMM error (test_host_head.py:38-88)."""
    V, H = 151936, 1536
    g = torch.Generator().manual_seed(n)
    h = torch.randn((n, H), generator=g) * 2.0
    weight = (torch.randn((V, H), generator=g) * 0.03).half().to(DEV)
    targets = torch.randint(0, V, (n,), generator=g)
    targets[n - n_prompt:] = -100  # supervised rows first (head order)
    n_sup = n - n_prompt
    targets = targets.to(DEV)
    hn = h.half().to(DEV)
    logits = (hn.float() @ weight.float().t()).half()
    ref = logits.clone()
    loss_a = torch.empty(n, device=DEV)
    ent_a = torch.empty(n, device=DEV)
    cor_a = torch.empty(n, device=DEV, dtype=torch.int32)
    pkg.ops._ce(ref, targets, loss_a, ent_a, cor_a)
    dh_a = (ref[:n_sup].float() @ weight.float()).half()
    loss_b, ent_b, cor_b, dh_b = _piece_run(pkg, logits, weight, targets, n_sup, H)
    assert torch.equal(loss_a, loss_b)
    assert torch.equal(ent_a, ent_b)
    assert torch.equal(cor_a, cor_b)
    if n_sup:
        exact = (torch.softmax(logits[:n_sup].double(), -1)
                 - torch.nn.functional.one_hot(targets[:n_sup], V).double()) @ weight.double()
        err_a = (dh_a.double() - exact).norm() / exact.norm()
        err_b = (dh_b[:n_sup].double() - exact).norm() / exact.norm()
        assert err_b < 1e-3 and err_b <= 1.5 * err_a + 1e-6, (err_a.item(), err_b.item())


@pytest.mark.parametrize("V", [151936, 5000])
def test_ce_leaves_unsupervised_rows(pkg, V):
    """zero_unsupervised=False (the step's head, whose dh product reads the supervised rows
    only): the statistics and the supervised rows' gradient are those of the zeroing form bit
    for bit, and the rows of ignored tokens keep their logits."""
    n = 300
    g = torch.Generator().manual_seed(V)
    targets = torch.randint(0, V, (n,), generator=g)
    targets[::3] = -100
    targets = targets.to(DEV)
    logits = (torch.randn(n, V, generator=g) * 3).half().to(DEV)
    out = {}
    for zero in (True, False):
        work = logits.clone()
        st = (torch.empty(n, device=DEV), torch.empty(n, device=DEV),
              torch.empty(n, device=DEV, dtype=torch.int32))
        pkg.ops._ce(work, targets, *st, zero_unsupervised=zero)
        out[zero] = (work, *st)
    sup = targets >= 0
    for a, b in zip(out[True][1:], out[False][1:]):
        assert torch.equal(a, b)
    assert torch.equal(out[True][0][sup], out[False][0][sup])
    assert torch.equal(out[False][0][~sup], logits[~sup])
    assert not out[True][0][~sup].any()


def test_ce_kernels_take_the_target_logit_before_the_row_is_overwritten(pkg):
    """Over many launches every token's loss is logsumexp - its target's logit
    (test_host_head.py:91-125: the in-place gradient write must not race the target read)."""
    V, H, n = 151936, 64, 1024
    g = torch.Generator().manual_seed(5)
    targets = torch.randint(0, V, (n,), generator=g)
    targets[724:] = -100
    targets = targets.to(DEV)
    logits = (torch.randn(n, V, generator=g) * 3).half().to(DEV)
    lf = logits.float()
    exact = torch.logsumexp(lf, -1) - lf.gather(1, targets.clamp(min=0)[:, None])[:, 0]
    exact = torch.where(targets >= 0, exact, 0.0)
    for _ in range(10):
        loss = torch.empty(n, device=DEV)
        ent = torch.empty(n, device=DEV)
        cor = torch.empty(n, device=DEV, dtype=torch.int32)
        pkg.ops._ce(logits.clone(), targets, loss, ent, cor)
        assert (loss - exact).abs().max() < 1e-3


@pytest.mark.parametrize("n,H,Nq,Nv", [(300, 1536, 1536, 256), (1, 1536, 1536, 256),
                                       (77, 256, 256, 128), (4100, 896, 896, 128),
                                       (33, 3584, 3584, 512)])
def test_lora_bwd_rows(pkg, n, H, Nq, Nv, r=16):
    """dx = fp16(fp16(g B) s), t = fp16(dx A) for both adapters against fp64 of the same
    roundings (engine.py:1326-1330); g are column slices of one fused gradient (row stride C)."""
    g = torch.Generator().manual_seed(n + r)
    C = Nq + 2 * Nv
    dqkv = torch.randn(n, C, generator=g).half()
    aq = (torch.randn(r, H, generator=g) * 0.05).half()
    av = (torch.randn(r, H, generator=g) * 0.05).half()
    bq = (torch.randn(Nq, r, generator=g) * 0.05).half()
    bv = (torch.randn(Nv, r, generator=g) * 0.05).half()
    s = 2.0
    qc, vc = slice(0, Nq), slice(Nq + Nv, C)
    tr = [w.t().contiguous().to(DEV) for w in (aq, bq, av, bv)]
    dxq, dxv, tq, tv = pkg.ops._lora_bwd_rows(dqkv.to(DEV), qc, vc, *tr, s)
    for cols, b, a, dx, t in ((qc, bq, aq, dxq, tq), (vc, bv, av, dxv, tv)):
        gd = dqkv[:, cols].double()
        want = ((gd @ b.double()).half().double() * s).half()
        # fp16 GEMM outputs may differ from fp64 in the last bit (summation order)
        close(dx, want, 2e-3 * want.abs().max().item())
        tw = (dx.cpu().double() @ a.double()).half()
        close(t, tw, 2e-3 * tw.abs().max().item())
    dq2, dv2, t0, t1 = pkg.ops._lora_bwd_rows(dqkv.to(DEV), qc, vc, *tr, s, need_t=False)
    assert t0 is None and t1 is None
    assert torch.equal(dq2, dxq) and torch.equal(dv2, dxv)


@pytest.mark.parametrize("n,H,Nq,Nv", [(300, 1536, 1536, 256), (1, 1536, 1536, 256),
                                       (77, 256, 256, 128), (4100, 896, 896, 128),
                                       (33, 3584, 3584, 512), (2540, 1536, 1536, 256)])
def test_lora_fwd_rows(pkg, n, H, Nq, Nv, r=16):
    """x = fp16(a A^T), l = fp16(x B^T) for both adapters (engine.py:1088-1093) against fp64 of
    the same roundings."""
    g = torch.Generator().manual_seed(n + 1 + r)
    aq = torch.randn(n, H, generator=g).half()
    av = torch.randn(n, H, generator=g).half()
    Aq = (torch.randn(r, H, generator=g) * 0.05).half()
    Av = (torch.randn(r, H, generator=g) * 0.05).half()
    Bq = (torch.randn(Nq, r, generator=g) * 0.05).half()
    Bv = (torch.randn(Nv, r, generator=g) * 0.05).half()
    xq, xv, lq, lv = pkg.ops._lora_fwd_rows(aq.to(DEV), av.to(DEV), Aq.to(DEV), Bq.to(DEV),
                                            Av.to(DEV), Bv.to(DEV))
    for a, A, B, x, l in ((aq, Aq, Bq, xq, lq), (av, Av, Bv, xv, lv)):
        want = (a.double() @ A.double().t()).half()
        close(x, want, 2e-3 * want.abs().max().item())
        lw = (x.cpu().double() @ B.double().t()).half()
        close(l, lw, 2e-3 * lw.abs().max().item())


@pytest.mark.parametrize("n,H,Nq,Nv", [(300, 1536, 1536, 256), (1, 1536, 1536, 256),
                                       (129, 256, 256, 128), (4100, 896, 896, 128),
                                       (0, 256, 256, 128), (70, 250, 250, 66)])
def test_lora_grad(pkg, n, H, Nq, Nv, r=16):
    """dB = s g^T x and dA = dx^T a of both adapters (engine.py:1327, 1329) against fp64 sums of
    the same fp16 operands (fp32 accumulation: relative error ~ 1e-6 of the magnitudes). Widths
    that are multiples of 8 take the MFMA pass; (70, 250, 250, 66) has rows without whole
    16-byte chunks and takes the v_dot2 pass."""
    g = torch.Generator().manual_seed(n + 7 + r)
    C = Nq + 2 * Nv
    dqkv = torch.randn(n, C, generator=g).half()
    xs = [torch.randn(n, r, generator=g).half() for _ in range(4)]  # x_q, x_v, dx_q, dx_v
    aq = torch.randn(n, H, generator=g).half()
    av = torch.randn(n, H, generator=g).half()
    s = 2.0
    qc, vc = slice(0, Nq), slice(Nq + Nv, C)
    d = [t.to(DEV) for t in (dqkv, *xs, aq, av)]
    dA_q, dB_q, dA_v, dB_v = pkg.ops._lora_grad(d[0], qc, vc, d[1], d[2], d[5], d[6], d[3],
                                                d[4], s)
    for got, want in ((dB_q, s * dqkv[:, qc].double().t() @ xs[0].double()),
                      (dB_v, s * dqkv[:, vc].double().t() @ xs[1].double()),
                      (dA_q, xs[2].double().t() @ aq.double()),
                      (dA_v, xs[3].double().t() @ av.double())):
        assert got.dtype == torch.float32 and got.shape == want.shape
        scale = max(1.0, math.sqrt(max(n, 1))) * 8
        close(got, want, 1e-5 * scale)



@pytest.mark.parametrize("r", [8, 32, 64])
@pytest.mark.parametrize("n,H,Nq,Nv", [(300, 1536, 1536, 256), (33, 896, 896, 128)])
def test_lora_other_ranks(pkg, n, H, Nq, Nv, r):
    """The three LoRA kernels at ranks 8, 32 and 64 (PEFT's other common choices): the same
    fp64 checks as at rank 16."""
    print(f"lora rank {r} n={n} H={H}", flush=True)
    test_lora_fwd_rows(pkg, n, H, Nq, Nv, r)
    test_lora_bwd_rows(pkg, n, H, Nq, Nv, r)
    test_lora_grad(pkg, n, H, Nq, Nv, r)


def test_dequant_timed_form(pkg):
    """The timed form writes what the plain launch writes, and its events (recorded by the
    dispatch at the kernel's start and end) lie inside a pair recorded around the call."""
    import ctypes
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((1536, 1536)) * 0.02).astype(np.float16)
    packed, st = ON.quantize_nf4(w)
    item = pkg.ops.NF4Weight(_device_state(packed, st))
    want = pkg.ops.dequant_many([item], torch.device(DEV))[0]
    timer = pkg.profiling.LaunchTimer("qlora_nf4_dequant_many")
    outer0, outer1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with timer:
        outer0.record()
        got = pkg.ops.dequant_many([item], torch.device(DEV))[0]
        outer1.record()
    torch.cuda.synchronize()
    assert torch.equal(bits16(got), bits16(want))
    s = timer.summary()
    assert s["launches"] == 1 and 0 < s["avg_us"] <= outer0.elapsed_time(outer1) * 1e3


def test_event_bracketed_timer_excludes_the_spin(pkg):
    """An entry without a timed form (the RMSNorm forward) is bracketed by events behind a spin
    kernel: the launch still computes what an untimed launch computes, and its recorded
    duration is positive and shorter than the spin plus the launch measured around both."""
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(2048, 1536, generator=g) * 2).to(DEV)
    w = (torch.rand(1536, generator=g) + 0.5).to(DEV)
    packed = _Packed(0.0)
    _, want, _, _, _ = pkg.ops._rms_fwd(_Spec, x, w, packed)
    timer = pkg.profiling.LaunchTimer("qlora_rms_fwd", work=lambda a: 1.0, bound="hbm")
    outer0, outer1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with timer:
        outer0.record()
        _, got, _, _, _ = pkg.ops._rms_fwd(_Spec, x, w, packed)
        outer1.record()
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    s = timer.summary()
    outer_us = outer0.elapsed_time(outer1) * 1e3
    assert s["launches"] == 1 and 0 < s["avg_us"] < outer_us
