"""The fused NF4 dequant + MFMA GEMM (qlora_nf4_gemm): bit-exact decode, both orientations at the
step's shapes, every epilogue, ragged token counts, and the config-2 MLP forward/backward against
the oracle (1e-3 relative, fp16)."""

import numpy as np
import pytest
import torch

from oracle import ops as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _weight(pkg, shape, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = (torch.randn(shape, generator=g, device=DEV) * 0.02).half()
    return pkg.ops.NF4Weight(pkg.quant.quantize_nf4(w))


def _group(pkg, shapes, seed):
    return pkg.ops.NF4Group.of([_weight(pkg, s, seed + i) for i, s in enumerate(shapes)])


def rel_err(a, ref):
    a, ref = a.double(), ref.double()
    return ((a - ref).norm() / ref.norm().clamp_min(1e-30)).item()


@pytest.mark.parametrize("shape", [(1536, 1536), (2048, 1536), (1536, 8960)])
def test_decode_inside_gemm_is_bit_exact(pkg, shape):
    """With A = identity the product is the decoded weight itself (one exact fp32 term per
    output): NT gives W^T, NN gives W, both bit-equal to the standalone dequant."""
    L = pkg.linear
    w = _weight(pkg, shape, 0)
    ref = L.dequantize(w)
    N, K = shape
    eye_k = torch.eye(K, device=DEV, dtype=torch.float16)
    nt = L.nf4_gemm(eye_k, w, 0)
    assert torch.equal(nt.view(torch.int16), ref.t().contiguous().view(torch.int16))
    eye_n = torch.eye(N, device=DEV, dtype=torch.float16)
    nn = L.nf4_gemm(eye_n, w, 1)
    assert torch.equal(nn.view(torch.int16), ref.view(torch.int16))


def test_group_decode_bit_exact(pkg):
    """q|k|v stacked (three double-quant offsets by segment) decode inside the GEMM."""
    L = pkg.linear
    grp = _group(pkg, [(1536, 1536), (256, 1536), (256, 1536)], 5)
    ref = L.dequantize(grp)
    eye = torch.eye(2048, device=DEV, dtype=torch.float16)
    assert torch.equal(L.nf4_gemm(eye, grp, 1).view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("M", [2048, 2049, 37, 1])
@pytest.mark.parametrize("wshape", [(17920, 1536), (1536, 8960), (2048, 1536)])
def test_gemm_nt_nn_against_fp64(pkg, M, wshape):
    L = pkg.linear
    w = _weight(pkg, wshape, 1)
    wd = L.dequantize(w).double()
    g = torch.Generator(device=DEV).manual_seed(M)
    x = torch.randn(M, wshape[1], generator=g, device=DEV).half()
    y = L.nf4_gemm(x, w, 0)
    ref = x.double() @ wd.t()
    assert rel_err(y, ref) < 1e-3
    torch.testing.assert_close(y.double(), ref, rtol=2e-3, atol=2e-3 * ref.abs().max().item())
    dy = torch.randn(M, wshape[0], generator=g, device=DEV).half()
    dx = L.nf4_gemm(dy, w, 1)
    ref = dy.double() @ wd
    assert rel_err(dx, ref) < 1e-3
    torch.testing.assert_close(dx.double(), ref, rtol=2e-3, atol=2e-3 * ref.abs().max().item())


def test_epilogues(pkg):
    L = pkg.linear
    M = 300
    g = torch.Generator(device=DEV).manual_seed(9)
    # bias (the qkv projection)
    grp = _group(pkg, [(1536, 1536), (256, 1536), (256, 1536)], 7)
    wq = L.dequantize(grp).double()
    x = torch.randn(M, 1536, generator=g, device=DEV).half()
    bias = (torch.randn(2048, generator=g, device=DEV) * 0.1).half()
    y = L.nf4_gemm(x, grp, 0, epi=1, bias=bias)
    assert rel_err(y, x.double() @ wq.t() + bias.double()) < 1e-3
    # residual add in fp32 of the fp16-rounded product (h3 = h2 + d)
    wd = _weight(pkg, (1536, 8960), 8)
    m = torch.randn(M, 8960, generator=g, device=DEV).half()
    h2 = torch.randn(M, 1536, generator=g, device=DEV)
    d = L.nf4_gemm(m, wd, 0)
    h3 = L.nf4_gemm(m, wd, 0, epi=2, resid=h2)
    assert h3.dtype == torch.float32
    assert torch.equal(h3, h2 + d.float())
    # SwiGLU over gate|up without materialising it
    gu_w = _group(pkg, [(8960, 1536), (8960, 1536)], 10)
    mm = L.nf4_gemm(x, gu_w, 0, epi=3, swiglu_I=8960)
    gu = L.nf4_gemm(x, gu_w, 0, splits=1)  # the SwiGLU epilogue sums K in one slice
    assert torch.equal(mm, pkg.ops._glu_fwd(gu, 8960))
    # the same from the fp16 B path (gate and up rows placed per wavefront by the B loader)
    wgu = L.dequantize(gu_w)
    assert torch.equal(L.hgemm(x, wgu, 0, epi=3, swiglu_I=8960), mm)
    # fp32 A rounded to fp16 on load
    a32 = torch.randn(M, 1536, generator=g, device=DEV)
    assert torch.equal(L.nf4_gemm(a32, wd, 1), L.nf4_gemm(a32.half(), wd, 1))


@pytest.mark.parametrize("path", ["step", "fused"])
def test_mlp_up_path_config2(pkg, path):
    """x [2048, 1536] ~ N(0,1), NF4 [gate|up] [17920, 1536] and down
    [1536, 8960] from N(0, 0.02); h = silu(gate) * up, y = h W_d^T; backward w.r.t. x with
    dy ~ N(0,1), against the oracle's fp32 products of the same fp16 values. path "step": the
    projections as the step runs them (linear.nf4_linear*, whichever backend is the default);
    "fused": the fused NF4 GEMM kernel itself (SwiGLU epilogue, NT, NN)."""
    L = pkg.linear
    gu_w = _group(pkg, [(8960, 1536), (8960, 1536)], 20)
    wd = _weight(pkg, (1536, 8960), 22)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2048, 1536, generator=g).half()
    dy = torch.randn(2048, 1536, generator=g).half()
    h_o, y_o, dx_o = O.mlp(x, L.dequantize(gu_w).cpu(), L.dequantize(wd).cpu(), dy)
    xg, dyg = x.to(DEV), dy.to(DEV)
    if path == "step":
        h = L.nf4_linear_swiglu(xg, gu_w, 8960)
        y = L.nf4_linear(h, wd)
        dh = L.nf4_linear_t(dyg, wd)
        gu = L.nf4_linear(xg, gu_w)
        pkg.ops._glu_bwd(dh, gu, 8960)
        dx = L.nf4_linear_t(gu, gu_w)
    else:
        h = L.nf4_gemm(xg, gu_w, 0, epi=3, swiglu_I=8960)
        y = L.nf4_gemm(h, wd, 0)
        dh = L.nf4_gemm(dyg, wd, 1)
        gu = L.nf4_gemm(xg, gu_w, 0)
        pkg.ops._glu_bwd(dh, gu, 8960)
        dx = L.nf4_gemm(gu, gu_w, 1)
    for got, want in ((h, h_o), (y, y_o), (dx, dx_o)):
        assert rel_err(got.cpu(), want) < 1e-3


@pytest.mark.parametrize("splits", [1, 2, 3])
@pytest.mark.parametrize("mode", [0, 1])
def test_every_split(pkg, splits, mode):
    """Split-K settings (forced) against fp64, with the residual and bias epilogues through the
    split-K reduce, for the NF4 and the fp16-B kernels."""
    L = pkg.linear
    w = _weight(pkg, (1536, 2048), 31)
    wd16 = L.dequantize(w)
    wd = wd16.double()
    g = torch.Generator(device=DEV).manual_seed(splits * 7 + mode)
    M = 531
    if mode == 0:
        x = torch.randn(M, 2048, generator=g, device=DEV).half()
        ref = x.double() @ wd.t()
        bias = (torch.randn(1536, generator=g, device=DEV) * 0.1).half()
        y = L.nf4_gemm(x, w, 0, epi=1, bias=bias, splits=splits)
        assert rel_err(y, ref + bias.double()) < 1e-3
        assert torch.equal(L.hgemm(x, wd16, 0, epi=1, bias=bias, splits=splits), y)
        res = torch.randn(M, 1536, generator=g, device=DEV)
        h = L.nf4_gemm(x, w, 0, epi=2, resid=res, splits=splits)
        assert rel_err(h - res, ref) < 1e-3
    else:
        dy = torch.randn(M, 1536, generator=g, device=DEV)  # fp32 A, rounded to fp16 first
        ref = dy.half().double() @ wd
        y = L.nf4_gemm(dy, w, 1, splits=splits)
        assert rel_err(y, ref) < 1e-3
        assert torch.equal(L.hgemm(dy, wd16, 1, splits=splits), y)


@pytest.mark.parametrize("M", [2560, 1, 300])
@pytest.mark.parametrize("mode", [0, 1])
def test_fp16_b_gemm_equals_fused(pkg, M, mode):
    """qlora_gemm16 on the dequantized weight equals qlora_nf4_gemm on the NF4 weight bit for bit
    (same B values, same summation order) at the step's widest shapes, and both match fp64."""
    L = pkg.linear
    gu_w = _group(pkg, [(8960, 1536), (8960, 1536)], 40)
    wd16 = L.dequantize(gu_w)
    g = torch.Generator(device=DEV).manual_seed(M + mode)
    a = torch.randn(M, 1536 if mode == 0 else 17920, generator=g, device=DEV).half()
    fused = L.nf4_gemm(a, gu_w, mode)
    plain = L.hgemm(a, wd16, mode)
    assert torch.equal(fused, plain)
    ref = a.double() @ (wd16.double().t() if mode == 0 else wd16.double())
    assert rel_err(plain, ref) < 1e-3


def test_lm_head_shapes(pkg):
    """The lm_head products on the fp16 path: logits = hn E^T (N = 151,936) and G E (K =
    151,936, split-K) against fp64."""
    L = pkg.linear
    g = torch.Generator(device=DEV).manual_seed(11)
    E = (torch.randn(151936, 1536, generator=g, device=DEV) * 0.02).half()
    hn = torch.randn(300, 1536, generator=g, device=DEV).half()
    logits = L.hgemm(hn, E, 0)
    assert rel_err(logits, hn.double() @ E.double().t()) < 1e-3
    G = (torch.randn(300, 151936, generator=g, device=DEV) * 1e-3).half()
    dh = L.hgemm(G, E, 1)
    assert rel_err(dh, G.double() @ E.double()) < 1e-3


@pytest.mark.parametrize("epi", [0, 1, 2, 3])
def test_tile_major_order_equals_bnb_order(pkg, epi):
    """The fused GEMM over the weight's tile-major copy of codes and scales (the order its DMA
    reads in 1 KB runs) gives the results of the bitsandbytes order bit for bit: every NT
    epilogue, split-K, a ragged M; and the copy holds the same bytes."""
    L = pkg.linear
    M = 700
    if epi == 3:
        w = _group(pkg, [(8960, 1536), (8960, 1536)], 21)
        N = 8960
    else:
        w = _weight(pkg, (2048, 1536), 21)
        N = 2048
    g = torch.Generator(device=DEV).manual_seed(5)
    x = (torch.randn(M, 1536, generator=g, device=DEV) * 0.5).half()
    kw = {}
    if epi == 1:
        kw["bias"] = (torch.randn(N, generator=g, device=DEV) * 0.1).half()
    if epi == 2:
        kw["resid"] = torch.randn(M, N, generator=g, device=DEV)
    if epi == 3:
        kw["swiglu_I"] = 8960
    for splits in ([1] if epi == 3 else [1, 2]):
        a = L.nf4_gemm(x, w, 0, epi=epi, tiled=True, splits=splits, **kw)
        b = L.nf4_gemm(x, w, 0, epi=epi, tiled=False, splits=splits, **kw)
        assert torch.equal(a, b)
    codes, scales = pkg.ops.gemm_tiles(w, kw.get("swiglu_I", 0))
    assert torch.equal(torch.sort(codes).values, torch.sort(w.packed.reshape(-1)).values)
    assert torch.equal(torch.sort(scales).values, torch.sort(w.block_scales()).values)


@pytest.mark.parametrize("mode,epi", [(0, 0), (0, 1), (0, 2), (0, 3), (1, 0), (1, 2)])
def test_fp16_b_gemm_tail_slices(pkg, mode, epi):
    """One slice with a last round of at most 64 tiles: qlora_gemm16 given its workspace runs those
    tiles as K slices (partials summed in slice order, then the epilogue). The tail tiles agree
    with fp64 to fp16 rounding, every other output is the same bits as without the workspace
    (all tiles whole), for every epilogue and both orientations."""
    L = pkg.linear
    g = torch.Generator(device=DEV).manual_seed(40 + 10 * mode + epi)
    if epi == 3:  # SwiGLU, I = 8960: 2,600 rows -> 770 tiles, tiles 768-769 sliced
        M, N, K, I = 2600, 8960, 1536, 8960
        w = (torch.randn(2 * I, K, generator=g, device=DEV) * 0.02).half()
        tail_rows, tail_cols = slice(2304, M), slice(69 * 128, N)
    else:  # 2,048 columns, 8,348 rows -> 264 tiles, tiles 256-263 (column tile 7) sliced
        M, N, K = 8348, 2048, 1536
        w = (torch.randn(*((N, K) if mode == 0 else (K, N)), generator=g, device=DEV) *
             0.02).half()
        tail_rows, tail_cols = slice(25 * 256, M), slice(7 * 256, N)
    assert L.hgemm_workspace(M, N, K, epi, 1) > 0
    a = torch.randn(M, K, generator=g, device=DEV).half()
    kw = {"splits": 1}
    if epi == 1:
        kw["bias"] = (torch.randn(N, generator=g, device=DEV) * 0.1).half()
    if epi == 2:
        kw["resid"] = torch.randn(M, N, generator=g, device=DEV)
    if epi == 3:
        kw["swiglu_I"] = I
    sliced = L.hgemm(a, w, mode, epi=epi, tail=True, **kw)
    whole = L.hgemm(a, w, mode, epi=epi, tail=False, **kw)
    outside = torch.ones(M, N, dtype=torch.bool, device=DEV)
    outside[tail_rows, tail_cols] = False
    assert torch.equal(sliced[outside], whole[outside])
    assert not torch.equal(sliced, whole)  # the sliced tiles sum in another order
    prod = a.double() @ (w.double().t() if mode == 0 else w.double())
    if epi == 3:
        gt, up = prod[:, :I].half().double(), prod[:, I:].half().double()
        want = gt * torch.sigmoid(gt) * up
    else:
        want = prod + (kw["bias"].double() if epi == 1 else 0)
        if epi == 2:
            want = kw["resid"].double() + prod.half().double()
    got, want = sliced[tail_rows, tail_cols].double(), want[tail_rows, tail_cols]
    err = (got - want).abs()
    assert bool((err <= want.abs() * 2.0**-9 + 2e-3 * want.abs().max()).all())


@pytest.mark.parametrize("splits", [1, 2])
def test_gemm16_timed_form(pkg, splits):
    """qlora_gemm16_timed gives qlora_gemm16's output bit for bit and records its two events
    around the kernels (the bench's per-launch timing of the package GEMM)."""
    L, lib = pkg.linear, pkg._lib
    g = torch.Generator(device=DEV).manual_seed(3 + splits)
    a = torch.randn(700, 1536, generator=g, device=DEV).half()
    b = (torch.randn(2048, 1536, generator=g, device=DEV) * 0.02).half()
    want = L.hgemm(a, b, 0, splits=splits)
    got = torch.empty_like(want)
    ws = torch.empty(splits * 700 * 2048, device=DEV) if splits > 1 else None
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()  # creates the events on the device
    stop.record()
    stream = torch.cuda.current_stream().cuda_stream
    lib.call("qlora_gemm16_timed", a.data_ptr(), 1536, b.data_ptr(), 1536, 700, 2048, 1536, 0,
             got.data_ptr(), 2048, None, None, 0, 0, 0, None, 0, 256, 2, splits,
             None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), stream,
             start.cuda_event, stop.cuda_event)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert start.elapsed_time(stop) > 0


@pytest.mark.parametrize("mode,epi,M,N", [(0, 0, 700, 2048), (0, 1, 2600, 2048),
                                          (0, 2, 2549, 1536), (0, 3, 1875, 8960),
                                          (1, 0, 2560, 1536), (1, 2, 301, 8960),
                                          (0, 0, 1, 1536), (1, 0, 129, 1536)])
def test_tile128_equals_tile256(pkg, mode, epi, M, N):
    """qlora_gemm16 on 128 x 128 tiles gives the 256 x 256 tiles' results bit for bit in one
    slice (each output sums its k-steps of 16 in order), for every epilogue, both orientations,
    ragged M; and matches fp64."""
    L = pkg.linear
    g = torch.Generator(device=DEV).manual_seed(M + 10 * epi + mode)
    K = 1536
    kw = {}
    if epi == 3:
        w = (torch.randn(2 * N, K, generator=g, device=DEV) * 0.02).half()
        kw["swiglu_I"] = N
    else:
        w = (torch.randn(*((N, K) if mode == 0 else (K, N)), generator=g, device=DEV) *
             0.02).half()
    a = torch.randn(M, K, generator=g, device=DEV).half()
    if epi == 1:
        kw["bias"] = (torch.randn(N, generator=g, device=DEV) * 0.1).half()
    if epi == 2:
        kw["resid"] = torch.randn(M, N, generator=g, device=DEV)
    big = L.hgemm(a, w, mode, epi=epi, splits=1, tail=False, tile=256, **kw)
    small = L.hgemm(a, w, mode, epi=epi, splits=1, tail=False, tile=128, **kw)
    assert torch.equal(big, small)
    deep = L.hgemm(a, w, mode, epi=epi, splits=1, tail=False, tile=128, stages=4, **kw)
    assert torch.equal(big, deep)
    prod = a.double() @ (w.double().t() if mode == 0 else w.double())
    if epi == 3:
        gt, up = prod[:, :N].half().double(), prod[:, N:].half().double()
        want = gt * torch.sigmoid(gt) * up
    elif epi == 2:
        want = kw["resid"].double() + prod.half().double()
    else:
        want = prod + (kw["bias"].double() if epi == 1 else 0)
    assert rel_err(small, want) < 1e-3


@pytest.mark.parametrize("mode,epi,M,N,K", [(0, 2, 2560, 1536, 8960), (1, 0, 2560, 1536, 17920),
                                            (0, 1, 2949, 2048, 1536), (0, 3, 2949, 8960, 1536),
                                            (1, 0, 2949, 8960, 1536), (0, 0, 1875, 1536, 1536)])
def test_tile128_splits_and_tail_against_fp64(pkg, mode, epi, M, N, K):
    """128 x 128 tiles with split-K (2 and 4 slices) and with the K-sliced last round (the
    step's token counts: 2,949 tokens -> 24 row tiles, 288 or 1,680 tiles over 512 slots)
    against fp64 of the same operands."""
    L = pkg.linear
    g = torch.Generator(device=DEV).manual_seed(M + N + K + epi)
    kw = {}
    if epi == 3:
        w = (torch.randn(2 * N, K, generator=g, device=DEV) * 0.02).half()
        kw["swiglu_I"] = N
    else:
        w = (torch.randn(*((N, K) if mode == 0 else (K, N)), generator=g, device=DEV) *
             0.02).half()
    a = torch.randn(M, K, generator=g, device=DEV).half()
    if epi == 1:
        kw["bias"] = (torch.randn(N, generator=g, device=DEV) * 0.1).half()
    if epi == 2:
        kw["resid"] = torch.randn(M, N, generator=g, device=DEV)
    prod = a.double() @ (w.double().t() if mode == 0 else w.double())
    if epi == 3:
        gt, up = prod[:, :N].half().double(), prod[:, N:].half().double()
        want = gt * torch.sigmoid(gt) * up
    elif epi == 2:
        want = kw["resid"].double() + prod.half().double()
    else:
        want = prod + (kw["bias"].double() if epi == 1 else 0)
    variants = [(1, True)] + ([] if epi == 3 else [(2, False), (4, False)])
    for stages in (2, 4):
        for splits, tail in variants:
            kt = K // 64
            per = -(-(-(-kt // splits)) // stages) * stages  # k-tiles a slice, whole loop trips
            if per * (splits - 1) >= kt:
                continue  # the split would leave a slice empty (refused by the library)
            got = L.hgemm(a, w, mode, epi=epi, splits=splits, tail=tail, tile=128, stages=stages,
                          **kw)
            err = rel_err(got, want)
            print(f"tile 128 stages {stages} splits {splits} tail {tail}: rel {err:.2e}",
                  flush=True)
            assert err < 1e-3


@pytest.mark.parametrize("M", [1, 300, 1875, 2113, 2949])
def test_auto_plan_against_fp64(pkg, M):
    """qlora_gemm16 with its automatic plan (tile 0) at the step's nine products, every epilogue
    they use, against fp64 of the same operands; and the same bits on a second call."""
    L = pkg.linear
    g = torch.Generator(device=DEV).manual_seed(M)
    cases = [(0, 2048, 1536, 1), (0, 1536, 1536, 2), (0, 17920, 1536, 0), (0, 8960, 1536, 3),
             (0, 1536, 8960, 2), (1, 1536, 2048, 0), (1, 1536, 1536, 0), (1, 1536, 17920, 0),
             (1, 8960, 1536, 0)]
    for mode, N, K, epi in cases:
        kw = {}
        if epi == 3:
            w = (torch.randn(2 * N, K, generator=g, device=DEV) * 0.02).half()
            kw["swiglu_I"] = N
        else:
            w = (torch.randn(*((N, K) if mode == 0 else (K, N)), generator=g, device=DEV) *
                 0.02).half()
        a = torch.randn(M, K, generator=g, device=DEV).half()
        if epi == 1:
            kw["bias"] = (torch.randn(N, generator=g, device=DEV) * 0.1).half()
        if epi == 2:
            kw["resid"] = torch.randn(M, N, generator=g, device=DEV)
        got = L.hgemm(a, w, mode, epi=epi, tile=0, **kw)
        again = L.hgemm(a, w, mode, epi=epi, tile=0, **kw)
        assert torch.equal(got, again)
        prod = a.double() @ (w.double().t() if mode == 0 else w.double())
        if epi == 3:
            gt, up = prod[:, :N].half().double(), prod[:, N:].half().double()
            want = gt * torch.sigmoid(gt) * up
        elif epi == 2:
            want = kw["resid"].double() + prod.half().double()
        else:
            want = prod + (kw["bias"].double() if epi == 1 else 0)
        err = rel_err(got, want)
        print(f"M={M} mode={mode} N={N} K={K} epi={epi} plan={L.gemm_plan(M, N, K, mode, epi)}"
              f" rel {err:.2e}", flush=True)
        assert err < 1e-3


@pytest.mark.parametrize("mode,N,K,epi,M", [(0, 4096, 1536, 0, 4160), (0, 4096, 1536, 1, 4160),
                                            (0, 4096, 1536, 2, 4160), (1, 4096, 1536, 0, 4160),
                                            (1, 4096, 1536, 2, 4160), (0, 2048, 1536, 5, 4160),
                                            (0, 8960, 1536, 5, 2113), (1, 8960, 1536, 0, 2113),
                                            (0, 8960, 1536, 5, 1875), (0, 151936, 1536, 0, 2325)])
def test_split_plan_equals_whole_tiles(pkg, mode, N, K, epi, M):
    """The automatic plan's split (the leading columns in whole rounds of 256 x 256 tiles, the
    rest as a second launch on 128 x 128 tiles) gives the same bits as one launch of whole
    256 x 256 tiles without the K-sliced last round (both tile shapes sum each output's k-steps
    in the same order), for every epilogue: store, bias, fp32 residual, SwiGLU with [g | u]."""
    L = pkg.linear
    plan = L.gemm_plan_split(M, N, K, mode, epi)
    print(f"split plan M={M} N={N} K={K} mode={mode} epi={epi}: {plan}", flush=True)
    assert plan[3] in (2, 4) and 0 < plan[4] < N
    g = torch.Generator(device=DEV).manual_seed(M + N + epi)
    wshape = (2 * N, K) if epi == 5 else ((N, K) if mode == 0 else (K, N))
    w = (torch.randn(*wshape, generator=g, device=DEV) * 0.02).half()
    a = torch.randn(M, K, generator=g, device=DEV).half()
    kw = {}
    if epi == 1:
        kw["bias"] = (torch.randn(N, generator=g, device=DEV) * 0.1).half()
    if epi == 2:
        kw["resid"] = torch.randn(M, N, generator=g, device=DEV)
    if epi == 5:
        kw["swiglu_I"] = N
    outs = []
    for whole in (False, True):
        if epi == 5:
            kw["gu"] = torch.full((M, 2 * N), float("nan"), device=DEV, dtype=torch.float16)
        plan_kw = dict(tile=256, stages=2, splits=1, tail=False) if whole else dict(tile=0)
        out = L.hgemm(a, w, mode, epi=epi, **kw, **plan_kw)
        outs.append((out, kw.get("gu")))
    assert torch.equal(outs[0][0], outs[1][0])
    if epi == 5:
        assert torch.equal(outs[0][1], outs[1][1]) and not torch.isnan(outs[0][1]).any()
    prod = a.double() @ (w.double().t() if mode == 0 else w.double())
    if epi == 5:
        gt, up = prod[:, :N].half().double(), prod[:, N:].half().double()
        want = gt * torch.sigmoid(gt) * up
    elif epi == 2:
        want = kw["resid"].double() + prod.half().double()
    else:
        want = prod + (kw["bias"].double() if epi == 1 else 0)
    assert rel_err(outs[0][0], want) < 1e-3


@pytest.mark.parametrize("mode,M,N,K,tile,stages,splits", [(1, 2560, 1536, 17920, 256, 2, 4),
                                                          (1, 1406, 1536, 17920, 256, 2, 7),
                                                          (0, 700, 2048, 1536, 128, 4, 2),
                                                          (1, 2949, 1536, 17920, 256, 2, 3),
                                                          (1, 1875, 1536, 17920, 256, 2, 5),
                                                          (1, 1, 1536, 17920, 256, 2, 16),
                                                          (1, 300, 1536, 2048, 128, 2, 8)])
def test_gemm16_parts_sum_to_the_split_product(pkg, mode, M, N, K, tile, stages, splits):
    """qlora_gemm16_parts leaves the K slices of the split-K product unsummed: summed in slice
    order and rounded to fp16 they are the split-K product bit for bit, and the slice sums add
    up to the fp64 product."""
    L = pkg.linear
    g = torch.Generator(device=DEV).manual_seed(M + splits)
    a = torch.randn(M, K, generator=g, device=DEV).half()
    w = (torch.randn(*((N, K) if mode == 0 else (K, N)), generator=g, device=DEV) *
         0.02).half()
    ws = torch.full((splits, M, N), float("nan"), device=DEV)
    pkg._lib.call("qlora_gemm16_parts", a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0),
                  M, N, K, mode, tile, stages, splits, ws.data_ptr(), ws.numel(),
                  L._stream(a.device))
    whole = L.hgemm(a, w, mode, tile=tile, stages=stages, splits=splits)
    s = ws[0].clone()
    for k in range(1, splits):
        s += ws[k]
    assert torch.equal(s.half(), whole)
    prod = a.double() @ (w.double().t() if mode == 0 else w.double())
    assert rel_err(s, prod) < 1e-3


@pytest.mark.parametrize("M,tile,stages,tail", [(2560, 256, 2, False), (2600, 256, 2, True),
                                                (1875, 128, 2, True), (1875, 128, 2, False),
                                                (700, 128, 4, False), (1, 0, 0, True),
                                                (2113, 0, 0, True)])
def test_swiglu_keep_epilogue(pkg, M, tile, stages, tail):
    """Epilogue 5: the SwiGLU output equals epilogue 3's bit for bit and the kept product
    [g | u] equals the plain GEMM's store of it bit for bit (each output sums the same k-steps
    in the same order), for both tile shapes, with the K-sliced last round (2,600 rows: 770
    tiles, the last two sliced) and through the automatic plan (tile 0)."""
    L = pkg.linear
    I, K = 8960, 1536
    g = torch.Generator(device=DEV).manual_seed(M + tile)
    w = (torch.randn(2 * I, K, generator=g, device=DEV) * 0.02).half()
    a = torch.randn(M, K, generator=g, device=DEV).half()
    kw = dict(tile=tile, stages=stages) if tile else dict(tile=0)
    if tile:
        kw.update(splits=1, tail=tail)
    gu = torch.full((M, 2 * I), float("nan"), device=DEV, dtype=torch.float16)
    m5 = L.hgemm(a, w, 0, epi=5, swiglu_I=I, gu=gu, **kw)
    m3 = L.hgemm(a, w, 0, epi=3, swiglu_I=I, **kw)
    plain = L.hgemm(a, w, 0, tile=tile or 0, **({"splits": 1, "tail": False, "stages": stages}
                                                 if tile else {}))
    assert torch.equal(m5, m3)
    if tile and not tail:  # whole tiles: the same bits as the plain product's
        assert torch.equal(gu, plain)
    ref = (a.double() @ w.double().t())
    assert rel_err(gu, ref) < 1e-3
    assert not torch.isnan(gu).any()


def _f32_ref(a, b, mode, alpha, row_scale=None, resid=None):
    A = a.double() if mode == 1 else a.double().t()
    want = alpha * (A @ b.double())
    if resid is not None:
        rs = row_scale.double()[:, None] if row_scale is not None else 1.0
        want = want + rs * resid.double()
    return want


@pytest.mark.parametrize("mode,M,K", [(1, 300, 8192), (1, 2048, 4480), (1, 1, 128),
                                      (2, 8192, 384), (2, 3712, 1664), (2, 128, 128)])
def test_gemm_f32_against_fp64(pkg, mode, M, K):
    """qlora_gemm16_f32 (the LM head's fp32 products): out = alpha A op(B) + row_scale * resid,
    A B (mode 1) or A^T B with A stored [K, M] (mode 2), updated in place (out is resid), at
    every tile / stage / split variant that takes the shape and the automatic plan, against
    fp64. In one slice every tile shape gives the same bits."""
    L = pkg.linear
    N = 1536
    g = torch.Generator(device=DEV).manual_seed(M + K + mode)
    a = (torch.randn(*((M, K) if mode == 1 else (K, M)), generator=g, device=DEV) * 0.5).half()
    b = (torch.randn(K, N, generator=g, device=DEV) * 0.02).half()
    resid = torch.randn(M, N, generator=g, device=DEV)
    rs = torch.rand(M, generator=g, device=DEV) + 0.5
    want = _f32_ref(a, b, mode, 0.25, rs, resid)
    plain = _f32_ref(a, b, mode, 1.0)
    one_slice = []
    variants = [(256, 2), (128, 2), (128, 4)]
    for tile, stages in variants:
        if (K // 64) % stages or N % tile or (mode == 2 and M % tile):
            continue
        for splits in (1, 2, 4):
            if (K // 64) < splits * stages:
                continue
            out = resid.clone()
            L.gemm_f32(a, b, mode, alpha=0.25, row_scale=rs, resid=out, out=out, tile=tile,
                       stages=stages, splits=splits)
            err = (out.double() - want).abs().max().item()
            assert err <= 1e-5 * want.abs().max().item() + 1e-6, (tile, stages, splits, err)
            if splits == 1:
                one_slice.append(out)
            p = L.gemm_f32(a, b, mode, tile=tile, stages=stages, splits=splits)
            assert rel_err(p, plain) < 1e-6
    assert one_slice and all(torch.equal(o, one_slice[0]) for o in one_slice[1:])
    auto = L.gemm_f32(a, b, mode, alpha=0.25, row_scale=rs, resid=resid)
    assert (auto.double() - want).abs().max().item() <= 1e-5 * want.abs().max().item() + 1e-6
    assert torch.equal(auto, L.gemm_f32(a, b, mode, alpha=0.25, row_scale=rs, resid=resid))
