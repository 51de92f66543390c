"""The projections' plain GEMMs through qlora_gemm (rocBLAS with an explicit solution) and
qlora_gemmlt (hipBLASLt) against an fp64 product of the same fp16 operands: every solution
computes fp16(sum in fp32 (+ bias)), so results agree with fp64 to fp16 rounding plus fp32
summation-order noise."""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def ref(a, b, op, bias=None):
    bd = b.double()
    r = a.double() @ (bd.t() if op == 0 else bd)
    if bias is not None:
        r = r + bias.double()
    return r


def check(out, want):
    # one fp16 rounding of the fp32 sum: |err| <= 2^-11 |x| + accumulation noise
    err = (out.double() - want).abs()
    tol = want.abs() * 2.0**-10 + 1e-3 * want.abs().max()
    assert bool((err <= tol).all()), float((err - tol).max())


@pytest.mark.parametrize("op", [0, 1])
@pytest.mark.parametrize("M,N,K", [(1, 256, 128), (37, 384, 200), (600, 1536, 1536),
                                   (2537, 2048, 1536)])
def test_gemm_default_and_listed_solutions(pkg, op, M, N, K):
    g = torch.Generator(device=DEV).manual_seed(M + N + K + op)
    a = torch.randn((M, K), device=DEV, generator=g).half()
    b = (torch.randn((N, K) if op == 0 else (K, N), device=DEV, generator=g) * 0.05).half()
    want = ref(a, b, op)
    sols = pkg.gemm.solutions(op, a, b, torch.empty((M, N), device=DEV, dtype=torch.float16))
    assert len(sols) > 0
    for sol in [0] + sols[:: max(1, len(sols) // 6)]:
        out = torch.full((M, N), float("nan"), device=DEV, dtype=torch.float16)
        pkg.gemm._run((sol, 1), op, a, b, out, None, M, N, K, K, b.stride(0), N, a.device)
        check(out, want)


def test_gemm_strided_views_alpha_beta(pkg):
    """Row strides larger than the width (column slices of wider buffers), alpha and beta."""
    g = torch.Generator(device=DEV).manual_seed(5)
    M, N, K = 300, 256, 320
    abuf = torch.randn((M, K + 64), device=DEV, generator=g).half()
    bbuf = (torch.randn((N, K + 32), device=DEV, generator=g) * 0.05).half()
    cbuf = torch.randn((M, N + 128), device=DEV, generator=g).half()
    a, b, c = abuf[:, 16:16 + K], bbuf[:, :K], cbuf[:, 64:64 + N]
    c0, outside = c.clone(), cbuf[:, :64].clone()
    pkg._lib.call("qlora_gemm", 0, M, N, K, a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0),
                  c.data_ptr(), c.stride(0), 0.5, 2.0, 0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    check(c, 0.5 * ref(a, b, 0) + 2.0 * c0.double())
    assert torch.equal(cbuf[:, :64], outside)  # columns outside the view are not written


def test_mm_bias_and_tuned_choice(pkg):
    """gemm.mm with a tuned bucket (a rocBLAS solution or torch's matmul), with and without the
    bias (one rounding of acc + bias), and at sizes of neighbouring buckets."""
    G = pkg.gemm
    G.reset()
    try:
        N, K = 512, 256
        G.tune([(G.NT, N, K), (G.NT, N, K, True), (G.NN, K, N)], [700], DEV)
        assert (0, G.NT, N, K, False, G._bucket(700)) in G._CHOICE
        assert (0, G.NT, N, K, True, G._bucket(700)) in G._CHOICE
        g = torch.Generator(device=DEV).manual_seed(9)
        w = (torch.randn((N, K), device=DEV, generator=g) * 0.05).half()
        bias = (torch.randn((N,), device=DEV, generator=g) * 0.1).half()
        for M in (700, 650, 1, 1500):
            x = torch.randn((M, K), device=DEV, generator=g).half()
            check(G.mm(x, w, G.NT), ref(x, w, 0))
            check(G.mm(x, w, G.NT, bias=bias), ref(x, w, 0, bias))
            dy = torch.randn((M, N), device=DEV, generator=g).half()
            check(G.mm(dy, w, G.NN), ref(dy, w, 1))
        # force a rocBLAS solution for the bucket and check the bias path through it
        sols = G.solutions(G.NT, x, w, torch.empty((x.shape[0], N), device=DEV,
                                                   dtype=torch.float16))
        G._CHOICE[(0, G.NT, N, K, True, G._bucket(x.shape[0]))] = (sols[0], 1)
        check(G.mm(x, w, G.NT, bias=bias), ref(x, w, 0, bias))
        # and hipBLASLt's first choice, bias in its epilogue
        G._CHOICE[(0, G.NT, N, K, True, G._bucket(x.shape[0]))] = G.LT_DEFAULT
        check(G.mm(x, w, G.NT, bias=bias), ref(x, w, 0, bias))
    finally:
        G.reset()



@pytest.mark.parametrize("op", [0, 1])
@pytest.mark.parametrize("splits", [2, 4, 8])
@pytest.mark.parametrize("M,N,K", [(1, 256, 8192), (300, 1536, 17920), (37, 512, 4096)])
def test_gemm_splitk(pkg, op, splits, M, N, K):
    """qlora_gemm_splitk: fp32 partial products over K slices, one fixed-order sum, one rounding
    (with and without bias), for rocBLAS's default and listed solutions of the batched problem;
    the output's row stride may exceed its width."""
    G = pkg.gemm
    g = torch.Generator(device=DEV).manual_seed(M * splits + N + op)
    a = torch.randn((M, K), device=DEV, generator=g).half()
    b = (torch.randn((N, K) if op == 0 else (K, N), device=DEV, generator=g) * 0.05).half()
    bias = (torch.randn((N,), device=DEV, generator=g) * 0.1).half()
    want = ref(a, b, op)
    work = torch.empty((splits * M * N,), device=DEV, dtype=torch.float32)
    sols = G.solutions(op, a, b, None, splits, work)
    assert len(sols) > 0
    cbuf = torch.full((M, N + 8), float("nan"), device=DEV, dtype=torch.float16)
    out = cbuf[:, :N]
    for sol in [0] + sols[:: max(1, len(sols) // 3)]:
        G._run((sol, splits), op, a, b, out, None, M, N, K, K, b.stride(0), out.stride(0),
               a.device, work=work)
        check(out, want)
    G._run((0, splits), op, a, b, out, bias, M, N, K, K, b.stride(0), out.stride(0), a.device)
    check(out, want + bias.double())
    assert torch.isnan(cbuf[:, N:].float()).all()  # columns past the view are not written


def test_mm_uses_a_tuned_split_variant(pkg):
    G = pkg.gemm
    G.reset()
    try:
        N, K, M = 512, 16384, 600
        G._CHOICE[(0, G.NN, N, K, False, G._bucket(M))] = (0, 4)
        g = torch.Generator(device=DEV).manual_seed(3)
        dy = torch.randn((M, K), device=DEV, generator=g).half()
        w = (torch.randn((K, N), device=DEV, generator=g) * 0.05).half()
        check(G.mm(dy, w, G.NN), ref(dy, w, 1))
    finally:
        G.reset()


def test_package_gemm_variant(pkg):
    """The package's MFMA GEMM as a tuned variant of gemm.mm (PKG): a candidate of the tuner for
    the NT shapes it tiles, with and without the bias, at sizes of neighbouring buckets; an
    output it does not take (unaligned row stride) runs rocBLAS's default instead and the
    bucket keeps its choice."""
    G = pkg.gemm
    G.reset()
    try:
        N, K = 2048, 1536
        G.tune([(G.NT, N, K)], [700], DEV)
        assert G.PKG in G._CANDIDATES[(0, G.NT, N, K, False)]
        assert G.pkg_fits(G.NT, N, K) and not G.pkg_fits(G.NN, N, K)
        assert not G.pkg_fits(G.NT, N, 200)
        g = torch.Generator(device=DEV).manual_seed(12)
        w = (torch.randn((N, K), device=DEV, generator=g) * 0.02).half()
        bias = (torch.randn((N,), device=DEV, generator=g) * 0.1).half()
        for M in (700, 1, 300, 2600):
            for b in (None, bias):
                G._CHOICE[(0, G.NT, N, K, b is not None, G._bucket(M))] = G.PKG
            x = torch.randn((M, K), device=DEV, generator=g).half()
            y = G.mm(x, w, G.NT)
            check(y, ref(x, w, 0))
            assert torch.equal(y, pkg.linear.hgemm(x, w, 0, splits=1))
            check(G.mm(x, w, G.NT, bias=bias), ref(x, w, 0, bias))
        cbuf = torch.empty((M, N + 4), device=DEV, dtype=torch.float16)
        out = G.mm(x, w, G.NT, out=cbuf[:, :N])  # row stride N + 4: not 16-byte rows
        check(out, ref(x, w, 0))
        assert G._CHOICE[(0, G.NT, N, K, False, G._bucket(M))] == G.PKG
    finally:
        G.reset()


def test_swiglu_tuned_choice(pkg):
    """The forward's SwiGLU product per token bucket: tune_swiglu times the package's GEMM with
    the SwiGLU epilogue against the library GEMM + SwiGLU kernel; either form, forced, matches
    fp64 silu(g) u of the fp16-rounded [g | u]."""
    G, L = pkg.gemm, pkg.linear
    G.reset()
    L._SWIGLU_ON_PKG.clear()
    gemm_was, L.GEMM = L.GEMM, "library"  # the step's library path (the per-bucket choice)
    try:
        I, K, M = 1024, 1536, 700
        g = torch.Generator(device=DEV).manual_seed(13)
        w16 = (torch.randn((2 * I, K), device=DEV, generator=g) * 0.02).half()
        w = pkg.ops.NF4Weight(pkg.quant.quantize_nf4(w16))
        G.tune([(G.NT, 2 * I, K)], [M], DEV)
        L.tune_swiglu(I, K, [M], DEV)
        assert (0, I, K, G._bucket(M)) in L._SWIGLU_ON_PKG
        x = torch.randn((M, K), device=DEV, generator=g).half()
        gu = (x.double() @ L.dequantize(w).double().t()).half().double()
        gt, up = gu[:, :I], gu[:, I:]
        want = gt * torch.sigmoid(gt) * up
        for on_pkg in (True, False):
            L._SWIGLU_ON_PKG[(0, I, K, G._bucket(M))] = on_pkg
            assert L.swiglu_on_package(0, I, K, M) == on_pkg
            m = L.nf4_linear_swiglu(x, w, I)
            err = (m.double() - want).abs()
            assert bool((err <= want.abs() * 2.0**-9 + 2e-3 * want.abs().max()).all())
    finally:
        L.GEMM = gemm_was
        G.reset()
        L._SWIGLU_ON_PKG.clear()


@pytest.mark.parametrize("variant", [(0, 4), (0, 2), (0, 1), (-2, 1)])
@pytest.mark.parametrize("M", [2537, 37])
def test_mm_resid_equals_mm_then_resid_add(pkg, variant, M):
    """The down projection with the residual add (gemm.mm_resid): with a split-K variant the
    split's reduce adds the fp32 residual itself, with the package's GEMM (-2, 1) its epilogue;
    the result equals mm() followed by the residual-add kernel bit for bit (the same fp16
    rounding of the product, the same fp32 add), also in place (out = resid); without a split
    it is that two-pass form."""
    G = pkg.gemm
    G.reset()
    try:
        N, K = 1536, 8960
        G._CHOICE[(0, G.NT, N, K, False, G._bucket(M))] = variant
        g = torch.Generator(device=DEV).manual_seed(M + variant[1])
        x = torch.randn((M, K), device=DEV, generator=g).half()
        w = (torch.randn((N, K), device=DEV, generator=g) * 0.02).half()
        res = torch.randn((M, N), device=DEV, generator=g)
        want = pkg.ops._resid_add(res, G.mm(x, w, G.NT))
        assert torch.equal(G.mm_resid(x, w, G.NT, res), want)
        inplace = res.clone()
        G.mm_resid(x, w, G.NT, inplace, out=inplace)
        assert torch.equal(inplace, want)
        check((want - res).half(), ref(x, w, 0))
    finally:
        G.reset()


def _lt_listed(pkg, op, M, N, K, lda, ldb, ldc, bias, ws_bytes):
    cnt = ctypes.c_int32(0)
    arr = (ctypes.c_int32 * 512)()
    pkg._lib.call("qlora_gemmlt_solutions", op, M, N, K, lda, ldb, ldc, int(bias), ws_bytes, arr,
                  512, ctypes.byref(cnt))
    return list(arr)[:min(cnt.value, 512)]


@pytest.mark.parametrize("op", [0, 1])
@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("M,N,K", [(1, 256, 128), (37, 384, 200), (2537, 2048, 1536)])
def test_gemmlt_first_choice_and_listed_solutions(pkg, op, with_bias, M, N, K):
    """qlora_gemmlt: hipBLASLt's first choice and a spread of its listed solutions for the exact
    problem, with the bias added in the epilogue (one rounding), on strided views; columns
    outside the output view stay untouched."""
    g = torch.Generator(device=DEV).manual_seed(M + N + K + op + 7 * with_bias)
    abuf = torch.randn((M, K + 8), device=DEV, generator=g).half()
    b = (torch.randn((N, K) if op == 0 else (K, N), device=DEV, generator=g) * 0.05).half()
    bias = (torch.randn((N,), device=DEV, generator=g) * 0.1).half() if with_bias else None
    a = abuf[:, 8:]
    want = ref(a, b, op, bias)
    ws_bytes = pkg.gemm.LT_WORKSPACE
    ws = torch.empty((ws_bytes,), device=DEV, dtype=torch.uint8)
    cbuf = torch.full((M, N + 16), float("nan"), device=DEV, dtype=torch.float16)
    out = cbuf[:, :N]
    sols = _lt_listed(pkg, op, M, N, K, a.stride(0), b.stride(0), out.stride(0), with_bias,
                      ws_bytes)
    assert len(sols) > 0
    for sol in [0] + sols[:: max(1, len(sols) // 5)]:
        out.fill_(float("nan"))
        pkg._lib.call("qlora_gemmlt", op, M, N, K, a.data_ptr(), a.stride(0), b.data_ptr(),
                      b.stride(0), out.data_ptr(), out.stride(0),
                      bias.data_ptr() if bias is not None else None, 1.0, 0.0, sol,
                      ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
        check(out, want)
    assert torch.isnan(cbuf[:, N:].float()).all()


def test_gemmlt_alpha_beta_and_unlisted_solution(pkg):
    g = torch.Generator(device=DEV).manual_seed(11)
    M, N, K = 300, 256, 320
    a = torch.randn((M, K), device=DEV, generator=g).half()
    b = (torch.randn((N, K), device=DEV, generator=g) * 0.05).half()
    c = torch.randn((M, N), device=DEV, generator=g).half()
    c0 = c.clone()
    stream = torch.cuda.current_stream().cuda_stream
    pkg._lib.call("qlora_gemmlt", 0, M, N, K, a.data_ptr(), K, b.data_ptr(), K, c.data_ptr(), N,
                  None, 0.5, 2.0, 0, None, 0, stream)
    torch.cuda.synchronize()
    check(c, 0.5 * ref(a, b, 0) + 2.0 * c0.double())
    listed = set(_lt_listed(pkg, 0, M, N, K, K, K, N, False, 0))
    bogus = max(listed) + 1000
    c1 = c.clone()
    with pytest.raises(RuntimeError):
        pkg._lib.call("qlora_gemmlt", 0, M, N, K, a.data_ptr(), K, b.data_ptr(), K,
                      c.data_ptr(), N, None, 1.0, 0.0, bogus, None, 0, stream)
    torch.cuda.synchronize()
    assert torch.equal(c, c1)  # nothing ran
