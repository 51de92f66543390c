"""The LM head over vocabulary pieces: loss, the gradient w.r.t. the head
input and w.r.t. the tied embedding. Against an fp64 CPU autograd reference of the same math
(fp16 GEMM inputs; the reference's head test, test_host_head.py:164-178: gradient within 1e-3
relative), and at the full config-4 size (T = 2048, V = 151,936) against the whole-row path
(test_host_head.py:157-161 tolerances: per-token loss rtol 1e-4 / atol 1e-3, loss 1e-5)."""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _inputs(T, V, H, seed, ignore=0.25):
    g = torch.Generator(device=DEV).manual_seed(seed)
    hn = torch.randn(T, H, generator=g, device=DEV).half()
    E = (torch.randn(V, H, generator=g, device=DEV) * 0.02).half()
    targets = torch.randint(0, V, (T,), generator=g, device=DEV)
    drop = torch.rand(T, generator=g, device=DEV) < ignore
    targets[drop] = -100
    return hn, E, targets


@pytest.mark.parametrize("T,V,piece", [(37, 20096, 8192), (16, 151936, 8192), (9, 12288, 4096),
                                        (300, 8320, 4096)])
@pytest.mark.parametrize("path", ["chunked", "full"])
def test_head_against_fp64(pkg, T, V, piece, path):
    """Loss, per-token loss, dh and dE of either head (pieces, whole rows) against fp64
    autograd: row counts off the 128-row blocks of the dE product, a last piece narrower than
    the others (and than 256 columns: the GEMM's 128 x 128 tiles)."""
    H = 1536
    hn, E, targets = _inputs(T, V, H, T)
    targets[1] = -100  # at least one ignored row
    denom = float((targets >= 0).sum())
    if path == "chunked":
        r = pkg.head.chunked_head(hn, E, targets, denom, piece=piece)
    else:
        r = pkg.head.full_head(hn, E, targets, denom)
    x = hn.double().cpu().requires_grad_(True)
    w = E.double().cpu().requires_grad_(True)
    tg = targets.cpu()
    ce = torch.nn.functional.cross_entropy(x @ w.t(), tg.clamp(min=0), reduction="none")
    loss = (ce * (tg >= 0)).sum() / denom
    dx, dw = torch.autograd.grad(loss, [x, w])
    assert abs(r.loss.item() - loss.item()) <= 1e-4 * abs(loss.item())
    torch.testing.assert_close(r.tok_loss.cpu().double(), (ce * (tg >= 0)).detach(),
                               rtol=1e-4, atol=1e-3)
    assert rel(r.dhn, dx) < 1e-3
    assert rel(r.dE, dw) < 1e-3
    assert torch.equal(r.dhn[1].cpu(), torch.zeros(H))  # ignored row: no gradient


def test_config4_chunked_equals_whole_row(pkg):
    """T = 2048, V = 151,936, 8192-wide pieces, ~25 % ignored: the piece-wise loss, entropy and
    accuracy equal the whole-row kernel's up to the GEMM's summation order; dh and dE too."""
    T, V, H = 2048, 151936, 1536
    hn, E, targets = _inputs(T, V, H, 4)
    denom = float((targets >= 0).sum())
    a = pkg.head.chunked_head(hn, E, targets, denom)
    b = pkg.head.full_head(hn, E, targets, denom)
    torch.testing.assert_close(a.tok_loss, b.tok_loss, rtol=1e-4, atol=1e-3)
    torch.testing.assert_close(a.entropy, b.entropy, rtol=1e-4, atol=1e-3)
    assert (a.correct != b.correct).sum() <= 1
    torch.testing.assert_close(a.loss, b.loss, rtol=1e-5, atol=1e-5)
    assert rel(a.dhn, b.dhn) < 1e-3
    assert rel(a.dE, b.dE) < 1e-3


@pytest.mark.parametrize("path", ["chunked", "full"])
def test_config4_full_size_against_fp64(pkg, path):
    """Config 4 at its stated size (T = 2048, V = 151,936, ~25 % ignored): loss, every token's
    loss, dh and dE against fp64 autograd of the same fp16 operands (torch's double-precision
    products on the GPU, independent of this package's kernels), at the reference's head
    tolerances (test_host_head.py:157-178: loss 1e-5 relative, per-token loss rtol 1e-4 /
    atol 1e-3, gradients 1e-3 relative)."""
    T, V, H = 2048, 151936, 1536
    hn, E, targets = _inputs(T, V, H, 4)
    denom = float((targets >= 0).sum())
    fn = pkg.head.chunked_head if path == "chunked" else pkg.head.full_head
    r = fn(hn, E, targets, denom)
    torch.cuda.synchronize()
    x = hn.double().requires_grad_(True)
    w = E.double().requires_grad_(True)
    sup = targets >= 0
    ce = torch.nn.functional.cross_entropy(x @ w.t(), targets.clamp(min=0), reduction="none")
    ce = ce * sup
    loss = ce.sum() / denom
    dx, dw = torch.autograd.grad(loss, [x, w])
    print(f"{path}: loss {r.loss.item():.8f} fp64 {loss.item():.8f}", flush=True)
    assert abs(r.loss.item() - loss.item()) <= 1e-5 * abs(loss.item())
    torch.testing.assert_close(r.tok_loss.double(), ce.detach(), rtol=1e-4, atol=1e-3)
    assert rel(r.dhn, dx) < 1e-3
    assert rel(r.dE, dw) < 1e-3
    # every row on its own: no row's gradient off by more than the bound, ignored rows zero
    row_err = (r.dhn.double() - dx).norm(dim=1) / dx.norm(dim=1).clamp_min(1e-30)
    assert float(row_err[sup].max()) < 5e-3
    assert not r.dhn[~sup].any()
    del x, w, dx, dw, ce


def test_ce_grad_equals_whole_row_kernel(pkg):
    """qlora_ce_grad over a piece, after the pieces' finish, writes exactly the whole-row
    kernel's in-place gradient columns."""
    T, V, H = 64, 16384, 256
    hn, E, targets = _inputs(T, V, H, 11)
    order = torch.argsort((targets < 0).to(torch.int8), stable=True)
    hn, targets = hn[order].contiguous(), targets[order].contiguous()
    n_sup = int((targets >= 0).sum())
    logits = hn @ E.t()
    whole = logits.clone()
    z = torch.empty(T, device=DEV)
    pkg.ops._ce(whole, targets, z.clone(), z.clone(), torch.empty(T, device=DEV,
                                                                    dtype=torch.int32))
    state = torch.full((T, 4), float("-inf"), device=DEV)
    state[:, 1:3] = 0
    bi = torch.zeros(T, device=DEV, dtype=torch.int32)
    xt = torch.zeros(T, device=DEV)
    alpha = torch.empty(max(n_sup, 1), device=DEV)
    wt = torch.zeros(max(n_sup, 1), H, device=DEV, dtype=torch.float16)
    for v0 in range(0, V, 4096):
        piece = logits[:, v0:v0 + 4096].clone()
        pkg.ops._ce_piece(piece, E[v0:v0 + 4096], targets, state, bi, xt, alpha, wt, v0, n_sup)
    for v0 in range(0, V, 4096):
        g = logits[:, v0:v0 + 4096].clone()
        pkg.ops._ce_grad(g, targets, state, v0, n_sup)
        assert torch.equal(g[:n_sup].view(torch.int16), whole[:n_sup, v0:v0 + 4096].view(torch.int16))
