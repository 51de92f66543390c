"""Pins of the elementwise/reduction oracle (oracle/ops.py) against independent formulations:
autograd, float64, complex rotation, torch's own cross-entropy."""

import numpy as np
import pytest
import torch

from oracle import ops as O
from oracle import philox as P


def close(a, b, tol):
    torch.testing.assert_close(a.double(), b.double(), rtol=tol, atol=tol)


@pytest.mark.parametrize("n,H", [(37, 1536), (5, 100)])
def test_rms_against_autograd(n, H):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(n, H, generator=g) * 3
    delta = torch.randn(n, H, generator=g).half()
    w = torch.rand(H, generator=g) + 0.5
    p, eps = 0.25, 1e-6
    tok = torch.arange(n) * 3 + 1
    G, seed, ctrs = 40960, 77, (11, 12)
    xsum, y, yq, yv, rstd = O.rms_fwd(x, w, eps, delta=delta, tok=tok, p=p, seed=seed,
                                      ctrs=ctrs, G=G, vec=4, drop_q=True, drop_v=True)
    xr = (x.double() + delta.double()).requires_grad_()
    yr = w.double() * (xr * torch.rsqrt(xr.pow(2).mean(-1, keepdim=True) + eps))
    close(xsum, xr, 1e-6)
    close(y, yr, 2e-3)
    elems = (tok[:, None] * H + torch.arange(H)[None]).reshape(-1).numpy()
    kq = torch.from_numpy(P.keep_mask(elems, seed, ctrs[0], G, np.float32(1 - p), 4)).view(n, H)
    kv = torch.from_numpy(P.keep_mask(elems, seed, ctrs[1], G, np.float32(1 - p), 4)).view(n, H)
    assert torch.equal(yq != 0, kq) and torch.equal(yv != 0, kv)
    assert not torch.equal(kq, kv)
    close(yq, torch.where(kq, yr / (1 - p), 0.0), 2e-3)

    dy = torch.randn(n, H, generator=g).half()
    tq = torch.randn(n, H, generator=g).half()
    tv = torch.randn(n, H, generator=g).half()
    dres = torch.randn(n, H, generator=g)
    dx = O.rms_bwd(dy, xsum, rstd, w, dres=dres, tq=tq, tv=tv, tok=tok, p=p, seed=seed,
                   ctrs=ctrs, G=G, vec=4, grad_scale=0.5)
    g_total = dy.double() + (kq * tq.double() + kv * tv.double()) / (1 - p)
    (gx,) = torch.autograd.grad(yr, xr, g_total)
    close(dx, dres.double() + 0.5 * gx, 1e-4)


def test_rope_against_complex_rotation():
    g = torch.Generator().manual_seed(0)
    n, HQ, HKV, D, s = 23, 12, 2, 128, 2.0
    C = (HQ + 2 * HKV) * D
    qkv = torch.randn(n, C, generator=g).half()
    lq = torch.randn(n, HQ * D, generator=g).half()
    lv = torch.randn(n, HKV * D, generator=g).half()
    pos = torch.randint(0, 500, (n,), generator=g, dtype=torch.int32)
    cos, sin = O.rope_tables(512, D, 1e6)
    q, k, v = O.rope_fwd(qkv, lq, lv, cos, sin, pos, HQ, HKV, D, s)
    # x1 + i x2 times e^{i pos theta}, theta_k = 1e6^(-2k/D), in float64
    theta = 1e6 ** (-torch.arange(0, D, 2, dtype=torch.float64) / D)
    ang = pos.double()[:, None, None] * theta[None, None, :]
    rot = torch.polar(torch.ones_like(ang), ang)

    def crot(x):
        z = torch.complex(x[..., :D // 2], x[..., D // 2:]) * rot
        return torch.cat([z.real, z.imag], -1)

    qf = qkv[:, :HQ * D].double().view(n, HQ, D) + s * lq.double().view(n, HQ, D)
    kf = qkv[:, HQ * D:(HQ + HKV) * D].double().view(n, HKV, D)
    vf = qkv[:, (HQ + HKV) * D:].double().view(n, HKV, D) + s * lv.double().view(n, HKV, D)
    close(q, crot(qf), 2e-3)
    close(k, crot(kf).repeat_interleave(HQ // HKV, 1), 2e-3)
    close(v, vf.repeat_interleave(HQ // HKV, 1), 2e-3)

    dq = torch.randn(n, HQ, D, generator=g).half()
    dk = torch.randn(n, HQ, D, generator=g).half()
    dv = torch.randn(n, HQ, D, generator=g).half()
    dqkv = O.rope_bwd(dq, dk, dv, cos, sin, pos, HQ, HKV, D)
    # the inverse rotation is the conjugate one; sum over the GQA replicas first
    conj = torch.polar(torch.ones_like(ang), -ang)

    def cinv(x):
        z = torch.complex(x[..., :D // 2], x[..., D // 2:]) * conj
        return torch.cat([z.real, z.imag], -1)

    close(dqkv[:, :HQ * D], cinv(dq.double()).reshape(n, -1), 3e-3)
    dks = dk.double().view(n, HKV, HQ // HKV, D).sum(2)
    dvs = dv.double().view(n, HKV, HQ // HKV, D).sum(2)
    close(dqkv[:, HQ * D:(HQ + HKV) * D], cinv(dks).reshape(n, -1), 1e-2)
    close(dqkv[:, (HQ + HKV) * D:], dvs.reshape(n, -1), 1e-2)


@pytest.mark.parametrize("n,I", [(9, 8960), (3, 1000)])
def test_glu_against_autograd(n, I):
    g = torch.Generator().manual_seed(0)
    gu = (torch.randn(n, 2 * I, generator=g) * 3).half()
    m = O.glu_fwd(gu, I)
    gg = gu[:, :I].double().requires_grad_()
    uu = gu[:, I:].double().requires_grad_()
    ref = torch.nn.functional.silu(gg) * uu
    close(m, ref, 2e-3)
    dm = torch.randn(n, I, generator=g).half()
    dg, du = torch.autograd.grad(ref, (gg, uu), dm.double())
    out = O.glu_bwd(dm, gu, I)
    close(out[:, :I], dg, 1e-2)
    close(out[:, I:], du, 1e-2)


@pytest.mark.parametrize("V", [151936, 5000])
def test_ce_against_torch_cross_entropy(V):
    g = torch.Generator().manual_seed(0)
    n = 37
    logits = (torch.randn(n, V, generator=g) * 4).half()
    target = torch.randint(0, V, (n,), generator=g)
    target[::5] = -100
    target[1] = logits[1].float().argmax()
    ref = logits.double().requires_grad_()
    ce = torch.nn.functional.cross_entropy(ref, target, ignore_index=-100, reduction="none")
    (grad,) = torch.autograd.grad(ce.sum(), ref)
    lse = torch.logsumexp(ref.detach(), -1)
    entropy = lse - (torch.softmax(ref.detach(), -1) * ref.detach()).sum(-1)
    loss, ent, correct, out = O.ce(logits, target)
    close(loss, ce.detach(), 1e-4)
    close(ent, entropy, 1e-3)
    assert torch.equal(correct.bool(), (target >= 0) & (logits.float().argmax(-1) == target))
    assert correct[1].item() == 1  # target = argmax known answer (test_kernels.py:217, 233)
    close(out, grad, 1e-3)


@pytest.mark.parametrize("n,n_sup", [(30, 18), (7, 0), (5, 5)])
def test_ce_pieces_equal_whole_rows(n, n_sup):
    """The online state over 8192-wide pieces gives the whole-row loss, entropy and accuracy, and
    sum_pieces alpha-rescaled exp(x - m) W - W[target] = (softmax - onehot) W."""
    g = torch.Generator().manual_seed(n)
    V, H, piece = 20000, 64, 8192
    logits = (torch.randn(n, V, generator=g) * 4).half()
    w = (torch.randn(V, H, generator=g) * 0.05).half()
    target = torch.randint(0, V, (n,), generator=g)
    target[n_sup:] = -100
    loss_a, ent_a, cor_a, grad = O.ce(logits, target)
    state, best_idx, xt = O.ce_state_init(n)
    acc = torch.zeros(max(n_sup, 1), H, dtype=torch.float64)
    wt = torch.zeros(max(n_sup, 1), H, dtype=torch.float16)
    for v0 in range(0, V, piece):
        width = min(piece, V - v0)
        state, best_idx, xt, alpha, wrows, inp, new = O.ce_piece(
            logits[:, v0:v0 + width], w[v0:v0 + width], target, state, best_idx, xt, v0, n_sup)
        if n_sup:
            acc[:n_sup] = acc[:n_sup] * alpha[:, None].double() \
                + new[:n_sup].double() @ w[v0:v0 + width].double()
            wt[:n_sup] = torch.where(inp[:, None], wrows, wt[:n_sup])
    loss_b, ent_b, cor_b, dh = O.ce_finish(state, best_idx, xt, target, acc.float(), wt, n_sup)
    close(loss_b, loss_a, 1e-4)
    close(ent_b, ent_a, 1e-4)
    assert torch.equal(cor_a, cor_b)
    if n_sup:
        exact = grad[:n_sup].double() @ w.double()
        close(dh, exact, 2e-3)
