"""CPU restatement (plain PyTorch, fp32) of the reference's fused elementwise/reduction kernels.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Each function follows one Triton kernel of solution/kernels.py, with fp16 rounding exactly where
the kernel stores fp16 and fp32 everywhere else. Inputs/outputs are CPU tensors.

Pins (tests/test_oracle_ops.py), none of which retypes the formula below:
  rms_fwd / rms_bwd     torch autograd of y = w * x * rsqrt(mean x^2 + eps) (the reference's own
                        check, test_kernels.py:109-135) and a float64 evaluation; masks against
                        oracle.philox
  rope_fwd / rope_bwd   complex-number rotation (x1 + i x2) * e^{i pos theta_k}, its conjugate for
                        the inverse, and autograd through torch's rotate_half form
                        (test_kernels.py:138-186)
  glu_fwd / glu_bwd     torch.nn.functional.silu + autograd (test_kernels.py:189-205)
  ce / ce_piece / ce_finish   torch.nn.functional.cross_entropy(ignore_index=-100),
                        torch.logsumexp, softmax entropy, argmax (test_kernels.py:208-234);
                        piece-wise == whole-row state (test_host_head.py:38-88); the target =
                        argmax known answer (test_kernels.py:217, 233)
"""

import numpy as np
import torch

from . import philox


def _keep(tok, H, n, seed, ctr, G, p_keep, vec):
    elems = (tok.to(torch.int64)[:, None] * H + torch.arange(H)[None, :]).reshape(-1).numpy()
    return torch.from_numpy(philox.keep_mask(elems, seed, ctr, G, p_keep, vec)).view(n, H)


def rms_fwd(x, weight, eps, *, delta=None, write_y=True, tok=None, p=0.0, seed=0, ctrs=(0, 0),
            G=1, vec=4, drop_q=False, drop_v=False):
    """kernels.py:145-175 -> (xsum fp32, y fp16, yq fp16, yv fp16, rstd fp32)."""
    x = x.float()
    n, H = x.shape
    if delta is not None:
        x = x + delta.float()
    rstd = 1.0 / torch.sqrt((x * x).sum(dim=1) / H + eps)
    y = weight.float()[None, :] * (x * rstd[:, None])
    p_keep = np.float32(1.0 - p)
    scale = np.float32(1.0 / (1.0 - p))
    out = [x, y.half() if write_y else None, None, None, rstd]
    for slot, on, ctr in ((2, drop_q, ctrs[0]), (3, drop_v, ctrs[1])):
        if on:
            keep = _keep(tok, H, n, seed, ctr, G, p_keep, vec)
            out[slot] = torch.where(keep, y * float(scale), torch.zeros_like(y)).half()
    return tuple(out)


def rms_bwd(dy, x, rstd, weight, *, dres=None, tq=None, tv=None, tok=None, p=0.0, seed=0,
            ctrs=(0, 0), G=1, vec=4, grad_scale=1.0):
    """kernels.py:178-205 -> dx fp32."""
    x = x.float()
    n, H = x.shape
    g_in = dy.float().clone()
    p_keep = np.float32(1.0 - p)
    scale = float(np.float32(1.0 / (1.0 - p)))
    for t, ctr in ((tq, ctrs[0]), (tv, ctrs[1])):
        if t is not None:
            keep = _keep(tok, H, n, seed, ctr, G, p_keep, vec)
            g_in = g_in + torch.where(keep, t.float() * scale, torch.zeros_like(g_in))
    g = g_in * weight.float()[None, :]
    xhat = x * rstd[:, None]
    dx = rstd[:, None] * (g - xhat * ((g * xhat).sum(dim=1, keepdim=True) / H)) * grad_scale
    if dres is not None:
        dx = dx + dres.float()
    return dx


def rope_tables(positions, D, theta):
    """cos/sin [positions, D/2] fp32 of inv_freq = theta^(-2i/D) (test_kernels.py:154-156)."""
    inv = 1.0 / (theta ** (torch.arange(0, D, 2).float() / D))
    freqs = torch.arange(positions).float()[:, None] * inv[None, :]
    return freqs.cos().contiguous(), freqs.sin().contiguous()


def _rot(x1, x2, c, s):
    return x1 * c - x2 * s, x2 * c + x1 * s


def rope_fwd(qkv, lq, lv, cos, sin, pos, HQ, HKV, D, lora_scale, kv_heads=None):
    """kernels.py:212-264 -> q [n,HQ,D], k, v [n,kv_heads,D] fp16 (kv_heads=HQ: repeated)."""
    n = qkv.shape[0]
    half = D // 2
    kh = HQ if kv_heads is None else kv_heads
    f = qkv.float()
    q = f[:, :HQ * D].reshape(n, HQ, D)
    k = f[:, HQ * D:(HQ + HKV) * D].reshape(n, HKV, D)
    v = f[:, (HQ + HKV) * D:].reshape(n, HKV, D)
    if lq is not None:
        q = q + lq.float().reshape(n, HQ, D) * lora_scale
    if lv is not None:
        v = v + lv.float().reshape(n, HKV, D) * lora_scale
    c = cos[pos.long()][:, None, :]
    s = sin[pos.long()][:, None, :]
    q1, q2 = _rot(q[..., :half], q[..., half:], c, s)
    k1, k2 = _rot(k[..., :half], k[..., half:], c, s)
    qo = torch.cat([q1, q2], -1).half()
    ko = torch.cat([k1, k2], -1).half()
    vo = v.half()
    rep = kh // HKV
    return qo, ko.repeat_interleave(rep, dim=1), vo.repeat_interleave(rep, dim=1)


def rope_bwd(dq, dk, dv, cos, sin, pos, HQ, HKV, D):
    """kernels.py:267-306 -> dqkv [n, (HQ+2HKV)D] fp16; dk/dv may have HQ (repeated) or HKV
    heads."""
    n = dq.shape[0]
    half = D // 2
    rep = dk.shape[1] // HKV
    gk = dk.float().reshape(n, HKV, rep, D).sum(2)
    gv = dv.float().reshape(n, HKV, rep, D).sum(2)
    c = cos[pos.long()][:, None, :]
    s = sin[pos.long()][:, None, :]

    def inv(g):
        g1, g2 = g[..., :half], g[..., half:]
        return torch.cat([g1 * c + g2 * s, g2 * c - g1 * s], -1)

    out = torch.cat([inv(dq.float()).reshape(n, -1), inv(gk).reshape(n, -1),
                     gv.reshape(n, -1)], dim=1)
    return out.half()


def glu_fwd(gu, I):
    """kernels.py:312-321 -> m fp16."""
    g, u = gu[:, :I].float(), gu[:, I:].float()
    return (g / (1.0 + torch.exp(-g)) * u).half()


def glu_bwd(dm, gu, I):
    """kernels.py:324-336 -> new gu fp16 ([dg | du])."""
    g, u, d = gu[:, :I].float(), gu[:, I:].float(), dm.float()
    sig = 1.0 / (1.0 + torch.exp(-g))
    return torch.cat([d * u * sig * (1.0 + g * (1.0 - sig)), d * g * sig], dim=1).half()


def _argmax_first(x):
    """First index of the row maximum."""
    return torch.argmax(x, dim=1)  # torch returns the first maximal index


def ce(logits, targets, zero_unsupervised=True):
    """kernels.py:344-388 -> (tok_loss, entropy, correct, new logits fp16)."""
    x = logits.float()
    lse = torch.logsumexp(x, dim=1)
    p = torch.exp(x - lse[:, None])
    entropy = lse - (p * x).sum(1)
    valid = targets >= 0
    tgt = targets.clamp(min=0)
    xt = x.gather(1, tgt[:, None])[:, 0]
    loss = torch.where(valid, lse - xt, torch.zeros_like(lse))
    correct = (valid & (_argmax_first(x) == targets)).to(torch.int32)
    grad = p.clone()
    grad[torch.arange(x.shape[0]), tgt] -= valid.float()
    out = torch.where(valid[:, None], grad, torch.zeros_like(grad) if zero_unsupervised else x)
    return loss, entropy, correct, out.half()


def ce_state_init(n):
    """(state [n,4] = (-inf, 0, 0, -inf), best_idx, xt) before the first piece."""
    state = torch.tensor([float("-inf"), 0.0, 0.0, float("-inf")]).repeat(n, 1)
    return state, torch.zeros(n, dtype=torch.int32), torch.zeros(n)


def ce_piece(logits, w, targets, state, best_idx, xt, v0, n_sup):
    """kernels.py:401-450 on one piece; returns (state, best_idx, xt, alpha [n_sup],
    wt rows [n_sup, H] or None where not in the piece, new logits fp16)."""
    x = logits.float()
    n, width = x.shape
    m_old, s, t, best = state[:, 0], state[:, 1], state[:, 2], state[:, 3]
    pm = x.max(1).values
    m = torch.maximum(m_old, pm)
    a = torch.where(m_old == float("-inf"), torch.zeros_like(m), torch.exp(m_old - m))
    e = torch.exp(x - m[:, None])
    s = s * a + e.sum(1)
    t = t * a + (e * x).sum(1)
    arg = _argmax_first(x)
    take = pm > best
    best_idx = torch.where(take, (v0 + arg).to(torch.int32), best_idx)
    best = torch.maximum(best, pm)
    local = targets - v0
    inp = (targets >= 0) & (local >= 0) & (local < width)
    xt = torch.where(inp, x.gather(1, local.clamp(0, width - 1)[:, None])[:, 0], xt)
    state = torch.stack([m, s, t, best], 1)
    new = logits.clone()
    new[:n_sup] = e[:n_sup].half()
    wt = w[local.clamp(0, width - 1)[:n_sup]]
    return state, best_idx, xt, a[:n_sup], wt, inp[:n_sup], new


def ce_finish(state, best_idx, xt, targets, acc, wt, n_sup):
    """kernels.py:458-479 -> (tok_loss, entropy, correct, dh fp16 [n_sup, H])."""
    m, s, t = state[:, 0], state[:, 1], state[:, 2]
    lse = m + torch.log(s)
    entropy = lse - t / s
    valid = targets >= 0
    loss = torch.where(valid, lse - xt, torch.zeros_like(lse))
    correct = (valid & (best_idx.long() == targets)).to(torch.int32)
    dh = (acc[:n_sup] / s[:n_sup, None] - wt[:n_sup].float()).half()
    return loss, entropy, correct, dh


def mlp(x, w_gu, w_d, dy):
    """The MLP of a layer with the reference's fp16 rounding points (engine.py:1163-1179,
    1238-1293), fp32 products of fp16 values: gu = fp16(x W_gu^T), h = fp16(silu(g) u),
    y = fp16(h W_d^T); backward: dh = fp16(fp16(dy) W_d), [dg|du] = glu_bwd(dh, gu),
    dx = fp16([dg|du] W_gu). Returns (h, y, dx)."""
    f = lambda t: t.float()  # noqa: E731
    I = w_gu.shape[0] // 2
    gu = (f(x) @ f(w_gu).t()).half()
    h = glu_fwd(gu, I)
    y = (f(h) @ f(w_d).t()).half()
    dh = (f(dy.half()) @ f(w_d)).half()
    dgu = glu_bwd(dh, gu, I)
    dx = (f(dgu) @ f(w_gu)).half()
    return h, y, dx
