"""The LM head over the vocabulary in pieces: mean cross-entropy of
logits = hn E^T with the online-softmax state carried across pieces of `piece` columns, the
gradient w.r.t. the head input hn, and w.r.t. the tied embedding E.

Pass 1 is the reference's streamed head (_head_streamed, engine.py:1498-1547): per piece, the
logits GEMM, qlora_ce_piece (state update; supervised rows' logits overwritten with
fp16(e^(x - m))), and the fp32 accumulation acc = acc * alpha + P~ E_piece; qlora_ce_finish then
gives loss, entropy, accuracy and dhn = fp16(acc / s - E[target]). The reference's embedding is
frozen, so it has no pass 2: here, per piece, the logits are recomputed, qlora_ce_grad turns the
supervised rows into fp16(e^(x - lse) - onehot) (the whole-row kernel's gradient, bit for bit)
and dE[piece] = G^T hn in fp32. Rows are processed supervised-first (engine.py:731).
"""

import torch

from .ops import _ce_finish, _ce_grad, _ce_piece

PIECE = 8192


class HeadResult:
    """loss (0-d fp32, sum of tok_loss / denom), dhn fp32 [T, H] (d loss / d hn), dE fp32 [V, H]
    or None, and the per-token tok_loss, entropy, correct in the input row order."""


def chunked_head(hn, E, targets, denom, piece=PIECE, want_dE=True):
    """hn fp16 [T, H] (the normed hidden state), E fp16 [V, H], targets int64 [T] (-100 =
    ignored), denom = the loss normaliser (supervised tokens)."""
    if hn.dtype != torch.float16 or E.dtype != torch.float16 or targets.dtype != torch.int64:
        raise ValueError("hn and E must be fp16, targets int64")
    if hn.dim() != 2 or E.dim() != 2 or E.shape[1] != hn.shape[1] or targets.shape != hn.shape[:1]:
        raise ValueError("hn [T, H], E [V, H], targets [T]")
    if piece % 4096:
        raise ValueError("pieces must be multiples of 4096 columns (the CE block)")
    T, H = hn.shape
    V = E.shape[0]
    dev = hn.device
    sup = targets >= 0
    order = torch.argsort((~sup).to(torch.int8), stable=True)
    n_sup = int(sup.sum())
    hp = hn.index_select(0, order).contiguous()
    tg = targets.index_select(0, order).contiguous()
    state = torch.full((T, 4), float("-inf"), device=dev, dtype=torch.float32)
    state[:, 1:3] = 0.0
    best_idx = torch.zeros((T,), device=dev, dtype=torch.int32)
    xt = torch.zeros((T,), device=dev, dtype=torch.float32)
    m = max(n_sup, 1)
    alpha = torch.empty((m,), device=dev, dtype=torch.float32)
    acc = torch.zeros((m, H), device=dev, dtype=torch.float32)
    wt = torch.zeros((m, H), device=dev, dtype=torch.float16)
    for v0 in range(0, V, piece):
        w = E[v0:v0 + piece]
        logits = hp @ w.t()
        _ce_piece(logits, w, tg, state, best_idx, xt, alpha, wt, v0, n_sup)
        if n_sup:
            acc[:n_sup].mul_(alpha[:n_sup, None])
            torch.addmm(acc[:n_sup], logits[:n_sup], w, out_dtype=torch.float32,
                        out=acc[:n_sup])
        del logits
    tok_loss = torch.empty((T,), device=dev, dtype=torch.float32)
    entropy = torch.empty((T,), device=dev, dtype=torch.float32)
    correct = torch.empty((T,), device=dev, dtype=torch.int32)
    dhn16 = torch.empty((m, H), device=dev, dtype=torch.float16)
    _ce_finish(state, best_idx, xt, tg, tok_loss, entropy, correct, acc, wt, dhn16, n_sup)
    del acc, wt, alpha
    inv = 1.0 / float(denom) if float(denom) else float("nan")
    dE = None
    if want_dE:
        dE = torch.zeros((V, H), device=dev, dtype=torch.float32)
        if n_sup:
            hs = hp[:n_sup]
            for v0 in range(0, V, piece):
                w = E[v0:v0 + piece]
                g = hp @ w.t()  # the same GEMM as pass 1, so the same logits
                _ce_grad(g, tg, state, v0, n_sup)
                torch.addmm(dE[v0:v0 + w.shape[0]], g[:n_sup].t(), hs, beta=0.0, alpha=inv,
                            out_dtype=torch.float32, out=dE[v0:v0 + w.shape[0]])
                del g
    dhn = torch.zeros((T, H), device=dev, dtype=torch.float32)
    if n_sup:
        dhn.index_copy_(0, order[:n_sup], dhn16[:n_sup].float() * inv)
    r = HeadResult()
    r.loss = tok_loss.sum() * inv
    r.dhn, r.dE = dhn, dE
    unsort = torch.empty_like(order)
    unsort[order] = torch.arange(T, device=dev)
    r.tok_loss = tok_loss.index_select(0, unsort)
    r.entropy = entropy.index_select(0, unsort)
    r.correct = correct.index_select(0, unsort)
    r.n_supervised = n_sup
    return r


def full_head(hn, E, targets, denom, want_dE=True):
    """The same outputs from whole-row logits [T, V] (one GEMM, qlora_ce in place, G E and
    G^T hn): the layout the step's head uses when the logits fit in memory."""
    from .ops import _ce
    T, H = hn.shape
    dev = hn.device
    logits = hn @ E.t()
    tok_loss = torch.empty((T,), device=dev, dtype=torch.float32)
    entropy = torch.empty((T,), device=dev, dtype=torch.float32)
    correct = torch.empty((T,), device=dev, dtype=torch.int32)
    _ce(logits, targets, tok_loss, entropy, correct, zero_unsupervised=True)
    inv = 1.0 / float(denom) if float(denom) else float("nan")
    r = HeadResult()
    r.loss = tok_loss.sum() * inv
    r.dhn = torch.mm(logits, E, out_dtype=torch.float32) * inv
    r.dE = torch.mm(logits.t(), hn, out_dtype=torch.float32) * inv if want_dE else None
    r.tok_loss, r.entropy, r.correct = tok_loss, entropy, correct
    r.n_supervised = int((targets >= 0).sum())
    return r
