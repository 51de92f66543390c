"""The LM head over the vocabulary in pieces: mean cross-entropy of
logits = hn E^T with the online-softmax state carried across pieces of `piece` columns, the
gradient w.r.t. the head input hn, and w.r.t. the tied embedding E. Every product runs on the
package's MFMA GEMM (linear.hgemm for the fp16 logits, linear.gemm_f32 for the fp32 products).

Pass 1 is the reference's streamed head (_head_streamed, engine.py:1498-1547): per piece, the
logits GEMM, qlora_ce_piece (state update; supervised rows' logits overwritten with
fp16(e^(x - m))), and the fp32 accumulation acc = acc * alpha + P~ E_piece (one GEMM whose
epilogue scales each row of acc by alpha); qlora_ce_finish then gives loss, entropy, accuracy
and dhn = fp16(acc / s - E[target]). The reference's embedding is frozen, so it has no pass 2:
here, per piece, the logits are recomputed, qlora_ce_grad turns the supervised rows into
fp16(e^(x - lse) - onehot) (the whole-row kernel's gradient, bit for bit) and dE[piece] = G^T hn
in fp32 (the GEMM's transposed-A form, reducing over the rows in blocks of 128: the rows past
the supervised ones are zeroed in G). Rows are processed supervised-first (engine.py:731).
"""

import torch

from . import linear as L
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
    if E.shape[0] % 128 or hn.shape[1] % 128:
        raise ValueError("the vocabulary and the hidden size must be multiples of 128 (the "
                         "package GEMM's blocks; every Qwen2 size is)")
    T, H = hn.shape
    V = E.shape[0]
    dev = hn.device
    sup = targets >= 0
    order = torch.argsort((~sup).to(torch.int8), stable=True)
    n_sup = int(sup.sum())
    # rows padded to a multiple of 128 with zeros (their logits are zeros): the dE product
    # reduces over rows in blocks of 128
    Tp = -(-T // 128) * 128
    hp = torch.zeros((Tp, H), device=dev, dtype=torch.float16)
    hp[:T] = hn.index_select(0, order)
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
        logits = L.hgemm(hp, w, 0, tile=0)  # [Tp, piece]: the pass-2 GEMM's exact problem
        _ce_piece(logits[:T], w, tg, state, best_idx, xt, alpha, wt, v0, n_sup)
        if n_sup:  # acc = acc * alpha + P~ E_piece
            L.gemm_f32(logits[:n_sup], w, 1, row_scale=alpha[:n_sup], resid=acc[:n_sup],
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
        # every row of dE is written by its piece's product (zeros without supervised rows)
        dE = (torch.empty if n_sup else torch.zeros)((V, H), device=dev, dtype=torch.float32)
        if n_sup:
            kp = -(-n_sup // 128) * 128  # rows of the dE reduction (n_sup <= kp <= Tp)
            for v0 in range(0, V, piece):
                w = E[v0:v0 + piece]
                g = L.hgemm(hp, w, 0, tile=0)  # the same GEMM as pass 1, so the same logits
                _ce_grad(g[:T], tg, state, v0, n_sup)
                g[n_sup:kp].zero_()
                L.gemm_f32(g[:kp], hp[:kp], 2, alpha=inv, out=dE[v0:v0 + w.shape[0]])
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
    G^T hn on the package GEMM in fp32): the layout the step's head uses when the logits fit in
    memory."""
    from .ops import _ce
    T, H = hn.shape
    if E.shape[0] % 128 or H % 128:
        raise ValueError("the vocabulary and the hidden size must be multiples of 128 (the "
                         "package GEMM's blocks; every Qwen2 size is)")
    dev = hn.device
    Tp = -(-T // 128) * 128  # zero rows: the dE product reduces over rows in blocks of 128
    hp = hn
    if Tp != T:
        hp = torch.zeros((Tp, H), device=dev, dtype=torch.float16)
        hp[:T] = hn
    logits = L.hgemm(hp, E, 0, tile=0)
    tok_loss = torch.empty((T,), device=dev, dtype=torch.float32)
    entropy = torch.empty((T,), device=dev, dtype=torch.float32)
    correct = torch.empty((T,), device=dev, dtype=torch.int32)
    _ce(logits[:T], targets, tok_loss, entropy, correct, zero_unsupervised=True)
    inv = 1.0 / float(denom) if float(denom) else float("nan")
    r = HeadResult()
    r.loss = tok_loss.sum() * inv
    r.dhn = L.gemm_f32(logits[:T], E, 1, alpha=inv)
    r.dE = L.gemm_f32(logits, hp, 2, alpha=inv) if want_dE else None
    r.tok_loss, r.entropy, r.correct = tok_loss, entropy, correct
    r.n_supervised = int((targets >= 0).sum())
    return r
