"""Packing of a right-padded batch (engine.py:705-751) on the CPU: the host-side lengths path
and the one-read path agree, the supervised count equals the packed targets', and a left-padded
mask is refused (engine.py:709-717)."""

import importlib

import pytest
import torch

pkg = importlib.import_module("hack-fe30cb28-opus-5-5-ultracode_amd")
E = pkg.engine


def _batch(lengths, T, seed):
    g = torch.Generator().manual_seed(seed)
    B = len(lengths)
    ids = torch.randint(0, 1000, (B, T), generator=g)
    mask = (torch.arange(T)[None, :] < torch.tensor(lengths)[:, None]).long()
    labels = torch.where(torch.rand(B, T, generator=g) < 0.7, ids, torch.full_like(ids, -100))
    labels[:, 0] = -100
    return ids, mask, labels


def _packed(ids, mask, labels, **kw):
    rope = E.RopeTable(1e6, 128, torch.device("cpu"))
    return E.Packed(ids, mask, labels, rope, None, 0.0, **kw)


@pytest.mark.parametrize("lengths,T", [([5, 9, 1, 9], 9), ([3, 0, 7], 8), ([16], 16)])
def test_one_read_matches_host_lengths(lengths, T):
    ids, mask, labels = _batch(lengths, T, sum(lengths))
    a = _packed(ids, mask, labels)
    b = _packed(ids, mask, labels, lengths=lengths)
    assert a.lengths == lengths and a.n == sum(lengths) and a.max_len == max(lengths)
    assert torch.equal(a.tok, b.tok) and torch.equal(a.targets, b.targets)
    assert a.n_supervised == b.n_supervised == int((a.targets >= 0).sum())
    assert a.cu_seqlens_host == b.cu_seqlens_host
    # the target of a row's last token is the label after it (the padding's), as the reference
    want = []
    for r, n in enumerate(lengths):
        for p in range(n):
            want.append(int(labels[r, p + 1]) if p + 1 < T else -100)
    assert a.targets.tolist() == want


def test_left_padding_is_refused():
    ids, mask, labels = _batch([4, 6], 6, 1)
    mask = mask.flip(1)
    with pytest.raises(E.UnsupportedBatch):
        _packed(ids, mask, labels)
