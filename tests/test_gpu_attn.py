"""The HIP varlen causal attention (qlora_attn_fwd/bwd) against fp32 autograd of
scaled_dot_product_attention per sequence on the CPU, at the reference's tolerances
(test_kernels.py:244-281: out 2e-3, dq/dk/dv 1e-2), including the reference's own case
(lengths 7, 130, 1, 64; 12 q heads over 2 kv heads; D 128), the config-3/5 shapes (lengths up to
1024), k/v in grouped and in repeated layout, head_dim 64, and the split of long key ranges over
several workgroups (qlora_attn_fwd_split / qlora_attn_bwd_split) at forced chunk sizes."""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


class _Packed:
    def __init__(self, lengths):
        self.cu_seqlens_host = [0, *torch.tensor(lengths).cumsum(0).tolist()]
        self.cu_seqlens = torch.tensor(self.cu_seqlens_host, device=DEV, dtype=torch.int32)
        self.max_len = max(lengths)


def _expand(x, group):
    n, kh, d = x.shape
    return x[:, :, None, :].expand(n, kh, group, d).reshape(n, kh * group, d)


def close(a, b, tol):
    torch.testing.assert_close(a.detach().cpu().float(), b.detach().cpu().float(), rtol=tol,
                               atol=tol)


def _reference(q, k, v, dout, lengths):
    """fp32 CPU autograd per sequence; k/v repeated to the q heads; dk/dv per q head."""
    group = q.shape[1] // k.shape[1]
    ke, ve = _expand(k.cpu().float(), group), _expand(v.cpu().float(), group)
    outs, lses, dqs, dks, dvs = [], [], [], [], []
    start = 0
    scale = q.shape[2] ** -0.5
    for length in lengths:
        sl = slice(start, start + length)
        qr = q[sl].cpu().float().transpose(0, 1).requires_grad_()
        kr = ke[sl].transpose(0, 1).requires_grad_()
        vr = ve[sl].transpose(0, 1).requires_grad_()
        ref = torch.nn.functional.scaled_dot_product_attention(qr, kr, vr, is_causal=True)
        g = torch.autograd.grad(ref, (qr, kr, vr), dout[sl].cpu().float().transpose(0, 1))
        s = (qr.detach() @ kr.detach().transpose(1, 2)) * scale
        s = s.masked_fill(torch.ones(length, length, dtype=torch.bool).triu(1), float("-inf"))
        lses.append(torch.logsumexp(s, dim=-1))  # [HQ, L]
        outs.append(ref.detach().transpose(0, 1))
        dqs.append(g[0].transpose(0, 1))
        dks.append(g[1].transpose(0, 1))
        dvs.append(g[2].transpose(0, 1))
        start += length
    return (torch.cat(outs), torch.cat(lses, dim=1), torch.cat(dqs), torch.cat(dks),
            torch.cat(dvs))


def _run(pkg, lengths, HQ, KH, D, seed=0, expand=False, chunk=None):
    torch.manual_seed(seed)
    n = sum(lengths)
    q = torch.randn(n, HQ, D, device=DEV, dtype=torch.float16)
    k = torch.randn(n, KH, D, device=DEV, dtype=torch.float16)
    v = torch.randn(n, KH, D, device=DEV, dtype=torch.float16)
    dout = torch.randn(n, HQ, D, device=DEV, dtype=torch.float16)
    packed = _Packed(lengths)
    if chunk is not None:  # force the split (0: none) instead of the cost model's choice
        packed._attn_plans = {("fwd", HQ, KH): chunk, ("dq", HQ, KH): chunk}
    kk, vv = (_expand(k, HQ // KH).contiguous(), _expand(v, HQ // KH).contiguous()) if expand \
        else (k, v)
    print(f"attn lengths={lengths} HQ={HQ} KH={KH} D={D} expand={expand} chunk={chunk}",
          flush=True)
    out, lse, _, _ = pkg.ops._attn_fwd(q, kk, vv, packed, D ** -0.5)
    dq, dk, dv = pkg.ops._attn_bwd(dout, q, kk, vv, out, lse, None, None, packed, D ** -0.5)
    torch.cuda.synchronize()
    ro, rl, rdq, rdk, rdv = _reference(q, k, v, dout, lengths)
    close(out, ro, 2e-3)
    close(lse, rl, 1e-4)
    close(dq, rdq, 1e-2)
    close(dk, rdk, 1e-2)
    close(dv, rdv, 1e-2)
    return out, lse, dq, dk, dv


def test_reference_case(pkg):
    """test_kernels.py:244-281: lengths 7, 130, 1, 64; 12/2 heads; D 128."""
    _run(pkg, [7, 130, 1, 64], 12, 2, 128)


@pytest.mark.parametrize("lengths", [[1], [32], [33], [64, 65], [63, 1, 97], [200, 5, 129]])
def test_block_edges(pkg, lengths):
    _run(pkg, lengths, 12, 2, 128, seed=len(lengths))


def test_repeated_kv_layout(pkg):
    """k/v already repeated to the q heads ([n, HQ, D], the reference's _expand_kv layout)."""
    _run(pkg, [7, 130, 1, 64], 12, 2, 128, expand=True)


def test_head_dim_64(pkg):
    _run(pkg, [17, 60, 33, 5], 4, 2, 64)


def test_config_shapes(pkg):
    """Config 3/5 shapes: 4 sequences, lengths in [128, 1024] (incl. the maximum)."""
    _run(pkg, [1024, 301, 777, 128], 12, 2, 128, seed=5)


def test_empty_sequences(pkg):
    """Zero-length rows inside cu_seqlens are skipped; n == 0 launches nothing."""
    _run(pkg, [5, 0, 40], 12, 2, 128, seed=7)
    packed = _Packed([0])
    q = torch.empty(0, 12, 128, device=DEV, dtype=torch.float16)
    k = torch.empty(0, 2, 128, device=DEV, dtype=torch.float16)
    out, lse, _, _ = pkg.ops._attn_fwd(q, k, k, packed, 128 ** -0.5)
    assert out.shape == (0, 12, 128) and lse.shape == (12, 0)


@pytest.mark.parametrize("chunk", [64, 128, 192, 512])
def test_split_key_ranges(pkg, chunk):
    """Key ranges cut into chunks of `chunk` keys (several workgroups per query tile and a merge
    kernel), incl. tiles of one chunk, a sequence of 1 and the longest row."""
    _run(pkg, [1024, 301, 777, 1, 128, 65], 12, 2, 128, seed=chunk, chunk=chunk)


def test_split_head_dim_64(pkg):
    _run(pkg, [300, 17, 129], 4, 2, 64, seed=3, chunk=64)


def test_split_is_deterministic_and_matches_unsplit(pkg):
    """The merge order is fixed: two split runs agree bit for bit, and with the unsplit kernels
    to fp32 summation order."""
    a = _run(pkg, [700, 300, 40], 12, 2, 128, seed=11, chunk=128)
    b = _run(pkg, [700, 300, 40], 12, 2, 128, seed=11, chunk=128)
    c = _run(pkg, [700, 300, 40], 12, 2, 128, seed=11, chunk=0)
    for x, y, z in zip(a, b, c):
        assert torch.equal(x, y)
        close(x, z, 2e-3)


def test_concurrent_backward_matches_sequential(pkg):
    """A batch of few long sequences runs dK/dV on a second stream beside dQ (delta from its own
    kernel); a full batch runs them one after the other (delta formed by dQ). Sequences are
    independent, so the rows of the shared sequences agree bit for bit."""
    HQ, KH, D = 12, 2, 128
    few, extra = [1024, 600], [1024] * 10
    n_few, n = sum(few), sum(few) + sum(extra)
    g = torch.Generator(device=DEV).manual_seed(21)
    q, dout = (torch.randn(n, HQ, D, device=DEV, generator=g).half() for _ in range(2))
    k, v = (torch.randn(n, KH, D, device=DEV, generator=g).half() for _ in range(2))
    res = []
    for lengths, rows in ((few, n_few), (few + extra, n)):
        print(f"attn concurrent/sequential lengths={lengths}", flush=True)
        packed = _Packed(lengths)
        packed._attn_plans = {("fwd", HQ, KH): 0, ("dq", HQ, KH): 0}  # no key-range split
        qq, kk, vv, dd = q[:rows], k[:rows], v[:rows], dout[:rows]
        out, lse, _, _ = pkg.ops._attn_fwd(qq, kk, vv, packed, D ** -0.5)
        dq, dk, dv = pkg.ops._attn_bwd(dd, qq, kk, vv, out, lse, None, None, packed, D ** -0.5)
        torch.cuda.synchronize()
        res.append((out[:n_few], lse[:, :n_few], dq[:n_few], dk[:n_few], dv[:n_few]))
    for x, y in zip(*res):
        assert torch.equal(x, y)


@pytest.mark.parametrize("HQ,KH,D", [(14, 2, 64), (16, 2, 128), (28, 4, 128), (8, 8, 64)])
def test_concurrent_backward_other_shapes(pkg, HQ, KH, D):
    """The concurrent backward (few sequences, max_len >= 512: dK/dV beside dQ, delta from its
    own kernel) at other head sizes and group counts (Qwen2 0.5B 14/2 x 64, 3B 16/2, 7B 28/4,
    and one q head per kv head) against fp32 SDPA, key ranges unsplit."""
    _run(pkg, [600, 300], HQ, KH, D, seed=HQ + D, chunk=0)
