"""Device-only packing and the step captured as a HIP graph (engine.Packed(padded=True),
engine.StepGraph). The padded step equals the CPU oracle step on the real tokens (the reference's
whole-step tolerance, test_kernels.py:314-400) and the unpadded step; a captured step replayed on
new batches, with eager work and synchronisation between the replays, equals the eager padded
step bit for bit, dropout masks included, and moves the dropout generator as that step does."""

import pytest
import torch

from oracle import step as OS

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _tiny(pkg, layers=2, dropout=0.05, H=256, HQ=4, HKV=2, D=64, r=16, I=640):
    cfg = pkg.engine.Qwen2Config(hidden_size=H, intermediate_size=I, num_hidden_layers=layers,
                                 num_attention_heads=HQ, num_key_value_heads=HKV, head_dim=D,
                                 vocab_size=3072, lora_dropout=dropout, lora_r=r,
                                 lora_alpha=2 * r)
    return pkg.engine.random_qwen2(cfg, DEV, seed=3)


def _batch(lengths, T, vocab, seed):
    g = torch.Generator().manual_seed(seed)
    B = len(lengths)
    ids = torch.randint(0, vocab, (B, T), generator=g)
    mask = (torch.arange(T)[None, :] < torch.tensor(lengths)[:, None]).long()
    ids = torch.where(mask.bool(), ids, torch.zeros_like(ids))
    labels = torch.where(mask.bool(), ids, torch.full_like(ids, -100))
    labels[:, :2] = -100
    return ids, mask, labels


def _grads(model):
    return [p.grad.detach().clone() for p in model.parameters()]


def _clear(model):
    for p in model.parameters():
        p.grad = None


def test_padded_step_matches_oracle_and_unpadded_step(pkg):
    model = _tiny(pkg)
    model.keep_all = False
    lengths, T = [17, 60, 33, 5], 64
    ids, mask, labels = _batch(lengths, T, model.cfg.vocab_size, 0)
    denom = float((labels[:, 1:] != -100).sum())
    cpu = OS.CpuQwen2(model)
    gen = model.dropout.gen
    torch.cuda.manual_seed(99)
    seed, offset = gen.initial_seed(), gen.get_offset()
    loss_u, _, _ = model.step(ids.to(DEV), mask.to(DEV), labels.to(DEV), denom)
    loss_u.backward()
    g_u = _grads(model)
    after = gen.get_offset()
    _clear(model)
    gen.set_offset(offset)
    loss_p, packed, stats = model.step(ids.to(DEV), mask.to(DEV), labels.to(DEV), denom,
                                       padded=True)
    loss_p.backward()
    g_p = _grads(model)
    assert gen.get_offset() == after  # the same dropout calls, drawn the same way
    assert bool(packed.metadata_ok) and packed.n == len(lengths) * T
    ref, _ = OS.forward_loss(cpu, ids, mask, labels, denom, drop_seed=seed, drop_offset=offset,
                             drop_G=model.dropout.max_blocks * 256, p=model.dropout_p, vec=4)
    ref.backward()
    assert abs(loss_p.item() - ref.item()) <= 2e-3 * abs(ref.item())
    assert abs(loss_p.item() - loss_u.item()) <= 1e-4 * abs(loss_u.item())
    for a, b, leaf in zip(g_p, g_u, cpu.lora_leaves()):
        want = leaf.grad.double()
        assert ((a.cpu().double() - want).norm() / want.norm()).item() < 2e-2
        assert ((a - b).double().norm() / b.double().norm()).item() < 5e-3
    # per-token losses of the real tokens: those of the unpadded step's rows
    real = mask.reshape(-1).bool().to(DEV)
    tok_loss = torch.empty_like(stats.tok_loss).index_copy_(0, stats.order, stats.tok_loss)
    sup = packed.targets >= 0
    assert bool((tok_loss[~sup] == 0).all()) and bool(sup[~real].logical_not().all())


@pytest.mark.parametrize("keep_all", [False, True])
def test_graph_replay_equals_eager_padded_step(pkg, keep_all):
    model = _tiny(pkg)
    model.keep_all = keep_all
    B, T = 3, 64
    torch.cuda.manual_seed(5)
    graph = pkg.engine.StepGraph(model, B, T)
    gen = model.dropout.gen
    params = model.parameters()
    for k, lengths in enumerate(([64, 30, 7], [12, 50, 64], [1, 2, 40])):
        print(f"replay {k}: keep_all={keep_all} lengths={lengths}", flush=True)
        ids, mask, labels = (t.to(DEV) for t in _batch(lengths, T, model.cfg.vocab_size, 10 + k))
        denom = float((labels[:, 1:] != -100).sum())
        scale = 2.0 ** (4 + k)
        # the eager padded step with the same device denominator and loss scale
        offset = gen.get_offset()
        _clear(model)
        d = torch.tensor(denom, device=DEV)
        s = torch.tensor(scale, device=DEV)
        loss_e, _, _ = model.step(ids, mask, labels, d, padded=True)
        (loss_e * s).backward()
        g_e = _grads(model)
        loss_e = loss_e.detach().clone()
        after = gen.get_offset()
        torch.cuda.synchronize()
        gen.set_offset(offset)
        _clear(model)
        loss_g = graph.replay(ids, mask, labels, denom, scale)
        torch.cuda.synchronize()
        assert gen.get_offset() == after
        assert torch.equal(loss_g, loss_e), (loss_g.item(), loss_e.item())
        for a, b in zip([p.grad for p in params], g_e):
            assert torch.equal(a, b)
    with pytest.raises(ValueError):
        graph.replay(ids[:, :32], mask[:, :32], labels[:, :32], 1.0)


def test_graph_replay_with_k_sliced_gemm_tail(pkg):
    """The forward's SwiGLU product on the package GEMM with a K-sliced last round (I = 8960:
    70 column tiles; 4 x 256 tokens: 280 tiles, the 24 past the first round of 256 CUs in K
    slices through a workspace) captured and replayed equals the eager padded step bit for
    bit."""
    model = _tiny(pkg, I=8960)
    B, T = 4, 256
    M, I, H = B * T, 8960, 256
    assert pkg.linear.hgemm_workspace(M, I, H, 3, 1) > 0
    torch.cuda.manual_seed(7)
    graph = pkg.engine.StepGraph(model, B, T)
    gen = model.dropout.gen
    params = model.parameters()
    lengths = [256, 200, 100, 256]
    ids, mask, labels = (t.to(DEV) for t in _batch(lengths, T, model.cfg.vocab_size, 21))
    denom = float((labels[:, 1:] != -100).sum())
    offset = gen.get_offset()
    _clear(model)
    loss_e, _, _ = model.step(ids, mask, labels, torch.tensor(denom, device=DEV), padded=True)
    (loss_e * torch.tensor(8.0, device=DEV)).backward()
    g_e = _grads(model)
    loss_e = loss_e.detach().clone()
    torch.cuda.synchronize()
    gen.set_offset(offset)
    _clear(model)
    loss_g = graph.replay(ids, mask, labels, denom, 8.0)
    torch.cuda.synchronize()
    assert torch.equal(loss_g, loss_e), (loss_g.item(), loss_e.item())
    for a, b in zip([p.grad for p in params], g_e):
        assert torch.equal(a, b)
