"""BASELINE configs 3 and 5 as whole units on the GPU against the CPU oracle.

Config 3: the attention-input block (engine.py:1073-1109 forward, 1296-1338 backward) at its
stated size: 4 packed sequences with lengths ~ U[128, 1024], hidden 1536, NF4 q/k/v, 12 q / 2 kv
heads of 128, RoPE theta 1e6 with per-sequence positions, LoRA r 16 / alpha 32 on q and v with
dropout 0.05 and the masks of the CUDA generator, forward and backward.

Config 5: the full-width Qwen2.5-1.5B step (hidden 1536, intermediate 8960, 12/2 heads, vocab
151,936, tied fp16 embedding) with 2 and with all 28 of its decoder layers, on one batch of 4
sequences with lengths ~ U[256, 1024], against oracle.step at the reference's whole-step
tolerance (test_kernels.py:314-400: loss relative 2e-3, LoRA gradients relative norm 2e-2).
"""

import numpy as np
import pytest
import torch

from oracle import philox
from oracle import step as OS

pytestmark = pytest.mark.gpu

DEV = "cuda"


def rel(a, b):
    a, b = a.detach().cpu().double(), b.detach().cpu().double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _lengths(lo, hi, rows, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, (rows,), generator=g).tolist()


def _batch(lengths, vocab, seed):
    g = torch.Generator().manual_seed(seed)
    B, T = len(lengths), max(lengths)
    ids = torch.randint(0, vocab, (B, T), generator=g)
    mask = (torch.arange(T)[None] < torch.tensor(lengths)[:, None]).long()
    ids = torch.where(mask.bool(), ids, 0)
    labels = torch.where(mask.bool(), ids, -100)
    for r, n in enumerate(lengths):
        labels[r, :n // 4] = -100  # the first quarter of each sequence is prompt
    return ids, mask, labels


def test_config3_attention_input_block(pkg):
    E = pkg.engine
    lengths = _lengths(128, 1024, 4, seed=3)
    print(f"config 3 block, lengths {lengths}", flush=True)
    cfg = E.Qwen2Config(num_hidden_layers=1, vocab_size=1024)
    model = E.random_qwen2(cfg, DEV, seed=3)
    spec = model.layers[0]
    H, HQ, HKV, D = cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads, \
        cfg.head_dim
    ids, mask, labels = _batch(lengths, cfg.vocab_size, seed=3)
    torch.cuda.manual_seed(33)
    packed = E.Packed(ids.to(DEV), mask.to(DEV), labels.to(DEV), model.rope, model.dropout,
                      model.dropout_p, lengths=lengths)
    n = packed.n
    seeds = (packed.draw(H), packed.draw(H))
    g = torch.Generator().manual_seed(4)
    h = torch.randn(n, H, generator=g)
    dq = torch.randn(n, HQ, D, generator=g).half()
    dk = torch.randn(n, HQ, D, generator=g).half()  # per q head, as the attention returns them
    dv = torch.randn(n, HQ, D, generator=g).half()
    lora = [t.detach().half() for t in spec.lora_params()]
    lora_t = [t.t().contiguous() for t in lora]
    q, k, v, saved = E.attn_input_fwd(spec, h.to(DEV), packed, lora, seeds)
    dh, dh16, (dA_q, dB_q, dA_v, dB_v) = E.attn_input_bwd(
        spec, dq.to(DEV), dk.to(DEV), dv.to(DEV), h.to(DEV), saved, packed, lora_t, seeds)
    torch.cuda.synchronize()

    cpu = OS.CpuQwen2(model).layers[0]
    T = ids.shape[1]
    tok = packed.tok.cpu()
    elems = (tok[:, None] * H + torch.arange(H)[None, :]).reshape(-1).numpy()
    p = model.dropout_p
    masks = tuple(torch.from_numpy(philox.keep_mask(elems, packed.drop_seed, c,
                                                    packed.drop_threads, np.float32(1 - p), 4))
                  .view(n, H) for c in seeds)
    kscale = float(np.float32(1.0 / (1 - p)))
    cos, sin = OS.rope_cos_sin(packed.pos.cpu().long(), D, cfg.rope_theta)
    hr = h.clone().requires_grad_()
    qo, ko, vo = OS.attn_input(cpu, hr, masks, kscale, cos, sin, HQ, HKV, D, cfg.rms_norm_eps)
    assert rel(q, qo) < 1e-3 and rel(k, ko) < 1e-3 and rel(v, vo) < 1e-3
    rep = HQ // HKV
    loss = (qo * dq.float()).sum() + (ko.repeat_interleave(rep, 1) * dk.float()).sum() \
        + (vo.repeat_interleave(rep, 1) * dv.float()).sum()
    loss.backward()
    assert rel(dh, hr.grad) < 1e-2
    assert torch.equal(dh16.cpu(), dh.cpu().half())
    leaves = [cpu.lora["q"][0], cpu.lora["q"][1], cpu.lora["v"][0], cpu.lora["v"][1]]
    for got, leaf in zip((dA_q, dB_q, dA_v, dB_v), leaves):
        assert rel(got, leaf.grad) < 2e-2, rel(got, leaf.grad)
    assert T == max(lengths)


def _config5_step(pkg, layers, overstate=0):
    """Loss and every LoRA gradient of the full-width 1.5B step (`layers` decoder layers, per-layer
    recompute) against the oracle. overstate: the caller's supervised-token count exceeds the
    batch's by this much (the step must still give the oracle's gradients; metadata_ok
    reports the mismatch)."""
    E = pkg.engine
    lengths = _lengths(256, 1024, 4, seed=5)
    print(f"config 5 step, {layers} layers, lengths {lengths}, n_supervised +{overstate}",
          flush=True)
    cfg = E.Qwen2Config(num_hidden_layers=layers)
    model = E.random_qwen2(cfg, DEV, seed=5)
    model.keep_all = False  # per-layer recompute, as config 5 states
    ids, mask, labels = _batch(lengths, cfg.vocab_size, seed=5)
    denom = float((labels[:, 1:] != -100).sum())
    torch.cuda.manual_seed(55)
    gen = model.dropout.gen
    seed, offset = gen.initial_seed(), gen.get_offset()
    loss, packed, _ = model.step(ids.to(DEV), mask.to(DEV), labels.to(DEV), denom,
                                 lengths=lengths, n_supervised=int(denom) + overstate)
    # fp16 training scales the loss (GradScaler's 2^16, as the trainer): unscaled, the
    # per-token gradients of a 151,936-way softmax over ~2,000 tokens sit in fp16's subnormal
    # range inside the layers' fp16 products
    scale = 2.0**16
    (loss * scale).backward()
    torch.cuda.synchronize()
    assert bool(packed.metadata_ok) == (overstate == 0)
    print(f"gpu loss {loss.item():.6f}; oracle...", flush=True)
    cpu = OS.CpuQwen2(model)
    ref, _ = OS.forward_loss(cpu, ids, mask, labels, denom, drop_seed=seed, drop_offset=offset,
                             drop_G=model.dropout.max_blocks * 256, p=model.dropout_p, vec=4)
    ref.backward()
    print(f"oracle loss {ref.item():.6f}", flush=True)
    assert abs(loss.item() - ref.item()) <= 2e-3 * abs(ref.item())
    for i, (g_gpu, leaf) in enumerate(zip(model.parameters(), cpu.lora_leaves())):
        r = rel(g_gpu.grad / scale, leaf.grad)
        assert r < 2e-2, (i, r)


@pytest.mark.parametrize("overstate", [0, 41])
def test_config5_full_width_step(pkg, overstate):
    _config5_step(pkg, 2, overstate)


def test_config5_28_layer_step(pkg):
    """The whole config-5 model: 28 layers of the full-width step against oracle.step (about half
    a minute of the host's cores for the oracle)."""
    _config5_step(pkg, 28)
