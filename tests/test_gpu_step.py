"""The whole step on the GPU against the CPU oracle step (autograd), and the varlen attention it
relies on against per-sequence SDPA (test_kernels.py:245-281, 314-400)."""

import pytest
import torch

from oracle import step as OS

pytestmark = pytest.mark.gpu

DEV = "cuda"


def close(a, b, tol):
    torch.testing.assert_close(a.detach().cpu().float(), b.detach().cpu().float(), rtol=tol,
                               atol=tol)


def test_varlen_attention_matches_sdpa(pkg):
    torch.manual_seed(0)
    lengths = [7, 130, 1, 64]
    HQ, D = 12, 128

    class P:
        pass

    packed = P()
    packed.cu_seqlens_host = [0, *torch.tensor(lengths).cumsum(0).tolist()]
    packed.cu_seqlens = torch.tensor(packed.cu_seqlens_host, device=DEV, dtype=torch.int32)
    packed.max_len = max(lengths)
    n = sum(lengths)
    q = torch.randn(n, HQ, D, device=DEV, dtype=torch.float16)
    k = torch.randn(n, HQ, D, device=DEV, dtype=torch.float16)
    v = torch.randn(n, HQ, D, device=DEV, dtype=torch.float16)
    scale = D ** -0.5
    out, lse, s, o = pkg.engine._attn_fwd(q, k, v, packed, scale)
    dout = torch.randn_like(q)
    dq, dk, dv = pkg.engine._attn_bwd(dout, q, k, v, out, lse, s, o, packed, scale)
    start = 0
    for length in lengths:
        sl = slice(start, start + length)
        qr = q[sl].float().cpu().transpose(0, 1).requires_grad_()
        kr = k[sl].float().cpu().transpose(0, 1).requires_grad_()
        vr = v[sl].float().cpu().transpose(0, 1).requires_grad_()
        ref = torch.nn.functional.scaled_dot_product_attention(qr, kr, vr, is_causal=True)
        g = torch.autograd.grad(ref, (qr, kr, vr), dout[sl].float().cpu().transpose(0, 1))
        close(out[sl], ref.transpose(0, 1), 2e-3)
        close(dq[sl], g[0].transpose(0, 1), 1e-2)
        close(dk[sl], g[1].transpose(0, 1), 1e-2)
        close(dv[sl], g[2].transpose(0, 1), 1e-2)
        start += length


def _tiny(pkg, layers=2, dropout=0.05, H=256, HQ=4, HKV=2, D=64, r=16):
    cfg = pkg.engine.Qwen2Config(hidden_size=H, intermediate_size=640, num_hidden_layers=layers,
                                 num_attention_heads=HQ, num_key_value_heads=HKV, head_dim=D,
                                 vocab_size=3072, lora_dropout=dropout, lora_r=r,
                                 lora_alpha=2 * r)
    return pkg.engine.random_qwen2(cfg, DEV, seed=3)


def _batch(lengths, vocab, prompt=3, seed=0):
    g = torch.Generator().manual_seed(seed)
    B, T = len(lengths), max(lengths)
    ids = torch.randint(0, vocab, (B, T), generator=g)
    mask = (torch.arange(T)[None] < torch.tensor(lengths)[:, None]).long()
    ids = torch.where(mask.bool(), ids, 0)
    labels = torch.where(mask.bool(), ids, -100)
    labels[:, :prompt] = -100
    return ids, mask, labels


@pytest.mark.parametrize("H,HQ,HKV,D,r", [(896, 14, 2, 64, 8), (512, 8, 1, 64, 32),
                                          (640, 10, 2, 64, 16), (512, 4, 1, 128, 64)])
def test_step_other_model_shapes(pkg, H, HQ, HKV, D, r):
    """Other Qwen2 family shapes through the whole step against the CPU oracle: 7 q heads per kv
    head with D 64 (Qwen2.5-0.5B: 14/2), 8 (3B, 72B), 5 (14B, 32B), D 128 with 4, and LoRA ranks
    8, 32, 64 beside 16."""
    print(f"step H={H} HQ={HQ} HKV={HKV} D={D} r={r}", flush=True)
    model = _tiny(pkg, H=H, HQ=HQ, HKV=HKV, D=D, r=r)
    model.keep_all = None
    cpu = OS.CpuQwen2(model)
    lengths = [17, 60, 33, 5]
    ids, mask, labels = _batch(lengths, model.cfg.vocab_size)
    denom = float((labels[:, 1:] != -100).sum())
    torch.cuda.manual_seed(99)
    gen = model.dropout.gen
    seed, offset = gen.initial_seed(), gen.get_offset()
    loss, _, _ = model.step(ids.to(DEV), mask.to(DEV), labels.to(DEV), denom)
    loss.backward()
    torch.cuda.synchronize()
    ref, _ = OS.forward_loss(cpu, ids, mask, labels, denom, drop_seed=seed, drop_offset=offset,
                             drop_G=model.dropout.max_blocks * 256, p=model.dropout_p, vec=4)
    ref.backward()
    assert abs(loss.item() - ref.item()) <= 2e-3 * abs(ref.item())
    for g_gpu, leaf in zip(model.parameters(), cpu.lora_leaves()):
        ga, gb = g_gpu.grad.detach().cpu().double(), leaf.grad.double()
        rel = (ga - gb).norm() / gb.norm().clamp_min(1e-30)
        assert rel < 2e-2, rel.item()


def test_kept_tensors_equal_recomputing_them(pkg):
    """A recomputing layer keeps its [gate|up] product (keep_gu), its attention tensors
    (keep_attn: q, k, v, output, log-sum-exp, o_proj output), its dequantized weights
    (keep_weights_recompute) and its input norm's dropout masks as bits (keep_bits) from the
    forward instead of forming them again in its backward, whose post-attention norm may be
    formed inside that norm's backward (norm_in_bwd), and its LoRA inputs' rank-r products
    (keep_lora_x): the same loss and LoRA gradients bit for bit in every combination (what is
    kept is the same bits as what the recompute forms)."""
    out = []
    for keep_gu, keep_attn, keep_w, keep_b, nib, kx in ((True, True, True, True, True, True),
                                                        (False, False, False, False, False,
                                                         False),
                                                        (True, False, True, False, True, True),
                                                        (False, True, False, True, True, True),
                                                        (True, True, False, True, False, False)):
        model = _tiny(pkg, H=512, HQ=8, HKV=2, D=64)
        model.keep_all, model.keep_gu, model.keep_attn = False, keep_gu, keep_attn
        model.keep_weights_recompute, model.keep_bits, model.norm_in_bwd = keep_w, keep_b, nib
        model.keep_lora_x = model.parts_to_norm = kx
        lengths = [17, 60, 33, 5]
        ids, mask, labels = _batch(lengths, model.cfg.vocab_size)
        denom = float((labels[:, 1:] != -100).sum())
        torch.cuda.manual_seed(7)
        loss, _, _ = model.step(ids.to(DEV), mask.to(DEV), labels.to(DEV), denom)
        loss.backward()
        torch.cuda.synchronize()
        out.append((loss.item(), [p.grad.clone() for p in model.parameters()]))
    for other in out[1:]:
        assert out[0][0] == other[0]
        for a, b in zip(out[0][1], other[1]):
            assert torch.equal(a, b)


@pytest.mark.parametrize("lengths,keep_all", [([17, 60, 33, 5], False), ([4], False),
                                              ([40, 40], True), ([17, 60, 33, 5], None),
                                              ([17, 60, 33, 5], "mixed"),
                                              ([40, 40], "no_weights")])
def test_step_matches_oracle(pkg, lengths, keep_all):
    """Loss and LoRA gradients of one GPU step equal the CPU oracle's (fp32 autograd with the
    same NF4 bytes and dropout masks) within the reference's whole-step tolerance; the CUDA
    generator advances exactly as the base's 2 x layers dropout calls would. keep_all: every
    layer recomputes (False), keeps (True; with its dequantized weights), the memory-cap plan
    (None: all keep), a cap that admits exactly one kept layer ("mixed": layer 0 recomputes,
    layer 1 keeps), or every layer keeps its intermediates but dequantizes again in its
    backward ("no_weights")."""
    model = _tiny(pkg)
    if keep_all == "mixed":
        model.keep_all = None
        n = sum(lengths)
        weights = model.weight_bytes_per_layer()
        work = weights + 64 * 2**20 + n * 96 * 1024 + n * model.cfg.vocab_size * 2
        # the plan's baseline pinned: torch's allocated bytes move when Python frees earlier
        # tests' tensors, which would shift the cap between here and the step
        base = torch.cuda.memory_allocated()
        model.allocated_bytes = lambda: base
        rec = model.recompute_bytes_per_layer(n)
        model.set_memory_cap(base + work + 2 * rec +
                             int(1.5 * (model.kept_bytes_per_layer(n) + weights - rec)))
        assert model.keep_plan(n) == 1
    elif keep_all == "no_weights":
        model.keep_all = True
        model.keep_weights = False
    else:
        model.keep_all = keep_all
        if keep_all is None:
            assert model.keep_plan(sum(lengths)) == len(model.layers)
    cpu = OS.CpuQwen2(model)
    ids, mask, labels = _batch(lengths, model.cfg.vocab_size)
    denom = float((labels[:, 1:] != -100).sum())
    torch.cuda.manual_seed(1234)
    gen = model.dropout.gen
    seed, offset = gen.initial_seed(), gen.get_offset()
    loss, packed, stats = model.step(ids.to(DEV), mask.to(DEV), labels.to(DEV), denom)
    loss.backward()
    torch.cuda.synchronize()
    ref, _ = OS.forward_loss(cpu, ids, mask, labels, denom, drop_seed=seed, drop_offset=offset,
                             drop_G=model.dropout.max_blocks * 256, p=model.dropout_p, vec=4)
    ref.backward()
    assert abs(loss.item() - ref.item()) <= 2e-3 * abs(ref.item())
    # the generator moved as the base's dropout calls would (engine.py:796-805)
    B, T = ids.shape
    want = offset
    for _ in range(2 * len(model.layers)):
        _, _, inc = OS.philox.draw(B * T * model.cfg.hidden_size, want, model.dropout.max_blocks)
        want += inc
    assert gen.get_offset() == want
    for g_gpu, leaf in zip(model.parameters(), cpu.lora_leaves()):
        ga, gb = g_gpu.grad.detach().cpu().double(), leaf.grad.double()
        rel = (ga - gb).norm() / gb.norm().clamp_min(1e-30)
        assert rel < 2e-2, rel.item()
    # per-token metrics: loss of supervised tokens, entropy finite, order supervised-first
    assert torch.isfinite(stats.entropy).all()
    assert int(packed.n_supervised) == int((packed.targets >= 0).sum())


def test_unsupported_batch_is_rejected_before_any_change(pkg):
    """Left padding raises UnsupportedBatch before the generator or anything else moves
    (engine.py:700-717)."""
    model = _tiny(pkg, layers=1)
    ids, mask, labels = _batch([5, 9], model.cfg.vocab_size)
    mask = mask.flip(1)
    before = model.dropout.gen.get_offset()
    with pytest.raises(pkg.engine.UnsupportedBatch):
        model.step(ids.to(DEV), mask.to(DEV), labels.to(DEV), 1.0)
    assert model.dropout.gen.get_offset() == before


def test_host_metadata_gives_the_same_step(pkg):
    """A step given the row lengths and the supervised count on the host (no device reads)
    equals the step that reads them back: same loss, same LoRA gradients, same packing."""
    lengths = [17, 60, 33, 5]
    ids, mask, labels = _batch(lengths, 3000)
    denom = float((labels[:, 1:] != -100).sum())
    out = []
    for meta in ({}, {"lengths": lengths, "n_supervised": int(denom)}):
        model = _tiny(pkg)
        torch.cuda.manual_seed(99)
        loss, packed, _ = model.step(ids.to(DEV), mask.to(DEV), labels.to(DEV), denom, **meta)
        loss.backward()
        torch.cuda.synchronize()
        out.append((loss.item(), [p.grad.clone() for p in model.parameters()],
                    packed.tok.cpu(), packed.cu_seqlens.cpu(), packed.n_supervised))
    (l0, g0, t0, c0, n0), (l1, g1, t1, c1, n1) = out
    assert l0 == l1 and n0 == n1 == int(denom)
    assert torch.equal(t0, t1) and torch.equal(c0, c1)
    for a, b in zip(g0, g1):
        assert torch.equal(a, b)


def _peft_tree(model):
    """A stand-in for a PEFT-wrapped bitsandbytes 4-bit Qwen2ForCausalLM over the same weights:
    the attribute paths engine.from_peft reads (engine.py:875-906, 1571-1600)."""
    from types import SimpleNamespace as NS
    cfg = model.cfg
    layers = []
    for spec in model.layers:
        D = spec.D
        nq, nk = spec.HQ * D, spec.HKV * D
        b = spec.bias_qkv
        biases = {"q_proj": b[:nq], "k_proj": b[nq:nq + nk], "v_proj": b[nq + nk:]}

        def proj(name, short=None):
            base = NS(weight=spec.w[name].param, bias=biases.get(name))
            m = NS(base_layer=base)
            if short is not None:
                A, B, s = spec.lora[short]
                m.lora_A = {"default": NS(weight=A)}
                m.lora_B = {"default": NS(weight=B)}
                m.scaling = {"default": s}
                m.lora_dropout = {"default": NS(p=cfg.lora_dropout)}
                m.active_adapter = ["default"]
            return m

        attn = NS(q_proj=proj("q_proj", "q"), k_proj=proj("k_proj"), v_proj=proj("v_proj", "v"),
                  o_proj=proj("o_proj"))
        mlp = NS(gate_proj=proj("gate_proj"), up_proj=proj("up_proj"),
                 down_proj=proj("down_proj"))
        layers.append(NS(self_attn=attn, mlp=mlp,
                         input_layernorm=NS(weight=spec.ln1, variance_epsilon=spec.eps),
                         post_attention_layernorm=NS(weight=spec.ln2,
                                                     variance_epsilon=spec.eps)))
    embed = NS(weight=model.embed)
    inner = NS(layers=layers, embed_tokens=embed,
               norm=NS(weight=model.norm_w, variance_epsilon=model.eps))
    config = NS(hidden_size=cfg.hidden_size, intermediate_size=cfg.intermediate_size,
                num_attention_heads=cfg.num_attention_heads,
                num_key_value_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                vocab_size=cfg.vocab_size, rope_theta=cfg.rope_theta)
    causal = NS(model=inner, lm_head=NS(weight=model.embed), config=config)
    return NS(get_base_model=lambda: causal)


def test_from_peft_and_trainer_drop_in(pkg):
    """engine.from_peft over a PEFT-shaped module tree of the same weights gives the same step
    (loss and LoRA gradients bit for bit), and trainer.install + compute_loss runs it."""
    import types
    model = _tiny(pkg)
    twin = pkg.engine.from_peft(_peft_tree(model))
    assert twin.dropout_p == model.dropout_p and len(twin.layers) == len(model.layers)
    lengths = [17, 60, 33, 5]
    ids, mask, labels = _batch(lengths, 3000)
    denom = float((labels[:, 1:] != -100).sum())
    out = []
    for m in (model, twin):
        for p in m.parameters():
            p.grad = None
        torch.cuda.manual_seed(5)
        loss, _, _ = m.step(ids.to(DEV), mask.to(DEV), labels.to(DEV), denom)
        loss.backward()
        torch.cuda.synchronize()
        out.append((loss.item(), [p.grad.clone() for p in m.parameters()]))
    assert out[0][0] == out[1][0]
    for a, b in zip(out[0][1], out[1][1]):
        assert torch.equal(a, b)

    class Tr:
        compute_loss_func = label_smoother = None
        model_accepts_loss_kwargs = False
        args = types.SimpleNamespace(average_tokens_across_devices=False, n_gpu=1)

        def __init__(self):
            self._metrics = {"train": {"entropy": [], "mean_token_accuracy": []}}
            self.cbs = []

        def compute_loss(self, model, inputs, return_outputs=False, num_items_in_batch=None):
            raise AssertionError("the fused step should run")

        def add_callback(self, cb):
            self.cbs.append(cb)

    tr = Tr()
    assert pkg.trainer.install(tr, engine=twin)
    torch.cuda.manual_seed(5)
    batch = {"input_ids": ids.to(DEV), "attention_mask": mask.to(DEV), "labels": labels.to(DEV)}
    loss = tr.compute_loss(types.SimpleNamespace(training=True), batch)
    assert loss.item() == out[0][0]
    tr.cbs[0].on_pre_optimizer_step(None, None, None)
    assert len(tr._metrics["train"]["entropy"]) == 1
    assert tr._metrics["train"]["num_tokens"] == [sum(lengths)]
    assert 0.0 <= tr._metrics["train"]["mean_token_accuracy"][0] <= 1.0
