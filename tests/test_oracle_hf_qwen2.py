"""The oracle's whole-model step (oracle.step.forward_loss) against an independent
implementation of the same architecture: transformers' own Qwen2ForCausalLM (fp32, eager
attention) on a tiny random model with the same weights and rank-4 LoRA adapters on q_proj and
v_proj, added as y = W x + b + s B (A x) (PEFT's LoRA without dropout). This pins what the
oracle's formulas alone cannot: the layer order, the grouped-query head mapping, RoPE's
half-rotation and its sign, the tied head, the shifted labels and the loss normalisation (a RoPE
position offset shared by a sequence's tokens cancels in its scores, so no loss can show one).
Planted in a copy of the oracle on the CPU, a flipped RoPE sine, the k/v heads tiled instead of
repeated per group, or a wrong norm epsilon move the gradients by 0.7-1.5 relative; the clean
oracle is within 1.2e-5 (loss) and 1.6e-3 (gradients) of the library model. The bar is the
reference's own whole-step test against HF + PEFT (test_kernels.py:314-400): loss relative
2e-3, LoRA gradient relative norm 2e-2; the oracle rounds at the reference's fp16 points, the
library model does not."""

import pytest
import torch

transformers = pytest.importorskip("transformers")

from oracle import step as OS  # noqa: E402

H, I, V, HQ, HKV, R, S = 64, 160, 300, 4, 2, 4, 2.0
D = H // HQ


class _Cfg:
    hidden_size, head_dim, num_attention_heads, num_key_value_heads = H, D, HQ, HKV
    rms_norm_eps, rope_theta = 1e-6, 1e6


class _Lora(torch.nn.Module):
    def __init__(self, base, a, b, s):
        super().__init__()
        self.base, self.s = base, s
        self.a, self.b = torch.nn.Parameter(a.clone()), torch.nn.Parameter(b.clone())

    def forward(self, x):
        return self.base(x) + self.s * ((x @ self.a.t()) @ self.b.t())


def _models(seed):
    cfg = transformers.Qwen2Config(vocab_size=V, hidden_size=H, intermediate_size=I,
                                   num_hidden_layers=2, num_attention_heads=HQ,
                                   num_key_value_heads=HKV, rope_theta=1e6, rms_norm_eps=1e-6,
                                   tie_word_embeddings=True, max_position_embeddings=64)
    torch.manual_seed(seed)
    hf = transformers.Qwen2ForCausalLM._from_config(cfg, attn_implementation="eager",
                                                    dtype=torch.float32)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():  # fp16-exact values (the oracle rounds its GEMM inputs to fp16)
        for name, p in hf.named_parameters():
            if name.endswith("norm.weight") or "layernorm" in name:
                p.copy_(1 + 0.02 * torch.randn(p.shape, generator=g))
            elif name.endswith("bias"):
                p.copy_(0.02 * torch.randn(p.shape, generator=g))
            else:
                p.copy_(0.05 * torch.randn(p.shape, generator=g))
            p.copy_(p.half().float())
    om = type("M", (), {})()
    om.cfg, om.layers = _Cfg(), []
    for layer in hf.model.layers:
        at, mlp = layer.self_attn, layer.mlp
        lay = OS.CpuLayer()
        lay.w_qkv = torch.cat([at.q_proj.weight, at.k_proj.weight, at.v_proj.weight]).detach()
        lay.bias = torch.cat([at.q_proj.bias, at.k_proj.bias, at.v_proj.bias]).detach()
        lay.w_o = at.o_proj.weight.detach()
        lay.w_gu = torch.cat([mlp.gate_proj.weight, mlp.up_proj.weight]).detach()
        lay.w_d = mlp.down_proj.weight.detach()
        lay.ln1 = layer.input_layernorm.weight.detach()
        lay.ln2 = layer.post_attention_layernorm.weight.detach()
        lay.lora = {}
        for k, proj, n_out in (("q", "q_proj", HQ * D), ("v", "v_proj", HKV * D)):
            a = ((torch.rand(R, H, generator=g) * 2 - 1) / H ** 0.5).half().float()
            b = (0.1 * torch.randn(n_out, R, generator=g)).half().float()
            setattr(at, proj, _Lora(getattr(at, proj), a, b, S))
            lay.lora[k] = (a.clone().requires_grad_(), b.clone().requires_grad_(), S)
        om.layers.append(lay)
    om.embed = hf.model.embed_tokens.weight.detach()
    om.norm_w = hf.model.norm.weight.detach()
    return hf, om


@pytest.mark.parametrize("lengths,prompt", [([12, 7, 9], 2), ([5], 0), ([16, 16], 5)])
def test_oracle_step_matches_transformers_qwen2(lengths, prompt):
    hf, om = _models(len(lengths) + prompt)
    B, T = len(lengths), max(lengths)
    g = torch.Generator().manual_seed(7)
    ids = torch.randint(0, V, (B, T), generator=g)
    mask = (torch.arange(T)[None, :] < torch.tensor(lengths)[:, None]).long()
    labels = torch.where(mask.bool(), ids, torch.full_like(ids, -100))
    labels[:, :prompt] = -100
    denom = float((labels[:, 1:] != -100).sum())

    hf.eval()
    out = hf(input_ids=ids, attention_mask=mask, labels=labels)
    out.loss.backward()
    want = [p.grad for layer in hf.model.layers for proj in ("q_proj", "v_proj")
            for p in (getattr(layer.self_attn, proj).a, getattr(layer.self_attn, proj).b)]

    loss, _ = OS.forward_loss(om, ids, mask, labels, denom)
    loss.backward()
    got = [t.grad for lay in om.layers for k in ("q", "v") for t in lay.lora[k][:2]]

    lo, lw = float(loss.detach()), float(out.loss.detach())
    assert abs(lo - lw) <= 2e-3 * abs(lw)
    assert len(got) == len(want) == 8
    for a, b in zip(got, want):
        assert float((a - b).norm() / b.norm()) < 2e-2
