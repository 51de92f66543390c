"""The GPU step against transformers' own Qwen2ForCausalLM: the reference's whole-step test
(test_kernels.py:314-400: a tiny Qwen2 with vocabulary 3,000, H 256, I 640, 2 layers, 4/2 heads,
packed lengths [17, 60, 33, 5], [4] and [40, 40], against HF + PEFT over the same NF4 weights),
with the library model in fp32 on the CPU over the step's own dequantized weights (oracle.nf4,
bit-exact to the GPU's dequant) and rank-16 LoRA on q and v added as s B (A x) (PEFT's LoRA;
dropout 0, so no masks to share). The vocabulary is 3,072 here: the package GEMM tiles in
multiples of 128. Bar: the reference's, loss relative 2e-3 and LoRA gradient relative norm
2e-2."""

import pytest
import torch

from oracle import step as OS

transformers = pytest.importorskip("transformers")

pytestmark = pytest.mark.gpu

DEV = "cuda"


class _Lora(torch.nn.Module):
    def __init__(self, base, a, b, s):
        super().__init__()
        self.base, self.s = base, s
        self.a, self.b = torch.nn.Parameter(a.clone()), torch.nn.Parameter(b.clone())

    def forward(self, x):
        return self.base(x) + self.s * ((x @ self.a.t()) @ self.b.t())


def _hf_model(cfg, cpu):
    H, I, HQ, HKV, D = (cfg.hidden_size, cfg.intermediate_size, cfg.num_attention_heads,
                        cfg.num_key_value_heads, cfg.head_dim)
    hcfg = transformers.Qwen2Config(vocab_size=cfg.vocab_size, hidden_size=H,
                                    intermediate_size=I, num_hidden_layers=len(cpu.layers),
                                    num_attention_heads=HQ, num_key_value_heads=HKV,
                                    rope_theta=cfg.rope_theta, rms_norm_eps=cfg.rms_norm_eps,
                                    tie_word_embeddings=True, max_position_embeddings=128)
    assert H // HQ == D
    hf = transformers.Qwen2ForCausalLM._from_config(hcfg, attn_implementation="eager",
                                                    dtype=torch.float32)
    nq, nk = HQ * D, HKV * D
    with torch.no_grad():
        hf.model.embed_tokens.weight.copy_(cpu.embed)
        hf.model.norm.weight.copy_(cpu.norm_w)
        for layer, lay in zip(hf.model.layers, cpu.layers):
            at, mlp = layer.self_attn, layer.mlp
            for proj, rows in ((at.q_proj, slice(0, nq)), (at.k_proj, slice(nq, nq + nk)),
                               (at.v_proj, slice(nq + nk, nq + 2 * nk))):
                proj.weight.copy_(lay.w_qkv[rows])
                proj.bias.copy_(lay.bias[rows])
            at.o_proj.weight.copy_(lay.w_o)
            mlp.gate_proj.weight.copy_(lay.w_gu[:I])
            mlp.up_proj.weight.copy_(lay.w_gu[I:])
            mlp.down_proj.weight.copy_(lay.w_d)
            layer.input_layernorm.weight.copy_(lay.ln1)
            layer.post_attention_layernorm.weight.copy_(lay.ln2)
            for k, name in (("q", "q_proj"), ("v", "v_proj")):
                a, b, s = lay.lora[k]
                setattr(at, name, _Lora(getattr(at, name), a.detach(), b.detach(), s))
    return hf


def _rel(a, b):
    a, b = a.detach().cpu().double(), b.detach().cpu().double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


@pytest.mark.parametrize("lengths", [[17, 60, 33, 5], [4], [40, 40]])
def test_step_matches_transformers_qwen2(pkg, lengths):
    E = pkg.engine
    print(f"step vs transformers Qwen2, lengths {lengths}", flush=True)
    cfg = E.Qwen2Config(hidden_size=256, intermediate_size=640, num_hidden_layers=2,
                        num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                        vocab_size=3072, lora_dropout=0.0)
    model = E.random_qwen2(cfg, DEV, seed=9)
    model.keep_all = False  # per-layer recompute
    g = torch.Generator().manual_seed(len(lengths))
    B, T = len(lengths), max(lengths)
    ids = torch.randint(0, cfg.vocab_size, (B, T), generator=g)
    mask = (torch.arange(T)[None] < torch.tensor(lengths)[:, None]).long()
    labels = torch.where(mask.bool(), ids, torch.full_like(ids, -100))
    denom = float((labels[:, 1:] != -100).sum())
    loss, _, _ = model.step(ids.to(DEV), mask.to(DEV), labels.to(DEV), denom, lengths=lengths,
                            n_supervised=int(denom))
    scale = 2.0**16  # as the trainer's loss scaling: fp16 gradients stay out of subnormals
    (loss * scale).backward()
    torch.cuda.synchronize()

    hf = _hf_model(cfg, OS.CpuQwen2(model))
    hf.eval()
    out = hf(input_ids=ids, attention_mask=mask, labels=labels)
    out.loss.backward()
    want = [p.grad for layer in hf.model.layers for name in ("q_proj", "v_proj")
            for p in (getattr(layer.self_attn, name).a, getattr(layer.self_attn, name).b)]
    lg, lw = float(loss.detach()), float(out.loss.detach())
    print(f"gpu loss {lg:.6f}, transformers {lw:.6f}", flush=True)
    assert abs(lg - lw) <= 2e-3 * abs(lw)
    got = [p.grad / scale for p in model.parameters()]
    assert len(got) == len(want) == 8
    for i, (a, b) in enumerate(zip(got, want)):
        r = _rel(a, b)
        assert r < 2e-2, (i, r)
