"""One Qwen2 NF4 + LoRA training step on the CPU: the reference's forward math with its fp16
rounding points, differentiated by torch autograd.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Forward (engine.py:1054-1181 per layer, 1359-1395 head; rounding points engine.py:27-31):
  a, aq, av = fp16(RMSNorm(h)), fp16(drop_q(RMSNorm(h))), fp16(drop_v(...))
  qkv = fp16(a W_qkv^T + bias);  lq = fp16(fp16(aq A_q^T) B_q^T);  lv likewise
  q, k = fp16(rope(qkv_q + s lq)), fp16(rope(qkv_k));  v = fp16(qkv_v + s lv)
  out = fp16(causal attention per sequence);  o = fp16(out W_o^T)
  h2 = h + o;  b = fp16(RMSNorm(h2));  gu = fp16(b W_gu^T);  m = fp16(silu(g) u)
  h3 = h2 + fp16(m W_d^T)
  head: hn = fp16(RMSNorm(h)); logits = fp16(hn E^T); loss = sum CE(logits) / denom
The NF4 weights are dequantised from the same bytes by oracle.nf4 (bit-exact), the dropout masks
come from oracle.philox with the generator state the GPU step starts from. Gradients are
autograd's through fp32 (the fp16 roundings are straight-through), an independent formulation
of the GPU step's hand-written backward (which rounds gradients to fp16 at GEMM inputs); the
parity bar is the reference's whole-step tolerance (test_kernels.py:314-400: loss relative
2e-3, LoRA gradient relative norm 2e-2).
"""

import numpy as np
import torch

from . import nf4 as ON
from . import philox


def _r16(x):
    """fp16 rounding, straight-through for autograd."""
    return x + (x.detach().half().float() - x.detach())


def dequant_param(param):
    """fp16 -> fp32 torch [N, K] of a Params4bit-like (GPU tensors), via oracle.nf4."""
    qs = param.quant_state
    if qs.nested:
        st = ON.QuantState(qs.absmax.cpu().numpy(), tuple(qs.shape), qs.code.cpu().numpy(),
                           qs.blocksize, offset=np.float32(float(qs.offset)),
                           state2=ON.QuantState2(qs.state2.absmax.cpu().numpy(),
                                                 qs.state2.code.cpu().numpy(),
                                                 qs.state2.blocksize))
    else:
        st = ON.QuantState(qs.absmax.cpu().numpy(), tuple(qs.shape), qs.code.cpu().numpy(),
                           qs.blocksize)
    out = ON.dequantize_nf4(param.data.cpu().numpy().reshape(-1), st,
                            levels=qs.code.cpu().numpy())
    return torch.from_numpy(out.astype(np.float32))


class CpuLayer:
    pass


class CpuQwen2:
    """CPU copy of a FusedQwen2: dequantised fp16-valued weights (as fp32), fp32 LoRA leaves."""

    def __init__(self, model, layers=None):
        cfg = model.cfg
        self.cfg = cfg
        self.layers = []
        for spec in (model.layers if layers is None else [model.layers[i] for i in layers]):
            lay = CpuLayer()
            w = {name: dequant_param(nw.param) for name, nw in spec.w.items()}
            lay.w_qkv = torch.cat([w["q_proj"], w["k_proj"], w["v_proj"]])
            lay.w_o, lay.w_d = w["o_proj"], w["down_proj"]
            lay.w_gu = torch.cat([w["gate_proj"], w["up_proj"]])
            lay.bias = spec.bias_qkv.float().cpu()
            lay.ln1, lay.ln2 = spec.ln1.float().cpu(), spec.ln2.float().cpu()
            lay.lora = {k: (a.detach().cpu().clone().requires_grad_(),
                            b.detach().cpu().clone().requires_grad_(), s)
                        for k, (a, b, s) in spec.lora.items()}
            self.layers.append(lay)
        self.embed = model.embed.float().cpu()
        self.norm_w = model.norm_w.float().cpu()

    def lora_leaves(self):
        return [t for lay in self.layers for k in ("q", "v") for t in lay.lora[k][:2]]


def _rms(x, w, eps):
    rstd = 1.0 / torch.sqrt((x * x).sum(-1, keepdim=True) / x.shape[-1] + eps)
    return w * (x * rstd)


def _rope(x, cos, sin):
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], -1)


def rope_cos_sin(pos, D, theta):
    """cos, sin [n, 1, D/2] fp32 of angle = pos * theta^(-2k/D) (test_kernels.py:154-156)."""
    inv = 1.0 / (theta ** (torch.arange(0, D, 2).float() / D))
    ang = pos.float()[:, None] * inv[None, :]
    return ang.cos()[:, None, :], ang.sin()[:, None, :]


def attn_input(lay, h, masks, kscale, cos, sin, HQ, HKV, D, eps):
    """The attention-input block (engine.py:1073-1109) with autograd: input RMSNorm, the
    dropout'ed LoRA inputs (masks = (keep_q, keep_v) bool [n, H], or None without dropout),
    qkv = fp16(a W_qkv^T + bias), lq = fp16(fp16(aq A_q^T) B_q^T), lv likewise, then
    q = fp16(rope(qkv_q + s lq)), k = fp16(rope(qkv_k)), v = fp16(qkv_v + s lv) with k, v in
    grouped layout [n, HKV, D]."""
    n = h.shape[0]
    (aq_w, bq_w, s), (av_w, bv_w, _) = lay.lora["q"], lay.lora["v"]
    y = _rms(h, lay.ln1, eps)
    a = _r16(y)
    if masks is not None:
        mq, mv = masks
        aq = _r16(torch.where(mq, y * kscale, torch.zeros_like(y)))
        av = _r16(torch.where(mv, y * kscale, torch.zeros_like(y)))
    else:
        aq = av = a
    qkv = _r16(a @ lay.w_qkv.t() + lay.bias)
    lq = _r16(_r16(aq @ _r16(aq_w).t()) @ _r16(bq_w).t())
    lv = _r16(_r16(av @ _r16(av_w).t()) @ _r16(bv_w).t())
    q = (qkv[:, :HQ * D] + s * lq).view(n, HQ, D)
    k = qkv[:, HQ * D:(HQ + HKV) * D].view(n, HKV, D)
    v = (qkv[:, (HQ + HKV) * D:] + s * lv).view(n, HKV, D)
    return _r16(_rope(q, cos, sin)), _r16(_rope(k, cos, sin)), _r16(v)


class Batch:
    """The packing of a right-padded batch (engine.py:705-751), on the CPU."""

    def __init__(self, input_ids, attention_mask, labels):
        B, T = input_ids.shape
        lengths = attention_mask.sum(1)
        mask = torch.arange(T)[None, :] < lengths[:, None]
        flat = mask.reshape(-1).nonzero().squeeze(1)
        self.B, self.T, self.n = B, T, int(flat.numel())
        self.tok = flat
        self.ids = input_ids.reshape(-1)[flat]
        self.pos = flat % T
        shifted = torch.full_like(labels, -100)
        shifted[:, :-1] = labels[:, 1:]
        self.targets = shifted.reshape(-1)[flat]
        self.lengths = [int(x) for x in lengths]


def forward_loss(model, input_ids, attention_mask, labels, denom, *, drop_seed=0,
                 drop_offset=0, drop_G=1, p=0.0, vec=4, first_layer_input=None):
    """Loss of the step (autograd graph to the LoRA leaves). Dropout calls are drawn in PEFT's
    order (layer i q, layer i v) from a generator at (drop_seed, drop_offset) with drop_G threads
    (oracle.philox.draw). With first_layer_input, the layers start from that fp32 [n, H]
    residual instead of the embedding (a bounded sample of the step's layers)."""
    cfg = model.cfg
    bt = Batch(input_ids.cpu(), attention_mask.cpu(), labels.cpu())
    n, H, D = bt.n, cfg.hidden_size, cfg.head_dim
    HQ, HKV, eps = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.rms_norm_eps
    cos, sin = rope_cos_sin(bt.pos, D, cfg.rope_theta)
    p_keep, kscale = np.float32(1 - p), float(np.float32(1.0 / (1 - p))) if p > 0 else 1.0
    offset = drop_offset
    nelem = bt.B * bt.T * H
    elems = (bt.tok[:, None] * H + torch.arange(H)[None, :]).reshape(-1).numpy()

    def next_mask():
        nonlocal offset
        ctr, G, inc = philox.draw(nelem, offset, drop_G // philox.BLOCK)
        offset += inc
        keep = philox.keep_mask(elems, drop_seed, ctr, G, p_keep, vec)
        return torch.from_numpy(keep).view(n, H)

    if first_layer_input is None:
        h = model.embed[bt.ids]
    else:
        h = first_layer_input
    for lay in model.layers:
        masks = (next_mask(), next_mask()) if p > 0 else None
        q, k, v = attn_input(lay, h, masks, kscale, cos, sin, HQ, HKV, D, eps)
        rep = HQ // HKV
        k = k.repeat_interleave(rep, 1)
        v = v.repeat_interleave(rep, 1)
        outs, start = [], 0
        for length in bt.lengths:
            sl = slice(start, start + length)
            o = torch.nn.functional.scaled_dot_product_attention(
                q[sl].transpose(0, 1), k[sl].transpose(0, 1), v[sl].transpose(0, 1),
                is_causal=True, scale=D ** -0.5)
            outs.append(o.transpose(0, 1))
            start += length
        out = _r16(torch.cat(outs).reshape(n, HQ * D))
        h2 = h + _r16(out @ lay.w_o.t())
        b = _r16(_rms(h2, lay.ln2, eps))
        gu = _r16(b @ lay.w_gu.t())
        I = gu.shape[1] // 2
        g, u = gu[:, :I], gu[:, I:]
        m = _r16(torch.nn.functional.silu(g) * u)
        h = h2 + _r16(m @ lay.w_d.t())
    hn = _r16(_rms(h, model.norm_w, eps))
    logits = _r16(hn @ model.embed.t())
    tok = torch.nn.functional.cross_entropy(logits, bt.targets.clamp(min=0), reduction="none")
    tok = torch.where(bt.targets >= 0, tok, torch.zeros_like(tok))
    return tok.sum() / denom, h
