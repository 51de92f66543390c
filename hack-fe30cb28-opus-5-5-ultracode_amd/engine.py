"""One Qwen2 + NF4 + LoRA training step around the gfx950 kernels (the counterpart of the
reference's solution/engine.py, FusedQwen2 and its layer/head autograd functions).

The math and rounding points are the reference's (engine.py:27-31, 1054-1400): fp32 residual
stream, norms, RoPE, softmax and loss; fp16 at the projection outputs, the attention inputs and
the MLP product. Pad tokens are dropped (Packed, varlen attention over cu_seqlens); every decoder
layer is one autograd.Function that recomputes its forward in backward from its fp32 input
(per-layer recompute), or keeps its intermediates (`keep=True`: with 288 GB of HBM the whole
step's activations fit); the head runs final norm + lm_head + cross-entropy + dh in chunks of rows
with the logits gradient formed in place. The LoRA-dropout masks are the ones PyTorch's
nn.Dropout would draw, in PEFT's call order (layer 0 q, layer 0 v, layer 1 q, ...), computed by
the kernels from the generator state, in backward again.

Everything stays resident in HBM: the reference's host-offload machinery (WeightStream,
InputStream, GuStream, AttnStream, HostHead, memory-cap planning) has no counterpart here.
"""

import itertools
import math

import torch

from . import linear as L
from .ops import (NF4Group, NF4Weight, TorchDropout, _attn_bwd, _attn_fwd, _ce, _glu_bwd,
                  _glu_fwd, _lora_bwd_rows, _lora_fwd_rows, _lora_grad, _rms_bwd, _rms_fwd,
                  _rope_bwd, _rope_fwd, _as_int64, keep_bits_shape)
from .quant import quantize_nf4


class UnsupportedBatch(ValueError):
    """The step does not take this batch; raised before anything changes (engine.py:700-702)."""


# ---------------------------------------------------------------------------------------------
# Model description
# ---------------------------------------------------------------------------------------------
class Qwen2Config:
    """Qwen2.5-1.5B by default (hidden 1536, intermediate 8960, 28 layers, 12/2 heads)."""

    def __init__(self, hidden_size=1536, intermediate_size=8960, num_hidden_layers=28,
                 num_attention_heads=12, num_key_value_heads=2, head_dim=128,
                 vocab_size=151936, rope_theta=1e6, rms_norm_eps=1e-6, lora_r=16,
                 lora_alpha=32, lora_dropout=0.05):
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.num_hidden_layers = num_hidden_layers
        self.num_attention_heads = num_attention_heads
        self.num_key_value_heads = num_key_value_heads
        self.head_dim = head_dim
        self.vocab_size = vocab_size
        self.rope_theta = rope_theta
        self.rms_norm_eps = rms_norm_eps
        self.lora_r = lora_r
        self.lora_alpha = lora_alpha
        self.lora_dropout = lora_dropout


class LayerSpec:
    """One decoder layer's frozen weights and LoRA parameters (engine.py:875-921)."""

    def __init__(self, index, cfg, ln1, ln2, nf4, bias_qkv, lora):
        self.index = index
        self.H = cfg.hidden_size
        self.D = cfg.head_dim
        self.HQ = cfg.num_attention_heads
        self.HKV = cfg.num_key_value_heads
        self.I = cfg.intermediate_size
        self.eps = cfg.rms_norm_eps
        self.ln1, self.ln2 = ln1, ln2
        self.scale = self.D ** -0.5
        self.w = {name: NF4Weight(p) for name, p in nf4.items()}
        self.qkv = NF4Group.of([self.w["q_proj"], self.w["k_proj"], self.w["v_proj"]])
        self.gu = NF4Group.of([self.w["gate_proj"], self.w["up_proj"]])
        self.nf4_all = [self.qkv, self.w["o_proj"], self.gu, self.w["down_proj"]]
        self.nf4_nogu = [self.qkv, self.w["o_proj"], self.w["down_proj"]]
        self.bias_qkv = bias_qkv
        self.lora = lora  # {"q": (A, B, scaling), "v": (A, B, scaling)}

    def lora_params(self):
        out = []
        for short in ("q", "v"):
            a, b, _ = self.lora[short]
            out += [a, b]
        return out


def _lora_scale(spec):
    scales = {v[2] for v in spec.lora.values()}
    assert len(scales) <= 1
    return scales.pop() if scales else 1.0


@torch.no_grad()
def random_qwen2(cfg, device, seed=0, norm_dtype=torch.float32):
    """A random-init Qwen2 with NF4 (double-quant, blocksize 64) frozen linears, fp16 tied
    embedding, fp32 RMSNorm weights ~ 1 + N(0, 0.02), fp16 qkv bias ~ N(0, 0.02), LoRA r/alpha on
    q and v (A kaiming-uniform fp32, B ~ N(0, 0.01) fp32). Weights ~ N(0, 0.02)."""
    g = torch.Generator(device=device).manual_seed(seed)
    H, I, D = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
    HQ, HKV, r = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.lora_r
    shapes = {"q_proj": (HQ * D, H), "k_proj": (HKV * D, H), "v_proj": (HKV * D, H),
              "o_proj": (H, HQ * D), "gate_proj": (I, H), "up_proj": (I, H),
              "down_proj": (H, I)}

    def randn(*shape, std=1.0, dtype=torch.float32):
        return (torch.randn(shape, generator=g, device=device) * std).to(dtype)

    layers = []
    bound = 1.0 / math.sqrt(H)  # kaiming_uniform_(a=sqrt(5)) on a [r, H] matrix
    scaling = cfg.lora_alpha / r
    for i in range(cfg.num_hidden_layers):
        nf4 = {name: quantize_nf4(randn(*shape, std=0.02, dtype=torch.float16))
               for name, shape in shapes.items()}
        ln1 = (1.0 + randn(H, std=0.02)).to(norm_dtype)
        ln2 = (1.0 + randn(H, std=0.02)).to(norm_dtype)
        bias = randn((HQ + 2 * HKV) * D, std=0.02, dtype=torch.float16)
        lora = {}
        for short, out_dim in (("q", HQ * D), ("v", HKV * D)):
            a = ((torch.rand((r, H), generator=g, device=device) * 2 - 1) * bound)
            b = randn(out_dim, r, std=0.01)
            lora[short] = (a.requires_grad_(), b.requires_grad_(), scaling)
        layers.append(LayerSpec(i, cfg, ln1, ln2, nf4, bias, lora))
    embed = randn(cfg.vocab_size, H, std=0.02, dtype=torch.float16)
    norm_w = (1.0 + randn(H, std=0.02)).to(norm_dtype)
    return FusedQwen2(cfg, layers, embed, norm_w, device)


SUPPORTED_RANKS = (8, 16, 32, 64)  # LoRA ranks of the HIP kernels


class UnsupportedModel(ValueError):
    """The model is not a PEFT-wrapped 4-bit Qwen2 the step supports (patch.py:_is_supported)."""


def _lora_targets(layer):
    """The adapter name of each LoRA-wrapped projection of a decoder layer, {"q": name, ...}."""
    out = {}
    projs = {"q": layer.self_attn.q_proj, "k": layer.self_attn.k_proj,
             "v": layer.self_attn.v_proj, "o": layer.self_attn.o_proj,
             "gate": layer.mlp.gate_proj, "up": layer.mlp.up_proj,
             "down": layer.mlp.down_proj}
    for short, module in projs.items():
        lora_a = getattr(module, "lora_A", None)
        if lora_a is None or len(lora_a) == 0:
            continue
        active = getattr(module, "active_adapter", None)
        if isinstance(active, (list, tuple)):
            active = active[0] if active else None
        out[short] = active if active in lora_a else next(iter(lora_a.keys()))
    return out


@torch.no_grad()
def from_peft(peft_model, keep_all=False):
    """The step over a PEFT-wrapped, bitsandbytes-4bit Qwen2ForCausalLM (engine.py:1571-1600,
    875-921): the NF4 weights and norms are borrowed (Params4bit `.data` / `.quant_state`), the
    LoRA A/B parameters are the PEFT modules' own (the optimizer's), the embedding is the tied
    lm_head. Supported: LoRA on q and v only, one dropout probability, one scaling."""
    causal = peft_model.get_base_model() if hasattr(peft_model, "get_base_model") else peft_model
    inner = causal.model
    hf = causal.config
    layers_hf = list(inner.layers)
    if not layers_hf:
        raise UnsupportedModel("no decoder layers")
    names = _lora_targets(layers_hf[0])
    if set(names) != {"q", "v"}:
        raise UnsupportedModel(f"LoRA on {sorted(names)}; the step takes LoRA on q and v only")
    H, HQ = hf.hidden_size, hf.num_attention_heads
    D = getattr(hf, "head_dim", None) or H // HQ
    rope = getattr(hf, "rope_parameters", None) or {}
    theta = getattr(hf, "rope_theta", None) or rope.get("rope_theta", 10000.0)
    # the rotary tables here are the plain ones, angle = pos * theta^(-2k/D); a scaled variant
    # (linear, dynamic, YaRN, ...) would train with other positions, so it is refused
    scaling = getattr(hf, "rope_scaling", None) or {}
    kinds = {str(d.get(key)) for d in (rope, scaling) for key in ("rope_type", "type")
             if d.get(key) is not None}
    if kinds - {"default"}:
        raise UnsupportedModel(f"rotary embedding type {sorted(kinds)}; the step takes the "
                               "default (unscaled) rotary embedding only")
    q0 = layers_hf[0].self_attn.q_proj
    qname = names["q"]
    r = int(q0.lora_A[qname].weight.shape[0])
    HKV = hf.num_key_value_heads
    if r not in SUPPORTED_RANKS:
        raise UnsupportedModel(f"LoRA rank {r}; the kernels take {SUPPORTED_RANKS}")
    if HQ % HKV or not 1 <= HQ // HKV <= 8 or D not in (64, 128) or H % 32:
        raise UnsupportedModel(f"attention heads {HQ}/{HKV} x {D}, hidden {H}: the kernels "
                               "take up to 8 q heads per kv head, head_dim 64 or 128, hidden "
                               "size a multiple of 32")
    scaling = float(q0.scaling[qname])
    drop = q0.lora_dropout[qname] if hasattr(q0, "lora_dropout") else None
    p = float(getattr(drop, "p", 0.0))
    cfg = Qwen2Config(hidden_size=H, intermediate_size=hf.intermediate_size,
                      num_hidden_layers=len(layers_hf), num_attention_heads=HQ,
                      num_key_value_heads=hf.num_key_value_heads, head_dim=D,
                      vocab_size=hf.vocab_size, rope_theta=float(theta),
                      rms_norm_eps=float(layers_hf[0].input_layernorm.variance_epsilon),
                      lora_r=r, lora_alpha=scaling * r, lora_dropout=p)

    def base_of(module):
        return getattr(module, "base_layer", module)

    specs = []
    for i, layer in enumerate(layers_hf):
        attn, mlp = layer.self_attn, layer.mlp
        projs = {name: getattr(attn, name) for name in ("q_proj", "k_proj", "v_proj", "o_proj")}
        projs.update({name: getattr(mlp, name) for name in ("gate_proj", "up_proj", "down_proj")})
        nf4 = {name: base_of(m).weight for name, m in projs.items()}
        biases = [base_of(projs[n]).bias for n in ("q_proj", "k_proj", "v_proj")]
        if any(b is None for b in biases):
            raise UnsupportedModel("q/k/v projections without bias (not Qwen2)")
        bias = torch.cat([b.detach().to(torch.float16) for b in biases]).contiguous()
        lora = {}
        for short in ("q", "v"):
            module, name = projs[f"{short}_proj"], names[short]
            if float(module.scaling[name]) != scaling:
                raise UnsupportedModel("LoRA scalings differ between adapters")
            lora[short] = (module.lora_A[name].weight, module.lora_B[name].weight, scaling)
        specs.append(LayerSpec(i, cfg, layer.input_layernorm.weight,
                               layer.post_attention_layernorm.weight, nf4, bias, lora))
    embed = inner.embed_tokens.weight
    lm = causal.lm_head.weight
    if lm.data_ptr() != embed.data_ptr():
        raise UnsupportedModel("lm_head is not tied to the embedding")
    if embed.dtype != torch.float16:
        raise UnsupportedModel("the tied embedding must be fp16")
    model = FusedQwen2(cfg, specs, embed.detach(), inner.norm.weight.detach(), embed.device,
                       keep_all=keep_all)
    model.eps = float(inner.norm.variance_epsilon)
    return model


# ---------------------------------------------------------------------------------------------
# Per-step packing (engine.py:705-764)
# ---------------------------------------------------------------------------------------------
class RopeTable:
    """cos / sin [positions, D/2] fp32 of the rotary embedding (rotate-half, Qwen2):
    inv_freq_k = theta^(-2k/D), angle = pos * inv_freq in fp32 (engine.py:831-851)."""

    def __init__(self, theta, head_dim, device):
        self.theta, self.half, self.device = theta, head_dim // 2, device
        self.cos = self.sin = None

    def table(self, length):
        if self.cos is None or self.cos.shape[0] < length:
            size = max(1024, 1 << max(0, (length - 1).bit_length()))
            inv = 1.0 / (self.theta ** (torch.arange(0, 2 * self.half, 2, device=self.device,
                                                     dtype=torch.int64).float()
                                        / (2 * self.half)))
            freqs = torch.arange(size, device=self.device).float()[:, None] * inv[None, :]
            self.cos = freqs.cos().contiguous()
            self.sin = freqs.sin().contiguous()
        return self.cos, self.sin


def _to_device(host, dev):
    """A small host tensor on the device through pinned memory, queued on the current stream
    (the host does not wait)."""
    if dev.type != "cuda":
        return host.to(dev)
    return host.pin_memory().to(dev, non_blocking=True)


def _read_lengths(attention_mask, labels):
    """Row lengths and supervised-token count from the device in one read, and whether the mask
    is right-padded (ones, then zeros)."""
    B, T = attention_mask.shape
    mask = attention_mask.bool()
    lengths = mask.sum(dim=1)
    right = torch.arange(T, device=mask.device)[None, :] < lengths[:, None]
    flags = torch.stack([(mask == right).all(),
                         ((labels[:, 1:] >= 0) & mask[:, :-1]).sum()]).to(torch.int64)
    host = torch.cat([lengths.to(torch.int64), flags]).tolist()
    if not host[B]:
        raise UnsupportedBatch("attention_mask is not right-padded")
    return host[:B], host[B + 1]


def _pack_index(lengths, T):
    """int64 host vector [4n + B + 1] of a packing with these row lengths in [B, T]: each
    token's flat index in the batch, the flat index of its next-token label (B*T, a -100
    sentinel, for a token in a row's last column), its position in its sequence, and
    cu_seqlens."""
    B = len(lengths)
    starts = torch.arange(B, dtype=torch.int64) * T
    tok = torch.cat([torch.arange(L, dtype=torch.int64) + s for L, s in zip(lengths, starts)]) \
        if B else torch.zeros((0,), dtype=torch.int64)
    pos = tok % T
    nxt = torch.where(pos + 1 < T, tok + 1, torch.full_like(tok, B * T))
    cu = torch.tensor([0, *itertools.accumulate(lengths)], dtype=torch.int64)
    return torch.cat([tok, nxt, pos, cu])


class Packed:
    """A right-padded micro-batch with its padding dropped: the real tokens of all rows, back to
    back, with the fields the reference's packing provides (engine.py:705-764): tok (each
    token's index in the padded [B, T] batch), ids, pos (position within its sequence),
    targets (next-token labels, -100 ignored), head_order (supervised tokens first),
    n_supervised, cu_seqlens, lengths, max_len, and the rotary tables.

    Whatever follows from the row lengths is computed on the host and reaches the device in one
    pinned copy. The lengths come from the caller when it has them (`lengths`, `n_supervised`:
    a collator knows both), which spares the step its one read of the device: a read waits for
    all queued work, the previous step's backward included, and the GPU then idles while this
    step's first launches are queued. The caller's metadata is then checked on the device
    without waiting: `metadata_ok` is a device bool, False when the mask is not right-padded to
    the given lengths or the supervised count differs (read it when the step is synchronised
    anyway). A caller's count that overstates the supervised tokens costs work only (the head
    zeroes the ignored rows it then takes in); one that understates them drops supervised rows
    from the head's gradient, which metadata_ok reports. Without lengths the count is read with
    them, and a caller's n_supervised that differs raises ValueError. `sup_exact`: n_supervised
    is the device's own count.

    `padded=True` keeps the padding in place instead (device-only packing): every row is one
    sequence of T tokens, its padding after its real tokens, so causal attention keeps the
    padding out of every real token's result, and the padding tokens take no label. Nothing is
    read from the device and no host lengths are needed: every shape follows from [B, T], so
    the step can be captured in a HIP graph (StepGraph). The step then computes over B*T rows;
    n_supervised is B*T, an upper bound (the head's unsupervised rows take a zero gradient);
    metadata_ok reports on the device whether the mask was right-padded. `ctr_base`: a device
    int64 holding the step's first dropout counter; the masks' counters are then relative to
    it (padded batches only)."""

    def __init__(self, input_ids, attention_mask, labels, rope, dropout, dropout_p, lengths=None,
                 n_supervised=None, padded=False, ctr_base=None):
        if input_ids.dim() != 2 or attention_mask.shape != input_ids.shape \
                or labels.shape != input_ids.shape:
            raise UnsupportedBatch("inputs are not [rows, tokens]")
        self.ctr_base, self.drawn = None, 0
        if padded:
            self._pack_padded(input_ids, attention_mask, labels, ctr_base)
        else:
            if ctr_base is not None:
                raise ValueError("a device counter base needs padded=True")
            self._pack(input_ids, attention_mask, labels, lengths, n_supervised)
        self.cos, self.sin = rope.table(max(self.max_len, 1))
        self.dropout_p, self.dropout = dropout_p, dropout
        self.drop_seed = self.drop_threads = None  # set by the step's first draw
        self.drop_vec = dropout.vec if dropout is not None else 4
        self.lora16_views = self.lora16t_views = None
        self.grad16 = None  # (dh, fp16(dh)) handed from a layer's backward to the one below

    def _pack_padded(self, input_ids, attention_mask, labels, ctr_base):
        B, T = input_ids.shape
        dev = input_ids.device
        self.rows, self.T, self.lengths = B, T, [T] * B
        self.max_len = T
        self.cu_seqlens_host = [T * r for r in range(B + 1)]
        n = self.n = B * T
        self.tok = torch.arange(n, device=dev)
        self.pos = (self.tok % max(T, 1)).to(torch.int32)
        self.cu_seqlens = torch.arange(0, n + 1, max(T, 1), device=dev, dtype=torch.int32)
        self.ids = input_ids.reshape(-1)
        real = attention_mask.bool()
        nxt = torch.cat([labels[:, 1:], torch.full_like(labels[:, :1], -100)], dim=1)
        self.targets = torch.where(real, nxt, torch.full_like(nxt, -100)).reshape(-1)
        self.head_order = torch.argsort((self.targets < 0).to(torch.int8), stable=True)
        self.n_supervised = n
        self.sup_exact = False  # n_supervised counts ignored tokens too
        right = torch.arange(T, device=dev)[None, :] < real.sum(dim=1, keepdim=True)
        self.metadata_ok = (real == right).all()
        if ctr_base is not None:
            if ctr_base.dtype != torch.int64 or ctr_base.numel() != 1 or \
                    ctr_base.device != dev:
                raise ValueError("ctr_base must be one int64 on the batch's device")
            self.ctr_base = ctr_base

    def _pack(self, input_ids, attention_mask, labels, lengths, n_supervised):
        B, T = input_ids.shape
        dev = input_ids.device
        given = lengths is not None
        # whether n_supervised is the device's own count (else the caller's, checked on the
        # device without a read: metadata_ok)
        exact = not given or n_supervised is None
        if not given:
            lengths, counted = _read_lengths(attention_mask, labels)
            if n_supervised is not None and int(n_supervised) != counted:
                raise ValueError(f"n_supervised {int(n_supervised)} differs from the batch's "
                                 f"{counted} supervised tokens")
            n_supervised = counted
        lengths = [int(x) for x in lengths]
        if len(lengths) != B or any(not 0 <= x <= T for x in lengths):
            raise UnsupportedBatch("lengths do not fit the batch")
        self.rows, self.T, self.lengths = B, T, lengths
        self.max_len = max(lengths, default=0)
        self.cu_seqlens_host = [0, *itertools.accumulate(lengths)]
        n = self.n = self.cu_seqlens_host[-1]
        index = _to_device(_pack_index(lengths, T), dev)
        self.tok = index[:n]
        self.pos = index[2 * n:3 * n].to(torch.int32)
        self.cu_seqlens = index[3 * n:].to(torch.int32)
        self.ids = input_ids.reshape(-1).index_select(0, self.tok)
        sentinel = torch.full((1,), -100, device=dev, dtype=labels.dtype)
        self.targets = torch.cat([labels.reshape(-1), sentinel]).index_select(0, index[n:2 * n])
        unsupervised = self.targets < 0
        self.head_order = torch.argsort(unsupervised.to(torch.int8), stable=True)
        counted = (n - unsupervised.sum()) if n_supervised is None or given else None
        self.n_supervised = int(counted) if n_supervised is None else int(n_supervised)
        self.sup_exact = exact
        self.metadata_ok = None
        if given:
            cu = index[3 * n:]
            right = torch.arange(T, device=dev)[None, :] < (cu[1:] - cu[:-1])[:, None]
            self.metadata_ok = (attention_mask.bool() == right).all() & \
                (counted == self.n_supervised)

    @property
    def row_of_token(self):
        """Each packed token's row of the batch (int64 [n], on the device)."""
        return self.tok // self.T

    def lora16(self, index, weights):
        if self.lora16_views is not None:
            return self.lora16_views[index]
        return tuple(None if t is None else t.detach().to(torch.float16) for t in weights)

    def lora16t(self, index, lora16):
        """(A_q^T, B_q^T, A_v^T, B_v^T) fp16 contiguous: the backward's operand layout."""
        if self.lora16t_views is not None:
            return self.lora16t_views[index]
        return tuple(None if t is None else t.t().contiguous() for t in lora16)

    def draw(self, H):
        """The counter of this step's next LoRA dropout mask: the next nn.Dropout call of the
        base, on its padded [B, T, H] LoRA input (engine.py:758-764). Every call of one step
        has the same seed and launch size. With a device counter base the counter is relative
        to the step's first and the generator is left alone: `drawn` counts the offset the
        step's draws cover, by which the caller moves the generator."""
        if self.ctr_base is not None:
            if (self.rows * self.T * H) % self.dropout.vec:
                raise ValueError("the LoRA input is not whole vector accesses")
            threads, advance = self.dropout.launch(self.rows * self.T * H)
            seed, ctr = _as_int64(self.dropout.gen.initial_seed()), self.drawn // 4
            self.drawn += advance
        else:
            seed, ctr, threads = self.dropout.draw(self.rows * self.T * H)
        if self.drop_seed is None:
            self.drop_seed, self.drop_threads = seed, threads
        elif (seed, threads) != (self.drop_seed, self.drop_threads):
            raise RuntimeError("the dropout generator was reseeded during the step")
        return ctr


# ---------------------------------------------------------------------------------------------
# Attention (engine.py:857-869): the HIP varlen causal kernels of ops (_attn_fwd/_attn_bwd) read
# k and v in their grouped layout [n, HKV, D]; dk/dv come back per q head and the RoPE backward
# sums each group, as the reference's backward through the repeated k/v does.
# ---------------------------------------------------------------------------------------------
# ---------------------------------------------------------------------------------------------
# One decoder layer (engine.py:1054-1340)
# ---------------------------------------------------------------------------------------------
def attn_input_fwd(spec, h, packed, lora16, seeds, keep_bits=False, qkv=None, bits=None,
                   lora_x=None):
    """The attention-input block (engine.py:1073-1109): input RMSNorm with the two LoRA-dropout
    copies, the qkv projection (+ bias), the q/v LoRA products and RoPE. Returns q [n, HQ, D],
    k and v in grouped layout [n, HKV, D], and what attn_input_bwd reads. keep_bits: store the
    dropout masks as bits for the backward (else it draws them again). qkv: (q, k, v) kept from
    the forward (a backward's recompute): then only the norm and the LoRA inputs' products
    the gradients read are formed again (no projection, no RoPE). bits: the masks the forward
    stored, which a recompute reads instead of drawing them again (and hands to the backward).
    lora_x: the forward's rank-r products (xq, xv) with qkv (not formed again)."""
    n, H = h.shape
    aq_w, bq_w, av_w, bv_w = lora16
    s = _lora_scale(spec)
    # LoRA dropout (engine.py:767-805); p = 0 is the identity (nn.Identity in PEFT), so both
    # adapters read the normed rows themselves
    drop = packed.dropout is not None
    drop_q, drop_v = drop and aq_w is not None, drop and av_w is not None
    bits = bits if drop_q or drop_v else None
    kbits = (torch.empty(keep_bits_shape(n, H), device=h.device, dtype=torch.uint8)
             if keep_bits and (drop_q or drop_v) and bits is None else None)
    _, a, aq, av, rstd1 = _rms_fwd(spec, h, spec.ln1, packed, seeds=seeds, drop_q=drop_q,
                                   drop_v=drop_v, keep=kbits, keep_in=bits,
                                   write_y=qkv is None or not drop)
    if bits is not None:
        kbits = bits
    if not drop:
        aq, av = (a if aq_w is not None else None), (a if av_w is not None else None)
    if qkv is not None:
        del a
        if lora_x is not None:
            xq, xv = lora_x
        else:
            xq, xv, _, _ = _lora_fwd_rows(aq, av, aq_w, bq_w, av_w, bv_w, need_l=False)
        q, k, v = qkv
        return q, k, v, dict(rstd1=rstd1, aq=aq, av=av, xq=xq, xv=xv, keep=kbits)
    proj = L.nf4_linear(a, spec.qkv, bias=spec.bias_qkv)
    del a
    xq, xv, lq, lv = _lora_fwd_rows(aq, av, aq_w, bq_w, av_w, bv_w)
    q, k, v = _rope_fwd(spec, proj, lq, lv, packed, s, kv_heads=spec.HKV)
    return q, k, v, dict(rstd1=rstd1, aq=aq, av=av, xq=xq, xv=xv, keep=kbits)


def attn_input_bwd(spec, dq, dk, dv, h, saved, packed, lora16t, seeds, dres=None,
                   need_dh=True):
    """Backward of attn_input_fwd (engine.py:1296-1338) from dq [n, HQ, D] and dk, dv per q
    head [n, HQ, D] (or grouped): (dh fp32 [n, H] or None, its fp16 copy, (dA_q, dB_q, dA_v,
    dB_v) fp32). dres: the residual stream's gradient added to dh."""
    s = _lora_scale(spec)
    n, H = h.shape
    D, HQ, HKV = spec.D, spec.HQ, spec.HKV
    C = (HQ + 2 * HKV) * D
    dqkv = _rope_bwd(spec, dq, dk, dv, packed)
    da = L.nf4_linear_t(dqkv, spec.qkv) if need_dh else None
    # LoRA (engine.py:1319-1331): dx = s g B and t = dx A per token in one kernel for both
    # adapters; the token reductions dB = s g^T x and dA = dx^T drop(a) of both in another
    qc, vc = slice(0, HQ * D), slice((HQ + HKV) * D, C)
    lt = lora16t
    dxq, dxv, tq, tv = _lora_bwd_rows(dqkv, qc, vc, lt[0], lt[1], lt[2], lt[3], s,
                                      need_t=need_dh)
    grads = _lora_grad(dqkv, qc, vc, saved["xq"], saved["xv"], saved["aq"], saved["av"], dxq,
                       dxv, s)
    del dqkv
    dh = dh16 = None
    if need_dh:
        dh16 = torch.empty((n, H), device=h.device, dtype=torch.float16)
        dh = _rms_bwd(spec, da, h, saved["rstd1"], spec.ln1, packed, dres=dres, tq=tq, tv=tv,
                      seeds=seeds, out16=dh16, keep=saved["keep"])
    return dh, dh16, grads


ATTN_KEPT = ("q", "k", "v", "out", "lse", "aseed", "aoffset", "o")


def _layer_forward(spec, h, packed, lora16, seeds, keep, kept=None, save=()):
    """The layer's forward.
    keep=True: returns (None, everything the backward reads). `kept`: what the forward kept
    (a recomputing layer's backward), used instead of computing it again: the [gate|up] product
    ("gu") and the attention's q, k, v, output, log-sum-exp and o_proj output (ATTN_KEPT); with
    both, only the two RMSNorms and the LoRA inputs' products are formed again.
    keep=False: (h3, kept) with the tensors `save` names ("gu": the product, written beside the
    SwiGLU by the same GEMM; "attn": ATTN_KEPT) for the backward."""
    n, H = h.shape
    D, HQ = spec.D, spec.HQ
    kept = kept or {}
    has_attn = "o" in kept
    # the dropout masks as bits: a keeping layer's backward reads them; a recomputing layer's
    # forward stores them for its recompute, which reads them instead of drawing them again
    q, k, v, f = attn_input_fwd(spec, h, packed, lora16, seeds,
                                keep_bits=keep or "bits" in save,
                                qkv=(kept["q"], kept["k"], kept["v"]) if has_attn else None,
                                bits=kept.get("bits"), lora_x=kept.get("lora_x"))
    if has_attn:
        out, lse, aseed, aoffset, o = (kept[x] for x in ATTN_KEPT[3:])
    else:
        out, lse, aseed, aoffset = _attn_fwd(q, k, v, packed, spec.scale)
        o = L.nf4_linear(out.reshape(n, HQ * D), spec.w["o_proj"])
    gu = kept.get("gu")
    if keep and gu is not None and getattr(packed, "norm_in_bwd", False):
        # a recompute with the [gate|up] product kept needs the post-attention norm only for
        # its backward, which forms h2 = h + o and its rstd itself (the same bits)
        f.update(q=q, k=k, v=v, out=out, lse=lse, aseed=aseed, aoffset=aoffset, h2=None,
                 rstd2=None, o2=o, gu=gu)
        return None, f
    h2, b, _, _, rstd2 = _rms_fwd(spec, h, spec.ln2, packed, delta=o,
                                  write_y=not (keep and gu is not None))
    saved = {}
    if not keep and "attn" in save:
        saved.update(q=q, k=k, v=v, out=out, lse=lse, aseed=aseed, aoffset=aoffset, o=o)
    if not keep and f["keep"] is not None:
        saved["bits"] = f["keep"]
    if not keep and "lora_x" in save and "attn" in save:
        saved["lora_x"] = (f["xq"], f["xv"])
    del o
    if keep:
        if gu is None:
            gu = L.nf4_linear_gu(b, spec.gu)
        f.update(q=q, k=k, v=v, out=out, lse=lse, aseed=aseed, aoffset=aoffset, h2=h2,
                 rstd2=rstd2, gu=gu)
        return None, f
    # gate|up GEMM with the SwiGLU in its epilogue ([gate|up] not stored unless kept for the
    # backward), then down_proj with the residual add in its epilogue: h3 = h2 + fp16(m W_d^T)
    both = L.nf4_linear_swiglu_keep(b, spec.gu, spec.I) if "gu" in save else None
    if both is not None:
        m, saved["gu"] = both
    else:
        m = L.nf4_linear_swiglu(b, spec.gu, spec.I)
    del b
    return L.nf4_linear_resid(m, spec.w["down_proj"], h2), saved


class _Layer(torch.autograd.Function):
    """One decoder layer: input (fp32 residual) kept; the backward recomputes the forward with
    the same dropout counters (or reads the kept intermediates) and goes back through it. The
    LoRA weights are inputs, so autograd hands their gradients to the optimizer."""

    @staticmethod
    def forward(ctx, h, spec, packed, keep_all, aq_w, bq_w, av_w, bv_w):
        with L.reuse_dequant() as weights:  # the layer's weights in one dequant launch
            # (a recomputing layer's gate|up product decodes its NF4 weight itself)
            fused_gu = not keep_all and L.swiglu_fused_nf4() and L._gemm_fits(spec.I, spec.H)
            L.dequant_layer(spec.nf4_nogu if fused_gu else spec.nf4_all)
            h3 = _Layer._forward(ctx, h, spec, packed, keep_all, aq_w, bq_w, av_w, bv_w)
        # a layer that keeps its intermediates may keep its dequantized weights as well, so
        # that its backward does not dequantize the same NF4 weights a second time
        keep_w = getattr(packed, "keep_weights", False) if keep_all else \
            getattr(packed, "keep_weights_recompute", False)
        ctx.weights = weights.copies if keep_w else None
        return h3

    @staticmethod
    def _forward(ctx, h, spec, packed, keep_all, aq_w, bq_w, av_w, bv_w):
        drop = packed.dropout is not None
        seeds = (packed.draw(spec.H) if drop else 0, packed.draw(spec.H) if drop else 0)
        lora16 = packed.lora16(spec.index, (aq_w, bq_w, av_w, bv_w))
        if keep_all:
            _, f = _layer_forward(spec, h, packed, lora16, seeds, keep=True)
            m = _glu_fwd(f["gu"], spec.I)
            h3 = L.nf4_linear_resid(m, spec.w["down_proj"], f["h2"])
            del m
            ctx.kept = f
        else:
            # a recomputing layer keeps its [gate|up] product for the backward (the reference's
            # plan keeps it first, on the GPU or in host memory, engine.py:1204-1213, 430-445):
            # the backward then recomputes the forward up to the MLP input only
            save = (("gu",) if getattr(packed, "keep_gu", False) else ()) + \
                (("attn",) if getattr(packed, "keep_attn", False) else ()) + \
                (("bits",) if getattr(packed, "keep_bits", False) else ()) + \
                (("lora_x",) if getattr(packed, "keep_lora_x", False) else ())
            h3, ctx.saved_fwd = _layer_forward(spec, h, packed, lora16, seeds, keep=False,
                                               save=save)
            ctx.kept = None
        ctx.save_for_backward(h, aq_w, bq_w, av_w, bv_w)
        ctx.spec, ctx.packed, ctx.seeds = spec, packed, seeds
        return h3

    @staticmethod
    def backward(ctx, dh3):
        h, aq_w, bq_w, av_w, bv_w = ctx.saved_tensors
        spec, packed, seeds = ctx.spec, ctx.packed, ctx.seeds
        kept, ctx.weights = ctx.weights, None
        # one dequant launch for the recompute and the dY W products (none with kept weights)
        with L.reuse_dequant(kept):
            L.dequant_layer(spec.nf4_all)
            return _Layer._backward(ctx, dh3, h, aq_w, bq_w, av_w, bv_w, spec, packed, seeds)

    @staticmethod
    def _backward(ctx, dh3, h, aq_w, bq_w, av_w, bv_w, spec, packed, seeds):
        n, H = h.shape
        D, HQ = spec.D, spec.HQ
        dh3 = dh3.contiguous()
        # the fp16 copy of this gradient written by the layer above's norm backward, when the
        # gradient is that very tensor; else it is rounded on load (dY.to(fp16) W)
        g16 = packed.grad16
        dh3_16 = g16[1] if g16 is not None and g16[0] is dh3 else dh3
        packed.grad16 = None
        lora16 = packed.lora16(spec.index, (aq_w, bq_w, av_w, bv_w))
        dm = L.nf4_linear_t(dh3_16, spec.w["down_proj"])
        del dh3_16
        if ctx.kept is not None:
            f, ctx.kept = ctx.kept, None
        else:
            saved, ctx.saved_fwd = getattr(ctx, "saved_fwd", None), None
            with torch.no_grad():
                _, f = _layer_forward(spec, h, packed, lora16, seeds, keep=True, kept=saved)
            del saved
        gu = f.pop("gu")
        _glu_bwd(dm, gu, spec.I)
        del dm
        # a split-K plan's slices go to the norm backward unsummed (it sums them in the
        # reduce's order): no reduce launch, no fp16 round trip of db
        db, db_parts = L.nf4_linear_t_parts(gu, spec.gu) if getattr(
            packed, "parts_to_norm", False) else (L.nf4_linear_t(gu, spec.gu), None)
        del gu
        dh2_16 = torch.empty((n, H), device=h.device, dtype=torch.float16)
        h2, o2 = f.pop("h2"), f.pop("o2", None)
        dh2 = _rms_bwd(spec, db, h if h2 is None else h2, f.pop("rstd2"), spec.ln2, packed,
                       dres=dh3, out16=dh2_16, xdelta=o2 if h2 is None else None,
                       dy_parts=db_parts)
        del h2, o2, db_parts
        del db, dh3
        dout = L.nf4_linear_t(dh2_16, spec.w["o_proj"]).view(n, HQ, D)
        del dh2_16
        dq, dk, dv = _attn_bwd(dout, f.pop("q"), f.pop("k"), f.pop("v"), f.pop("out"),
                               f.pop("lse"), f.pop("aseed"), f.pop("aoffset"), packed,
                               spec.scale)
        del dout
        need_dh = ctx.needs_input_grad[0]
        dh, dh16, (dA_q, dB_q, dA_v, dB_v) = attn_input_bwd(
            spec, dq, dk, dv, h, f, packed, packed.lora16t(spec.index, lora16), seeds,
            dres=dh2, need_dh=need_dh)
        del dq, dk, dv
        if need_dh:
            packed.grad16 = (dh, dh16)
        return dh, None, None, None, dA_q, dB_q, dA_v, dB_v


# ---------------------------------------------------------------------------------------------
# Final norm + lm_head + cross-entropy (engine.py:1352-1400)
# ---------------------------------------------------------------------------------------------
class HeadStats:
    """Row order, per-token loss, entropy and correct of the head (the logged metrics)."""


class _NormSpec:
    """The one field the RMSNorm wrappers read from a layer spec."""

    def __init__(self, eps):
        self.eps = eps


class _Head(torch.autograd.Function):
    """Final RMSNorm, the tied lm_head and the cross-entropy over the packed tokens: the loss
    sum(tok_loss) / denom and the logged per-token loss, entropy and accuracy (the outputs of
    engine.py:1352-1400).

    The loss is linear in the per-token losses, so its gradient w.r.t. h is formed during the
    forward and the backward only scales it. Tokens are taken in packed.head_order (supervised
    first). Per slab of at most `chunk` tokens: one GEMM forms the logits, the CE kernel
    reduces each row and overwrites it with softmax - onehot (with zeros for an ignored token's
    row below n_supervised), and the slab's first n_supervised rows alone go through G E and the
    norm's backward (scaled by 1/denom); the other rows' gradient is zero."""

    @staticmethod
    def forward(ctx, h, norm_w, eps, lm_w, packed, denom, stats, chunk):
        n = h.shape[0]
        dev = h.device
        norm = _NormSpec(eps)
        order, n_sup = packed.head_order, packed.n_supervised
        rows = h.index_select(0, order)
        targets = packed.targets.index_select(0, order)
        _, hn, _, _, rstd = _rms_fwd(norm, rows, norm_w, packed)
        tok_loss, entropy = (torch.empty((n,), device=dev, dtype=torch.float32)
                             for _ in range(2))
        correct = torch.empty((n,), device=dev, dtype=torch.int32)
        grad_rows = torch.zeros_like(rows)
        # a device denominator (a captured step) divides in the loss and in the backward's
        # incoming gradient; a host one scales the norm backward's output directly
        ctx.denom = denom if isinstance(denom, torch.Tensor) else None
        if ctx.denom is not None:
            scale = 1.0
        else:
            # a batch without supervised tokens: NaN, what sum / 0 of an empty sum gives
            scale = 1.0 / float(denom) if float(denom) else float("nan")
        for lo in range(0, n, chunk):
            hi = min(n, lo + chunk)
            logits = L.linear(hn[lo:hi], lm_w)
            # G E reads the rows below n_sup: an ignored token's row among them (n_sup an
            # upper bound: device-only packing, or a caller's count that overstates) is zeroed
            # by the CE kernel; the rows from n_sup on are never read again and keep what the
            # kernel leaves (no zero writes)
            top = min(hi, n_sup)
            for a, b, zero in ((lo, top, True), (max(lo, top), hi, False)):
                if b > a:
                    _ce(logits[a - lo:b - lo], targets[a:b], tok_loss[a:b], entropy[a:b],
                        correct[a:b], zero_unsupervised=zero)
            if top > lo:
                # a split-K plan's slices summed by the norm backward (the reduce's order)
                g_hn, g_parts = L.hgemm_parts(logits[:top - lo], lm_w, 1) if getattr(
                    packed, "parts_to_norm", False) else (L.linear_t(logits[:top - lo], lm_w),
                                                          None)
                _rms_bwd(norm, g_hn, rows[lo:top], rstd[lo:top], norm_w, packed,
                         grad_scale=scale, out=grad_rows[lo:top], dy_parts=g_parts)
                del g_hn, g_parts
            del logits
        dh = torch.empty_like(h).index_copy_(0, order, grad_rows)
        ctx.save_for_backward(dh)
        stats.order, stats.tok_loss, stats.entropy, stats.correct = \
            order, tok_loss, entropy, correct
        if ctx.denom is not None:
            return tok_loss.sum() / ctx.denom
        return tok_loss.sum() * scale

    @staticmethod
    def backward(ctx, grad):
        (dh,) = ctx.saved_tensors
        g = grad if ctx.denom is None else grad / ctx.denom
        return dh * g, None, None, None, None, None, None, None

# ---------------------------------------------------------------------------------------------
# The model
# ---------------------------------------------------------------------------------------------
def check_gemm_shapes(cfg):
    """Raise UnsupportedModel unless the package's GEMM takes every product of the step: each
    projection and the lm_head forward (NT) and their input gradients (NN), the reduction in
    blocks of 128 (every Qwen2 size: H, I, the q/k/v widths and the vocabulary are)."""
    H, I, V = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    qkv = (cfg.num_attention_heads + 2 * cfg.num_key_value_heads) * cfg.head_dim
    o = cfg.num_attention_heads * cfg.head_dim
    fwd = [(H, qkv), (o, H), (H, 2 * I), (I, H), (H, V)]  # (K, N) of y = x W^T
    ok = all(L.tiles(k, n, 0) and L.tiles(n, k, 1) for k, n in fwd) and I % 128 == 0
    if not ok:
        raise UnsupportedModel(
            f"hidden {H}, intermediate {I}, q/k/v width {qkv}, o width {o}, vocabulary {V}: "
            "the step's GEMM takes sizes that are multiples of 128")


class FusedQwen2:
    """The step of a Qwen2 NF4 + LoRA model (engine.py:1568-1922 without the host offload).

    By default every layer recomputes its forward in the backward from its fp32 input
    (`keep_all=False`, the per-layer recompute of the reference's step) as far as the reference's
    step does: its [gate|up] product (`keep_gu`) and its attention's q, k, v, output and o_proj
    output (`keep_attn`) are kept from the forward, as the reference keeps them (GuStream,
    AttnStream: in host memory on its GPU, in HBM here), and the backward forms the two
    RMSNorms and the LoRA inputs' products again; the layer's dequantized weights are kept too
    (`keep_weights_recompute`: the frozen weights stay resident in fp16 between the forward and
    the backward, 2.6 GB for the 1.5B model, instead of a second dequant). `keep_all=True`
    keeps every layer's intermediates instead; `keep_all=None` follows the reference's
    memory-cap plan (keep_plan, engine.py:1626-1640): the last layers keep
    everything as long as the step's predicted peak stays under the cap (the GPU's memory less
    a margin by default)."""

    HEAD_CHUNK = 4096  # rows of logits alive at a time (4096 x 151936 fp16 = 1.2 GB)
    CAP_MARGIN = 8 * 2**30  # bytes of device memory the default cap leaves free

    def __init__(self, cfg, layers, embed, norm_w, device, keep_all=False):
        check_gemm_shapes(cfg)
        self.cfg = cfg
        self.layers = layers
        self.embed = embed
        self.lm_w = embed  # tied
        self.norm_w = norm_w
        self.eps = cfg.rms_norm_eps
        self.device = torch.device(device)
        self.keep_all = keep_all
        self.memory_cap = None
        # layers that keep their intermediates also keep their dequantized weights for the
        # backward (one dequant per layer and step instead of two; 94 MB per 1.5B layer)
        self.keep_weights = True
        # ... and so does a recomputing layer (94 MB per 1.5B layer, 2.6 GB for the 28: the
        # frozen weights stay resident in fp16 from the forward to the backward, which then
        # skips the layer's second dequant; the activations are still recomputed). Config-5 step
        # on one box: 29.51 -> 28.80 ms
        self.keep_weights_recompute = True
        # recomputing layers keep their [gate|up] product (2 I fp16 per token: 2.6 GB over a
        # 1.5B step of 2,560 tokens) and recompute their forward up to the MLP input only, the
        # reference's plan (its [gate|up] is kept first, on the GPU or in pinned host memory,
        # engine.py:1204-1213, 430-445); False: they multiply again
        self.keep_gu = True
        # ... and the attention's q, k, v, output, log-sum-exp and o_proj output (about 10 KB a
        # token), so their backward recomputes only the two RMSNorms and the LoRA inputs'
        # products: the reference's AttnStream (engine.py:560-571), on by default there
        # (OFFLOAD_ATTN, patch.py:45-51) where host copies are fast enough; False: recompute
        self.keep_attn = True
        # ... and the input norm's two LoRA-dropout masks as bits (H / 4 bytes a token), which
        # the recompute reads instead of drawing them again with Philox (the same bits)
        self.keep_bits = True
        # the recompute's post-attention norm (h2 = h + o and its rstd: the [gate|up] product
        # kept, nothing else reads them) formed inside that norm's backward kernel rather than
        # by a forward launch of its own (the same bits)
        self.norm_in_bwd = True
        # ... and its LoRA inputs' rank-r products x = drop(a) A^T (2 r fp16 a token), so a
        # recompute with the attention tensors kept forms only the input norm again
        self.keep_lora_x = True
        # the gate|up input gradient's (and the head's dh = G E) split-K slices summed by the
        # following norm backward (the reduce's order: the same bits) instead of a reduce launch
        self.parts_to_norm = True
        self.dropout_p = cfg.lora_dropout
        self.rope = RopeTable(cfg.rope_theta, cfg.head_dim, self.device)
        self.dropout = TorchDropout(self.device, torch.float32) if self.dropout_p > 0 else None
        # one fp16 buffer for every LoRA weight, refreshed by a single foreach copy per step
        # (engine.py:1599-1624)
        self.lora_fp32 = [t for spec in layers for t in spec.lora_params()]
        total = sum(t.numel() for t in self.lora_fp32)
        self.lora_buf = torch.empty((total,), device=self.device, dtype=torch.float16)
        views, start = [], 0
        for t in self.lora_fp32:
            views.append(self.lora_buf[start:start + t.numel()].view(t.shape))
            start += t.numel()
        self.lora_views = views
        self.lora16_by_layer = [tuple(views[4 * i:4 * i + 4]) for i in range(len(layers))]
        # the same fp16 weights transposed (A^T [H, r], B^T [r, N]), for the backward: per kind
        # one [L, ...] tensor refreshed by one strided copy from lora_buf
        nl = len(layers)
        shapes = [tuple(t.shape) for t in self.lora_fp32]
        per_layer = total // nl
        self.lora_t_src, self.lora_t = [], []
        if all(shapes[4 * i:4 * i + 4] == shapes[:4] for i in range(nl)):
            off = 0
            for d0, d1 in shapes[:4]:
                self.lora_t_src.append(self.lora_buf.as_strided((nl, d1, d0),
                                                                (per_layer, 1, d1), off))
                self.lora_t.append(torch.empty((nl, d1, d0), device=self.device,
                                               dtype=torch.float16))
                off += d0 * d1
            self.lora16t_by_layer = [tuple(t[i] for t in self.lora_t) for i in range(nl)]
        else:
            self.lora16t_by_layer = None

    def parameters(self):
        return list(self.lora_fp32)

    def set_memory_cap(self, cap_bytes):
        """The step may keep activations as long as its predicted peak stays under this
        (engine.py:1626-1628); None = the device's memory less CAP_MARGIN."""
        self.memory_cap = cap_bytes

    def kept_bytes_per_layer(self, n):
        """Device bytes one layer's kept intermediates take for n tokens: the fp16 LoRA inputs
        (2 H), q/k/v and the attention output ((2 HQ + 2 HKV) D), the fp32 residual after
        attention (H), [gate | up] (2 I), the log-sum-exp, the two rstd and the dropout keep
        bits (2 ceil(H / 4) bytes)."""
        spec = self.layers[0]
        per_token = (2 * spec.H * 2 + (2 * spec.HQ + 2 * spec.HKV) * spec.D * 2 + spec.H * 4
                     + 2 * spec.I * 2 + spec.HQ * 4 + 2 * 4 + 2 * 16 * 2 + 2 * ((spec.H + 3) // 4))
        return n * per_token

    def recompute_bytes_per_layer(self, n):
        """Device bytes a recomputing layer holds from its forward to its backward beyond its
        fp32 input: its [gate | up] product (keep_gu: 2 I fp16 per token), its attention
        tensors (keep_attn: q, k, v, the output, the log-sum-exp and the o_proj output) and its
        dequantized weights (keep_weights_recompute)."""
        spec = self.layers[0]
        per_token = (2 * spec.I * 2 if self.keep_gu else 0)
        if self.keep_attn:
            per_token += (2 * spec.HQ + 2 * spec.HKV) * spec.D * 2 + spec.HQ * 4 + spec.H * 2
        return n * per_token + (self.weight_bytes_per_layer() if self.keep_weights_recompute
                                else 0)

    def weight_bytes_per_layer(self):
        """Device bytes of one layer's dequantized fp16 weights (qkv, o, gate|up, down)."""
        spec = self.layers[0]
        return 2 * spec.H * ((spec.HQ + 2 * spec.HKV) * spec.D + spec.HQ * spec.D + 3 * spec.I)

    def allocated_bytes(self):
        """Device memory the plan counts as taken (torch's allocator on this device)."""
        return torch.cuda.memory_allocated(self.device)

    def keep_plan(self, n):
        """The number of last layers that keep every intermediate for a step of n tokens: as
        many as fit under the memory cap above what is allocated now, one recomputing layer's
        working set (its dequantized weights and per-token buffers) and what every layer holds
        as a recomputing one (recompute_bytes_per_layer). With keep_weights a keeping layer also
        holds its dequantized weights from the forward to its backward (weight_bytes_per_layer
        more per layer)."""
        if self.keep_all is not None:
            return len(self.layers) if self.keep_all else 0
        cap = self.memory_cap
        if cap is None:
            cap = torch.cuda.get_device_properties(self.device).total_memory - self.CAP_MARGIN
        weights = self.weight_bytes_per_layer()
        work = weights + 64 * 2**20 + n * 96 * 1024 + n * self.cfg.vocab_size * 2
        rec = self.recompute_bytes_per_layer(n)
        free = cap - self.allocated_bytes() - work - len(self.layers) * rec
        per_layer = max(1, self.kept_bytes_per_layer(n) + (weights if self.keep_weights else 0)
                        - rec)
        return int(max(0, min(len(self.layers), free // per_layer)))

    def step(self, input_ids, attention_mask, labels, denom, lengths=None, n_supervised=None,
             padded=False, ctr_base=None):
        """The step's forward: (loss, packed, stats); autograd runs the backward. `lengths`
        and `n_supervised`: the batch's row lengths and supervised-token count when the caller
        has them on the host (then the step reads nothing back from the device). `padded`:
        device-only packing (Packed); `denom` may then be a device scalar and `ctr_base` the
        device int64 of the step's first dropout counter (StepGraph passes both)."""
        packed = Packed(input_ids, attention_mask, labels, self.rope, self.dropout,
                        self.dropout_p, lengths=lengths, n_supervised=n_supervised,
                        padded=padded, ctr_base=ctr_base)
        if self.dropout is not None and self.dropout.ok is None:
            self.dropout.ok = self.dropout.check(packed.rows,
                                                 min(packed.T, TorchDropout.CHECK_TOKENS),
                                                 self.cfg.hidden_size, self.dropout_p)
        if self.dropout is not None and not self.dropout.ok:
            raise UnsupportedBatch("LoRA dropout masks differ from PyTorch's on this GPU")
        with torch.no_grad():
            torch._foreach_copy_(self.lora_views, [t.detach() for t in self.lora_fp32])
            for dst, src in zip(self.lora_t, self.lora_t_src):
                dst.copy_(src)
        packed.lora16_views = self.lora16_by_layer
        packed.lora16t_views = self.lora16t_by_layer
        h = torch.nn.functional.embedding(packed.ids, self.embed).float()
        keep_from = len(self.layers) - self.keep_plan(packed.n)
        packed.keep_all_from = keep_from
        packed.keep_weights = self.keep_weights
        packed.keep_weights_recompute = self.keep_weights_recompute
        packed.keep_gu = self.keep_gu
        packed.keep_attn = self.keep_attn
        packed.keep_bits = self.keep_bits
        packed.norm_in_bwd = self.norm_in_bwd
        packed.keep_lora_x = self.keep_lora_x
        packed.parts_to_norm = self.parts_to_norm
        for i, spec in enumerate(self.layers):
            h = _Layer.apply(h, spec, packed, i >= keep_from, *spec.lora_params())
        stats = HeadStats()
        loss = _Head.apply(h, self.norm_w, self.eps, self.lm_w, packed, denom, stats,
                           self.HEAD_CHUNK)
        return loss, packed, stats


class StepGraph:
    """One training step of a FusedQwen2 (forward and backward, device-only packing) captured
    as a HIP graph for batches of one [rows, T] shape, and replayed with each new batch copied
    into the graph's input buffers: one launch of the graph instead of about a thousand kernel
    launches from Python (the reference's packing, engine.py:705-751, reads the lengths back
    from the device, which no graph can hold).

    What changes between steps reaches the graph through device memory: the batch (ids, mask,
    labels), the loss denominator and the loss scale (GradScaler's) as device scalars, and the
    step's first dropout counter (the generator's offset when the step runs, as an eager step
    would draw it; after a replay the generator moves on by the step's draws). The LoRA
    parameters' .grad are the graph's own tensors, overwritten by every replay with the step's
    gradient of loss * scale. Which layers keep their intermediates is decided at capture
    (model.keep_all; None follows the memory plan as it stands then). The LoRA weights are read
    from the fp32 parameters at every replay (the step's fp16 refresh is captured)."""

    def __init__(self, model, rows, T, warmup=2):
        dev = model.device
        self.model, self.rows, self.T = model, rows, T
        self.ids = torch.zeros((rows, T), device=dev, dtype=torch.int64)
        self.mask = torch.ones((rows, T), device=dev, dtype=torch.int64)
        self.labels = torch.zeros((rows, T), device=dev, dtype=torch.int64)
        self.denom = torch.ones((), device=dev, dtype=torch.float32)
        self.scale = torch.ones((), device=dev, dtype=torch.float32)
        self.ctr = torch.zeros((1,), device=dev, dtype=torch.int64)
        drop = model.dropout
        self.seed = _as_int64(drop.gen.initial_seed()) if drop is not None else None
        params = model.parameters()
        for p in params:
            p.grad = None
        # eager runs first, on a side stream: the GEMM choices for rows * T tokens, the dropout
        # self-check, the libraries' workspaces, the attention's second stream and the caching
        # allocator's blocks are then in place, and the capture only records launches
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self._run()
                for p in params:
                    p.grad = None
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            loss, self.packed, self.stats = self._run()
        # the loss without its autograd graph: holding the graph would keep its nodes (the
        # AccumulateGrad nodes of the captured stream among them) alive across later steps
        self.loss = loss.detach()
        del loss
        self.grads = [p.grad for p in params]
        self.advance = self.packed.drawn

    def _run(self):
        base = self.ctr if self.model.dropout is not None else None
        loss, packed, stats = self.model.step(self.ids, self.mask, self.labels, self.denom,
                                              padded=True, ctr_base=base)
        (loss * self.scale).backward()
        return loss, packed, stats

    def replay(self, input_ids, attention_mask, labels, denom, scale=1.0):
        """Runs the captured step on this batch ([rows, T] as captured; denom and scale host
        numbers or device scalars) and returns the loss, a device scalar the next replay
        overwrites; the parameters' .grad then hold this step's gradient of loss * scale, and
        self.stats / self.packed its per-token statistics and packing."""
        if tuple(input_ids.shape) != (self.rows, self.T):
            raise ValueError(f"the graph takes [{self.rows}, {self.T}] batches")
        self.ids.copy_(input_ids)
        self.mask.copy_(attention_mask)
        self.labels.copy_(labels)
        for dst, v in ((self.denom, denom), (self.scale, scale)):
            if isinstance(v, torch.Tensor):
                dst.copy_(v.reshape(()))
            else:
                dst.fill_(float(v))
        drop = self.model.dropout
        if drop is not None:
            if _as_int64(drop.gen.initial_seed()) != self.seed:
                raise RuntimeError("the dropout generator was reseeded after the capture")
            offset = drop.gen.get_offset()
            self.ctr.fill_(offset // 4)
            drop.gen.set_offset(offset + self.advance)
        self.graph.replay()
        for p, g in zip(self.model.parameters(), self.grads):
            p.grad = g
        return self.loss
