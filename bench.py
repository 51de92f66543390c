"""Benchmark: full Qwen2.5-1.5B NF4 + LoRA training steps on one MI355X.

A step = forward + backward with per-layer recompute as the reference's step does it (each
decoder layer keeps its input, its [gate|up] product and its attention's q, k, v, output and
o_proj output - the reference's GuStream and AttnStream, in host memory on its GPU, in HBM here -
and recomputes its two RMSNorms with the LoRA inputs' dropout and products in backward) + fp16
loss scaling (GradScaler) + fused AdamW on the LoRA parameters, over one synthetic batch of 4
packed sequences with lengths ~ U[256, 1024] and random token ids (first 25 % of each sequence
unsupervised). Random-init weights of the Qwen2.5-1.5B architecture, all linears NF4
double-quant (blocksize 64), tied fp16 embedding. `value` = tokens/s over the K timed steps,
inputs resident in HBM.

Beside it, on the same JSON line:
  loss_curve     the loss of steps 1..64 from the random init (warmup and timed steps included)
  full_recompute the same step with every layer recomputing its whole forward from its input
                 in backward (nothing but the input kept)
  keep_all       the same step with every layer keeping its intermediates (no recompute)
  roofline       the step's largest hand-written kernel by time, the package's MFMA GEMM
                 (hgemm_kernel: the gate|up forward with the SwiGLU epilogue), 2 M N K flops
                 over the dispatch-recorded duration, against the fp16 MFMA peak, over the
                 launches of four extra untimed steps (four batches' token counts)
  roofline_dequant  the step's NF4 dequant launches (the north star's dequant GB/s)
  roofline_mfma  the attention kernels against the fp16 MFMA peak (algorithmic flops of the
                 batch's causal pairs) and the package GEMM's launches by product class
  config1..4     BASELINE configs 1-4 on the GPU (dequant GB/s; MLP, attention-input block and
                 LM-head TFLOP/s on their algorithmic work), each with its CPU oracle time
  cpu_baseline   one full 28-layer step of the CPU oracle (oracle.step, torch fp32 autograd) on
                 this host's cores from the same init and batch as the GPU's first step, with
                 the two steps' loss and LoRA gradients compared

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--policy recompute|keep]
"""

import argparse
import concurrent.futures
import contextlib
import importlib
import json
import os
import statistics
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
PKG_NAME = "hack-fe30cb28-opus-5-5-ultracode_amd"

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
CURVE_STEPS = 64


def log(msg):
    print("[bench] " + msg, file=sys.stderr, flush=True)


def make_batches(count, vocab, seed=0, rows=4, lo=256, hi=1024, device="cuda"):
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(count):
        lengths = torch.randint(lo, hi + 1, (rows,), generator=g)
        T = int(lengths.max())
        ids = torch.randint(0, vocab, (rows, T), generator=g)
        mask = (torch.arange(T)[None, :] < lengths[:, None]).long()
        ids = torch.where(mask.bool(), ids, 0)
        labels = torch.where(mask.bool(), ids, -100)
        for r in range(rows):
            labels[r, :int(lengths[r]) // 4] = -100
        denom = float((labels[:, 1:] != -100).sum())
        # host-side metadata a collator has: row lengths and the supervised-token count (here
        # equal to denom: every label of a real token after the first is supervised or -100)
        meta = {"lengths": lengths.tolist(), "n_supervised": int(denom)}
        out.append((ids.to(device), mask.to(device), labels.to(device), denom,
                    int(lengths.sum()), meta))
    return out


class Trainer:
    """fp16 loss scaling (torch GradScaler, as HF Trainer with fp16) + AdamW on the LoRA
    parameters: the fused AdamW, HF TrainingArguments' default optimizer ("adamw_torch_fused")
    with torch >= 2.8, which takes the scaler's inf check on the device (no host sync)."""

    def __init__(self, model, lr=2e-4):
        self.model = model
        self.params = model.parameters()
        self.opt = torch.optim.AdamW(self.params, lr=lr, betas=(0.9, 0.999), eps=1e-8,
                                     weight_decay=0.0, fused=True)
        self.scaler = torch.amp.GradScaler("cuda", init_scale=2.0**16)

    def step(self, batch):
        ids, mask, labels, denom, _, meta = batch
        loss, packed, stats = self.model.step(ids, mask, labels, denom, **meta)
        self.scaler.scale(loss).backward()
        self.scaler.step(self.opt)
        self.scaler.update()
        self.opt.zero_grad(set_to_none=True)
        return loss


def first_step(model, batch, scale=2.0**16):
    """Loss and LoRA gradients of one step from the current state, backward through a loss
    scaled by `scale` as the trainer does, gradients unscaled; the dropout generator is put back
    where it was, so the first training step draws the same masks."""
    ids, mask, labels, denom, _, meta = batch
    gen = model.dropout.gen if model.dropout is not None else None
    seed, offset = (gen.initial_seed(), gen.get_offset()) if gen is not None else (0, 0)
    loss, packed, _ = model.step(ids, mask, labels, denom, **meta)
    (loss * scale).backward()
    grads = [p.grad.detach().clone() / scale for p in model.parameters()]
    for p in model.parameters():
        p.grad = None
    ok = packed.metadata_ok
    if gen is not None:
        gen.set_offset(offset)
    torch.cuda.synchronize()
    return {"loss": float(loss.detach()), "grads": grads, "seed": seed, "offset": offset,
            "metadata_ok": None if ok is None else bool(ok)}


GRAPH_T = 256  # a captured step's columns: the batch's longest row rounded up to a multiple


def graph_leg(pkg, trainer, batches, count=8):
    """Device-only packing and the step captured as a HIP graph (engine.StepGraph) on config-5
    batches: each batch padded to the next multiple of GRAPH_T columns, one graph per padded
    shape (the capture's time reported apart), replayed with the trainer's GradScaler scale (a
    device scalar) and followed by its AdamW step; beside it the same padded steps run eagerly.
    Tokens/s count the real tokens; the padded steps compute over rows x columns tokens."""
    model = trainer.model
    scaler, opt = trainer.scaler, trainer.opt
    padded = []
    for ids, mask, labels, denom, ntok, _ in batches[:count]:
        T = ids.shape[1]
        Tp = -(-T // GRAPH_T) * GRAPH_T

        def pad(t, v):
            return torch.nn.functional.pad(t, (0, Tp - T), value=v)
        padded.append((pad(ids, 0), pad(mask, 0), pad(labels, -100), denom, ntok))
    t0 = time.perf_counter()
    graphs = {}
    for ids, *_ in padded:
        if tuple(ids.shape) not in graphs:
            graphs[tuple(ids.shape)] = pkg.engine.StepGraph(model, *ids.shape)
    torch.cuda.synchronize()
    capture_s = time.perf_counter() - t0

    def run(replay):
        torch.cuda.synchronize()
        t = time.perf_counter()
        tokens, rows = 0, 0
        for ids, mask, labels, denom, ntok in padded:
            if replay:
                # GradScaler's scale as its device tensor (get_scale() would read it back)
                scale = scaler._scale if scaler._scale is not None else scaler.get_scale()
                graphs[tuple(ids.shape)].replay(ids, mask, labels, denom, scale)
            else:
                loss, _, _ = model.step(ids, mask, labels, denom, padded=True)
                scaler.scale(loss).backward()
            scaler.step(opt)
            scaler.update()
            opt.zero_grad(set_to_none=True)
            tokens += ntok
            rows += ids.numel()
        torch.cuda.synchronize()
        return tokens, rows, time.perf_counter() - t

    run(True)  # the first replay of each graph uploads it
    tok, rows, t_graph = run(True)
    _, _, t_eager = run(False)
    n = len(padded)
    return {"tokens_per_s_graph": tok / t_graph, "ms_per_step_graph": 1e3 * t_graph / n,
            "tokens_per_s_eager_padded": tok / t_eager, "ms_per_step_eager_padded":
                1e3 * t_eager / n, "steps": n, "real_tokens": tok, "padded_tokens": rows,
            "shapes": sorted(graphs), "capture_s": capture_s,
            "what": "device-only packing: padded [rows, T] batches (T rounded up to "
                    f"{GRAPH_T}), forward + backward replayed from a HIP graph, GradScaler + "
                    "AdamW after each; eager padded steps on the same batches beside it"}


def causal_pairs(lengths):
    return sum(L * (L + 1) // 2 for L in lengths)


def measure_step_kernels(pkg, trainer, batches, cfg):
    """Extra (untimed) steps, one per batch given (token counts spread as the timed steps'),
    with HIP events around every launch of the dequant, the attention and the GEMM entry points:
    the dequant's achieved GB/s (dispatch-recorded events), the attention forward / backward
    TFLOP/s on each batch's causal pairs (fwd: QK^T and PV, 4 D flops per pair and head; bwd: S,
    dP, dQ, dK, dV, 10 D flops per pair and head), and the package GEMM's TFLOP/s (2 M N K a
    product) over every launch and by product class, with the gate|up forward products with
    the SwiGLU epilogue (the largest MFMA kernel of the step) on their own. Rates are total
    work over total launch time across the steps."""
    P = pkg.profiling
    heads, D = cfg.num_attention_heads, cfg.head_dim
    fwd = P.LaunchTimer("qlora_attn_fwd_split", bound="mfma")
    bwd = P.LaunchTimer("qlora_attn_bwd_split", bound="mfma")
    dq = P.LaunchTimer(P.DEQUANT)
    own = P.LaunchTimer(P.DOMINANT, bound="mfma", work=P.hgemm_flops, nbytes=P.hgemm_bytes)
    # the package GEMM's other entry in the step (args a, lda, b, ldb, M, N, K, mode first):
    # the split-K slices summed by the next norm backward (gate|up dX, the head's G E); events
    # around the call (the launch gap in)
    parts = P.LaunchTimer("qlora_gemm16_parts", bound="mfma",
                          work=lambda a: 2.0 * a[4] * a[5] * a[6])
    work_f = work_b = 0.0
    with contextlib.ExitStack() as stack:
        for t in (dq, fwd, bwd, own, parts):
            stack.enter_context(t)
        for batch in batches:
            pairs = causal_pairs(batch[5]["lengths"])
            n_f, n_b = len(fwd.records), len(bwd.records)
            trainer.step(batch)
            work_f += 4.0 * D * heads * pairs * (len(fwd.records) - n_f)
            work_b += 10.0 * D * heads * pairs * (len(bwd.records) - n_b)
    torch.cuda.synchronize()
    out = [dict(fwd.summary(work_total=work_f), kernel="attn_fwd_kernel"),
           dict(bwd.summary(work_total=work_b),
                kernel="attn_delta + attn_dq + attn_dkdv kernels")]
    # the package's GEMM (qlora_gemm16, args: a, lda, b, ldb, M, N, K, mode, ..., epi at 13)
    H = cfg.hidden_size
    classes = (
        ("every package GEMM launch of the step (projections, lm_head, its dX products)", None),
        ("narrow products, K <= 2048 (qkv, o and their dX; 128 x 128 tiles)",
         lambda a: a[5] <= 2048 and a[6] <= 2048),
        ("long reductions (down forward, gate|up dX, the head's G E; 256 x 256 split-K)",
         lambda a: a[5] <= 2048 and a[6] > 2048),
        ("down dX (N = I)", lambda a: a[7] == 1 and a[5] == cfg.intermediate_size),
        ("lm_head logits (N = V)", lambda a: a[7] == 0 and a[5] == cfg.vocab_size))
    for name, sel in classes:
        r = own.summary(select=sel, also=(parts,))
        if r is not None:  # (HBM traffic was measured on the SwiGLU launches only)
            out.append(dict(r, kernel=name, traffic=None))
    mine = own.summary(select=lambda a: a[13] in P.SWIGLU_EPIS)
    if mine is not None:
        mine = dict(mine, kernel="hgemm_kernel (qlora_gemm16): the gate|up forward with the "
                                 "SwiGLU epilogue (and the [g|u] product kept for the backward), "
                                 "this package's MFMA GEMM")
    return mine, dq.summary(), out


def _median_time(fn, reps, sync=True):
    ts = []
    for _ in range(reps):
        if sync:
            torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        if sync:
            torch.cuda.synchronize()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def _event_time(fn, reps):
    """GPU seconds per call of fn over `reps` back-to-back calls, bracketed by two events behind
    a spin kernel that keeps the GPU busy while the host enqueues them (the host's Python and
    ctypes time per launch is then not in the figure; the GPU's gaps between launches are)."""
    torch.cuda.synchronize()
    h0 = time.perf_counter()
    fn()
    host_s = time.perf_counter() - h0  # the host's time to enqueue one call
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # shader-clock cycles for twice the host's enqueue time of the whole loop (2.4 GHz at most)
    torch.cuda._sleep(int(max(2e5, 2.0 * reps * host_s * 2.4e9)))
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) * 1e-3 / reps


def _nf4(pkg, g, shape, dev):
    w = (torch.randn(shape, generator=g, device=dev) * 0.02).half()
    return pkg.ops.NF4Weight(pkg.quant.quantize_nf4(w))


def _mfma_roof(flops, seconds):
    achieved = flops / seconds / 1e12
    return {"bound": "mfma", "achieved": achieved, "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": achieved / FP16_PEAK_TFLOPS}


def config1(pkg, copies=64, reps=20):
    """BASELINE config 1 on the GPU: NF4 double-quant dequant of one Qwen2.5-1.5B q_proj weight
    [1536, 1536] (N(0, 0.02) from seed 1, bitsandbytes layout), rotating over `copies`
    independent copies (> 256 MB of Infinity Cache per pass), and the same for the four weights
    of a layer in one launch (qkv | o | gate-up | down, the step's dequant). Beside them a plain
    device copy of 1 GiB (512 MiB read, 512 MiB written): the calibration kernel of the
    FETCH_SIZE / WRITE_SIZE counter runs. Returns achieved GB/s (algorithmic bytes / event
    time) and the CPU oracle's time for the same dequant."""
    from oracle import nf4 as ON
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(1)
    qs = [_nf4(pkg, g, (1536, 1536), dev) for _ in range(copies)]
    outs = [torch.empty((1536, 1536), device=dev, dtype=torch.float16) for _ in range(copies)]
    per_q = pkg.profiling._dequant_bytes([None] * 7 + [qs[0].blocks, 1, None, 64, 256,
                                                       2**63 - 1, 2**63 - 1])
    t_q = _event_time(lambda: [qs[i].dequant_into(outs[i]) for i in range(copies)], reps) \
        / copies
    layers = []
    for _ in range(8):
        grp = lambda shapes: pkg.ops.NF4Group.of([_nf4(pkg, g, sh, dev) for sh in shapes])  # noqa
        layers.append([grp([(1536, 1536), (256, 1536), (256, 1536)]),
                       _nf4(pkg, g, (1536, 1536), dev), grp([(8960, 1536), (8960, 1536)]),
                       _nf4(pkg, g, (1536, 8960), dev)])
    per_layer = sum(pkg.profiling._dequant_bytes(
        [None] * 7 + [w.blocks, 1, None, 64, 256, getattr(w, "seg1", 2**63 - 1),
                      getattr(w, "seg2", 2**63 - 1)]) for w in layers[0])
    t_l = _event_time(lambda: [pkg.ops.dequant_many(layers[i], dev) for i in range(8)], reps) / 8
    # the same 32 weights in one launch (the C-ABI's capacity): the kernel's rate once the launch
    # is large enough, beside the step's one-layer launches (which keep the weights the GEMMs
    # read next in the Infinity Cache)
    all_w = [w for lay in layers for w in lay]
    all_o = [torch.empty(w.shape, device=dev, dtype=torch.float16) for w in all_w]
    t_8 = _event_time(lambda: pkg.ops.dequant_many(all_w, dev, outs=all_o), reps)
    del all_o
    src = torch.empty(256 * 2**20, device=dev, dtype=torch.float16).normal_()
    dst = torch.empty_like(src)
    t_c = _event_time(lambda: dst.copy_(src), reps)
    # the CPU oracle's dequant of the same weight (numpy, bit-exact restatement)
    w0 = qs[0]
    st = ON.QuantState(w0.absmax.cpu().numpy(), (1536, 1536), w0.code.cpu().numpy(), 64,
                       offset=w0.offset.cpu().numpy()[0],
                       state2=ON.QuantState2(w0.absmax2.cpu().numpy(), w0.code2.cpu().numpy(),
                                             256))
    packed = w0.packed.cpu().numpy().reshape(-1)
    t_cpu = _median_time(lambda: ON.dequantize_nf4(packed, st), 5, sync=False)
    # the same dequant over the host's cores: the weight's blocks cut at double-quant group
    # boundaries, one numpy call per part on a thread pool (numpy releases the GIL in them)
    workers = len(os.sched_getaffinity(0))
    one = ON.dequantize_nf4(packed, st)
    with concurrent.futures.ThreadPoolExecutor(workers) as ex:
        assert np.array_equal(_dequant_parts(ON, packed, st, workers, ex).view(np.uint16),
                              one.view(np.uint16))
        t_cpu_n = _median_time(lambda: _dequant_parts(ON, packed, st, workers, ex), 5,
                               sync=False)
    return {"q_proj_dequant_GBs": per_q / t_q / 1e9, "q_proj_bytes": per_q,
            "q_proj_us": t_q * 1e6, "layer_dequant_GBs": per_layer / t_l / 1e9,
            "layer_bytes": per_layer, "layer_us": t_l * 1e6,
            "eight_layers_dequant_GBs": 8 * per_layer / t_8 / 1e9, "eight_layers_us": t_8 * 1e6,
            "eight_layers_frac": 8 * per_layer / t_8 / 8e12,
            "copy_GBs": 2 * src.numel() * 2 / t_c / 1e9, "copy_bytes": 2 * src.numel() * 2,
            "copies": copies,
            "cpu": {"q_proj_ms": t_cpu * 1e3, "GBs": per_q / t_cpu / 1e9, "threads": 1,
                    "q_proj_ms_threads": t_cpu_n * 1e3, "GBs_threads": per_q / t_cpu_n / 1e9,
                    "threads_used": workers, "kind": "port (oracle.nf4, numpy)"}}


def _dequant_parts(ON, packed, st, parts, ex):
    """oracle.nf4.dequantize_nf4 of a nested-quant weight in `parts` pieces on the executor `ex`,
    each a run of whole 256-block double-quant groups; the same values as one call."""
    bs, g2 = st.blocksize, st.state2.blocksize
    nb = st.absmax.size
    groups = -(-nb // g2)
    bounds = [min(nb, g2 * (groups * i // parts)) for i in range(parts + 1)]

    def part(b0, b1):
        sub = ON.QuantState(st.absmax[b0:b1], ((b1 - b0) * bs,), st.code, bs, offset=st.offset,
                            state2=ON.QuantState2(st.state2.absmax[b0 // g2:-(-b1 // g2)],
                                                  st.state2.code, g2))
        return ON.dequantize_nf4(packed[b0 * bs // 2:b1 * bs // 2], sub)

    futs = [ex.submit(part, b0, b1) for b0, b1 in zip(bounds[:-1], bounds[1:]) if b1 > b0]
    return np.concatenate([f.result() for f in futs]).reshape(st.shape)


def config2(pkg, reps=10):
    """x [2048, 1536] ~ N(0, 1), NF4 [gate|up] [17920, 1536] and down
    [1536, 8960] (N(0, 0.02), seed 2); forward h = silu(gate) up, y = h W_d^T; backward w.r.t.
    x with dy ~ N(0, 1): dh = dy W_d, [dg|du] = SwiGLU', dx = [dg|du] W_gu. Four products,
    338.2 GFLOP; the NF4 decode of both weights (the layer-wide dequant, or inside the fused
    GEMM) is in the timed region. CPU: oracle.ops.mlp on the same values."""
    from oracle import ops as O
    L, ops = pkg.linear, pkg.ops
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(2)
    gu_w = ops.NF4Group.of([_nf4(pkg, g, (8960, 1536), dev), _nf4(pkg, g, (8960, 1536), dev)])
    wd = _nf4(pkg, g, (1536, 8960), dev)
    x = torch.randn(2048, 1536, generator=g, device=dev).half()
    dy = torch.randn(2048, 1536, generator=g, device=dev).half()
    I = 8960

    def run():
        with L.reuse_dequant():
            L.dequant_layer([gu_w, wd])
            gu = L.nf4_linear(x, gu_w)
            h = ops._glu_fwd(gu, I)
            y = L.nf4_linear(h, wd)
            dh = L.nf4_linear_t(dy, wd)
            ops._glu_bwd(dh, gu, I)
            dx = L.nf4_linear_t(gu, gu_w)
        return y, dx

    flops = 2.0 * 2048 * 1536 * (2 * I) * 2 + 2.0 * 2048 * I * 1536 * 2
    t = _event_time(run, reps)
    wg, wdd = L.dequantize(gu_w).cpu(), L.dequantize(wd).cpu()
    xc, dyc = x.cpu(), dy.cpu()
    t_cpu = _median_time(lambda: O.mlp(xc, wg, wdd, dyc), 3, sync=False)
    return {"ms": t * 1e3, "gflop": flops / 1e9, "TFLOPs": flops / t / 1e12,
            "roofline": _mfma_roof(flops, t), "backend": L.BACKEND,
            "cpu": {"ms": t_cpu * 1e3, "TFLOPs": flops / t_cpu / 1e12,
                    "threads": torch.get_num_threads(), "kind": "port (oracle.ops.mlp)"}}


def config3(pkg, reps=10):
    """the attention-input block (engine.attn_input_fwd/_bwd: input RMSNorm
    with both LoRA-dropout copies, NF4 qkv projection + bias, LoRA r 16 on q and v, RoPE) on 4
    packed sequences with lengths ~ U[128, 1024] (seed 3), hidden 1536, 12/2 heads of 128,
    forward and backward (dh and the four LoRA gradients). Work: the qkv GEMMs, 4 N 1536 2048
    flops (forward and dX); HBM bytes of the RMSNorm forward (15,364 per token) and the RoPE
    forward (11,776 per token) from events around their launches. CPU: oracle.step.attn_input
    with autograd on the same sizes."""
    import numpy as np

    from oracle import step as OS
    E, P = pkg.engine, pkg.profiling
    dev = torch.device("cuda:0")
    # one layer; the block does not use the vocabulary (any multiple of 128 the GEMM takes)
    cfg = E.Qwen2Config(num_hidden_layers=1, vocab_size=1024)
    model = E.random_qwen2(cfg, dev, seed=3)
    spec = model.layers[0]
    H, HQ, HKV, D = cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads, \
        cfg.head_dim
    gl = torch.Generator().manual_seed(3)
    lengths = torch.randint(128, 1025, (4,), generator=gl).tolist()
    T = max(lengths)
    mask = (torch.arange(T)[None] < torch.tensor(lengths)[:, None]).long()
    ids = torch.zeros_like(mask)
    packed = E.Packed(ids.to(dev), mask.to(dev), torch.full_like(ids, -100).to(dev), model.rope,
                      model.dropout, model.dropout_p, lengths=lengths, n_supervised=0)
    n = packed.n
    seeds = (packed.draw(H), packed.draw(H))
    g = torch.Generator(device=dev).manual_seed(4)
    h = torch.randn(n, H, generator=g, device=dev)
    dq = torch.randn(n, HQ, D, generator=g, device=dev).half()
    dk = torch.randn(n, HQ, D, generator=g, device=dev).half()
    dv = torch.randn(n, HQ, D, generator=g, device=dev).half()
    lora = [t.detach().half() for t in spec.lora_params()]
    lora_t = [t.t().contiguous() for t in lora]

    def run():
        with pkg.linear.reuse_dequant():
            pkg.linear.dequant_layer([spec.qkv])
            q, k, v, saved = E.attn_input_fwd(spec, h, packed, lora, seeds)
            return E.attn_input_bwd(spec, dq, dk, dv, h, saved, packed, lora_t, seeds)

    t = _event_time(run, reps)
    flops = 4.0 * n * H * (HQ + 2 * HKV) * D
    rms = P.LaunchTimer("qlora_rms_fwd", work=lambda a: 15364.0 * a[10], bound="hbm")
    rope = P.LaunchTimer("qlora_rope_fwd", work=lambda a: 11776.0 * a[10], bound="hbm")
    with rms, rope:
        run()
    # CPU: the block with autograd on the same sizes
    cpu = OS.CpuQwen2(model).layers[0]
    hc = h.cpu()
    cos, sin = OS.rope_cos_sin(packed.pos.cpu().long(), D, cfg.rope_theta)
    keep = torch.rand(n, H) >= model.dropout_p
    dqc, dkc, dvc = dq.cpu().float(), dk.cpu().float(), dv.cpu().float()
    kscale = float(np.float32(1.0 / (1 - model.dropout_p)))

    def cpu_run():
        hr = hc.clone().requires_grad_()
        qo, ko, vo = OS.attn_input(cpu, hr, (keep, keep), kscale, cos, sin, HQ, HKV, D,
                                   cfg.rms_norm_eps)
        rep = HQ // HKV
        ((qo * dqc).sum() + (ko.repeat_interleave(rep, 1) * dkc).sum()
         + (vo.repeat_interleave(rep, 1) * dvc).sum()).backward()

    t_cpu = _median_time(cpu_run, 3, sync=False)
    return {"lengths": lengths, "tokens": n, "ms": t * 1e3, "gemm_gflop": flops / 1e9,
            "TFLOPs": flops / t / 1e12, "roofline": _mfma_roof(flops, t),
            "rms_fwd": rms.summary(), "rope_fwd": rope.summary(),
            "cpu": {"ms": t_cpu * 1e3, "threads": torch.get_num_threads(),
                    "kind": "port (oracle.step.attn_input + autograd)"}}


def config4(pkg, reps=3, cpu_reps=3):
    """BASELINE config 4 on the GPU: LM head loss over hidden [2048, 1536] (N(0, 1)) and the
    tied embedding [151936, 1536] (N(0, 0.02)), ~25 % of the labels ignored, with the hidden and
    embedding gradients: vocabulary pieces of 8192 (online softmax, head.chunked_head) and whole
    rows (head.full_head). Algorithmic work: the logits over all T rows (2 T V H) and the dh and
    dE products over the supervised rows (2 n_sup V H each). CPU: the oracle's cross-entropy
    with autograd over all T rows (logits, loss, dh, dE), the median of `cpu_reps` runs (the
    first pays the page faults of its 4 GB of buffers)."""
    from oracle import ops as O
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(4)
    T, V, H = 2048, 151936, 1536
    hn = torch.randn(T, H, generator=g, device=dev).half()
    E = (torch.randn(V, H, generator=g, device=dev) * 0.02).half()
    targets = torch.randint(0, V, (T,), generator=g, device=dev)
    targets[torch.rand(T, generator=g, device=dev) < 0.25] = -100
    denom = float((targets >= 0).sum())
    n_sup = int(denom)
    flops = 2.0 * T * V * H + 2 * (2.0 * n_sup * V * H)
    out = {"gflop": flops / 1e9, "n_supervised": n_sup}
    for name, fn in (("pieces", pkg.head.chunked_head), ("whole_rows", pkg.head.full_head)):
        fn(hn, E, targets, denom)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            r = fn(hn, E, targets, denom)
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / reps
        out[name] = {"ms": dt * 1e3, "TFLOPs": flops / dt / 1e12, "loss": float(r.loss),
                     "roofline": _mfma_roof(flops, dt)}
    hc, Ec, tc = hn.cpu(), E.cpu().float(), targets.cpu()

    def cpu_run():
        h = hc.float().requires_grad_()
        w = Ec.clone().requires_grad_()
        logits = h @ w.t()
        loss = torch.nn.functional.cross_entropy(logits, tc, ignore_index=-100,
                                                 reduction="sum") / denom
        loss.backward()
        return O  # (the oracle module's formulas are F.cross_entropy's)

    t_cpu = _median_time(cpu_run, cpu_reps, sync=False)
    out["cpu"] = {"ms": t_cpu * 1e3, "rows_timed": T,
                  "threads": torch.get_num_threads(), "kind": "port (torch fp32 autograd)"}
    return out


def cpu_step(pkg, model, cpu_model, batch, first):
    """The CPU oracle's full step (oracle.step.forward_loss + autograd, every layer) on the
    batch of the GPU's first step, from the same init and dropout generator state: its time is
    the CPU baseline, its loss and LoRA gradients are compared with the GPU's."""
    from oracle import step as OS
    ids, mask, labels, denom, ntok, _ = batch
    t0 = time.perf_counter()
    loss, _ = OS.forward_loss(cpu_model, ids, mask, labels, denom, drop_seed=first["seed"],
                              drop_offset=first["offset"], drop_G=model.dropout.max_blocks * 256,
                              p=model.dropout_p, vec=4)
    loss.backward()
    dt = time.perf_counter() - t0
    rels = []
    for g_gpu, leaf in zip(first["grads"], cpu_model.lora_leaves()):
        a, b = g_gpu.cpu().double(), leaf.grad.double()
        rels.append(float((a - b).norm() / b.norm().clamp_min(1e-30)))
    L = len(cpu_model.layers)
    return {"value": ntok / dt, "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": (f"one full {L}-layer step of oracle.step (torch fp32 autograd) on the "
                       f"GPU's first batch ({ntok} tokens), forward + backward: {dt:.2f} s"),
            "cpu": _cpu_model(),
            "parity": {"loss_gpu": first["loss"], "loss_cpu": float(loss),
                       "loss_rel_diff": abs(first["loss"] - float(loss)) / abs(float(loss)),
                       "lora_grad_rel_norm_max": max(rels), "lora_grads": len(rels),
                       "tolerance": {"loss": 2e-3, "lora_grad": 2e-2}}}


def _cpu_model():
    """The host CPU as the CPU-baseline record states it: model name (/proc/cpuinfo, and lscpu's
    vendor, family/model/stepping and socket/core/thread counts where lscpu runs), os.cpu_count(),
    the cores this process may run on, and torch's intra-op threads (the threads the oracle
    used)."""
    info = {"model": "unknown", "os_cpu_count": os.cpu_count(),
            "affinity_cores": len(os.sched_getaffinity(0)),
            "torch_threads": torch.get_num_threads()}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    info["model"] = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        keep = {"Vendor ID", "Model name", "CPU family", "Model", "Stepping", "Socket(s)",
                "Core(s) per socket", "Thread(s) per core", "CPU max MHz", "L3"}
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in keep:
                info["lscpu " + k.strip()] = v.strip()
    except Exception:
        pass
    return info


def time_steps(trainer, batches, start, count):
    """Runs `count` steps from batches[start]; returns (tokens, seconds, losses)."""
    torch.cuda.synchronize()
    tokens, losses = 0, []
    t0 = time.perf_counter()
    for i in range(start, start + count):
        losses.append(trainer.step(batches[i]).detach())
        tokens += batches[i][4]
    torch.cuda.synchronize()
    return tokens, time.perf_counter() - t0, [float(x) for x in losses]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--policy", choices=("recompute", "keep"), default="recompute",
                    help="recompute (config 5: every layer recomputes its forward in backward) "
                         "or keep (every layer keeps its intermediates)")
    ap.add_argument("--keep-steps", type=int, default=10,
                    help="also time this many steps with every layer keeping its "
                         "intermediates (0: skip)")
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--no-configs", action="store_true", help="skip the config 1-4 legs")
    ap.add_argument("--config1", action="store_true",
                    help="only the config-1 dequant measurement (and its copy calibration)")
    ap.add_argument("--only", choices=("config1", "config2", "config3", "config4"),
                    help="only this config leg (one JSON object; no step)")
    ap.add_argument("--profile", action="store_true",
                    help="a run to profile: no loss curve past the timed steps, no keep-all or "
                         "full-recompute extra, no config legs, no CPU baseline")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus}: this build measures one GPU only (the path is "
              "data-parallel; multi-GPU runs are out of scope)", file=sys.stderr)
        sys.exit(2)
    pkg = importlib.import_module(PKG_NAME)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.config1:
        args.only = "config1"
    if args.only:
        fn = {"config1": config1, "config2": config2, "config3": config3,
              "config4": config4}[args.only]
        print(json.dumps({args.only: fn(pkg)}), flush=True)
        return
    torch.manual_seed(0)
    torch.cuda.manual_seed(0)
    cfg = pkg.engine.Qwen2Config(num_hidden_layers=args.layers)
    model = pkg.engine.random_qwen2(cfg, dev, seed=0)
    model.keep_all = args.policy == "keep"
    trainer = Trainer(model)
    n_batches = max(CURVE_STEPS, args.warmup + args.steps) + 1
    batches = make_batches(n_batches, cfg.vocab_size, device=dev)
    log("model built")
    if args.profile:
        args.no_cpu, args.no_configs, args.keep_steps = True, True, 0
    cpu_model = None
    if not args.no_cpu:
        from oracle import step as OS
        cpu_model = OS.CpuQwen2(model)  # the init's weights, before any optimizer step
    first = first_step(model, batches[0])
    log(f"first step loss {first['loss']:.5f}; warmup {args.warmup}")
    _, _, warm_losses = time_steps(trainer, batches, 0, args.warmup)
    log("timing")
    tokens, elapsed, timed_losses = time_steps(trainer, batches, args.warmup, args.steps)
    value = tokens / elapsed
    log(f"{args.steps} steps {elapsed:.3f} s, {value:.0f} tokens/s")
    done = args.warmup + args.steps
    rest = []
    if not args.profile:
        _, _, rest = time_steps(trainer, batches, done, max(0, CURVE_STEPS - done))
    curve = (warm_losses + timed_losses + rest)[:CURVE_STEPS]
    kernels = measure_step_kernels(pkg, trainer, batches[-4:], cfg)
    full = None
    if args.keep_steps > 0 and args.policy != "keep":
        model.keep_gu = model.keep_attn = model.keep_weights_recompute = False
        model.keep_bits = model.keep_lora_x = False
        time_steps(trainer, batches, 0, 2)
        ftok, fel, _ = time_steps(trainer, batches, args.warmup, args.keep_steps)
        full = {"value": ftok / fel, "ms_per_step": 1000.0 * fel / args.keep_steps,
                "steps": args.keep_steps,
                "what": "every layer recomputes its whole forward from its input in backward "
                        "(the [gate|up] product, the attention tensors and the dequantized "
                        "weights formed again)"}
        model.keep_gu = model.keep_attn = model.keep_weights_recompute = True
        model.keep_bits = model.keep_lora_x = True
        log(f"full recompute: {full['value']:.0f} tokens/s")
    keep = None
    if args.keep_steps > 0 and args.policy != "keep":
        model.keep_all = True
        time_steps(trainer, batches, 0, 2)
        ktok, kel, _ = time_steps(trainer, batches, args.warmup, args.keep_steps)
        keep = {"value": ktok / kel, "ms_per_step": 1000.0 * kel / args.keep_steps,
                "steps": args.keep_steps,
                "what": "every layer keeps its intermediates and dequantized weights for the "
                        "backward (no recompute): not config 5, reported beside it"}
        model.keep_all = args.policy == "keep"
        log(f"keep-all: {keep['value']:.0f} tokens/s")
    graph = None
    if not args.profile:
        graph = graph_leg(pkg, trainer, batches[args.warmup:])
        log(f"graph: {graph['tokens_per_s_graph']:.0f} tokens/s replayed, "
            f"{graph['tokens_per_s_eager_padded']:.0f} eager padded")
    result = {
        "metric": "train tokens/s (1.5B NF4 QLoRA step, 1 GPU); NF4 dequant HBM GB/s",
        "value": value, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": 1000.0 * elapsed / args.steps,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (random token ids, random-init Qwen2.5-1.5B NF4 weights)",
        "config": {"workload": "config 5: full Qwen2.5-1.5B NF4+LoRA training step",
                   "batch": "4 packed sequences, lengths U[256,1024]",
                   "tokens": tokens, "layers": args.layers, "parallelism": "single GPU",
                   "activations": ("per-layer recompute as the reference's step does it: each "
                                   "layer keeps its input, its [gate|up] product and its "
                                   "attention's q, k, v, output and o_proj output (the "
                                   "reference's GuStream/AttnStream, in HBM here) and "
                                   "recomputes the two RMSNorms and the LoRA inputs' products "
                                   "in backward; its dequantized fp16 weights stay resident "
                                   "from the forward to the backward (2.6 GB in all) instead "
                                   "of a second dequant"
                                   if args.policy == "recompute" else
                                   "every layer keeps its intermediates (no recompute)"),
                   "gemm": ("the package's MFMA GEMM (qlora_gemm16, fixed tile/split plan) "
                            "after the layer-wide NF4 dequant" if pkg.linear.BACKEND == "dequant"
                            else "the package's NF4-decoding MFMA GEMM (qlora_nf4_gemm)")},
        "roofline": kernels[0],
        "roofline_dequant": kernels[1],
        "roofline_mfma": kernels[2],
        "loss_curve": curve,
        "full_recompute": full,
        "keep_all": keep,
        "graph": graph,
    }
    if not args.no_configs:
        for name, fn in (("config1", config1), ("config2", config2), ("config3", config3),
                         ("config4", config4)):
            log(name)
            result[name] = fn(pkg)
    if cpu_model is not None:
        log("cpu baseline: the oracle's full step")
        result["cpu_baseline"] = cpu_step(pkg, model, cpu_model, batches[0], first)
        if first["metadata_ok"] is not None:
            result["cpu_baseline"]["parity"]["packing_metadata_ok"] = first["metadata_ok"]
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
