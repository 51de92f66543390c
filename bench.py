"""Benchmark: full Qwen2.5-1.5B NF4 + LoRA training steps on one MI355X.

A step = forward + backward (intermediates kept per the reference's memory-cap plan, or
recomputed) + fp16 loss scaling (GradScaler) + fused AdamW on the LoRA parameters, over one synthetic batch of 4 packed sequences with lengths ~ U[256, 1024]
and random token ids (first 25% of each sequence unsupervised). Random-init weights of the
Qwen2.5-1.5B architecture, all linears NF4 double-quant (blocksize 64), tied fp16 embedding.

Prints ONE JSON line: value = tokens/s over the K timed steps (inputs resident in HBM), plus
  roofline      the dominant hand-written kernel, achieved vs MI355X peak, measured with HIP
                events around each of its launches in one extra (untimed) step
  cpu_baseline  the CPU oracle step (oracle.step, plain PyTorch fp32 autograd) on this host's
                cores, on a bounded sample (embedding + 2 layers + head, and the head alone),
                scaled to a 28-layer step

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--policy plan|recompute|keep]
"""

import argparse
import importlib
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
PKG_NAME = "hack-fe30cb28-opus-5-5-ultracode_amd"

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0


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


def measure_kernel(pkg, trainer, batch, which):
    """Average duration and algorithmic work of every launch of the dominant kernel in one step,
    from HIP events recorded on the launch stream around each launch."""
    timer = pkg.profiling.LaunchTimer(which)
    with timer:
        trainer.step(batch)
    torch.cuda.synchronize()
    return timer.summary()


def config1(pkg, copies=64, reps=20):
    """BASELINE config 1 on the GPU: NF4 double-quant dequant of one Qwen2.5-1.5B q_proj weight
    [1536, 1536] (N(0, 0.02) from seed 1, bitsandbytes layout), rotating over `copies`
    independent copies (> 256 MB of Infinity Cache per pass), and the same for the four weights
    of a layer in one launch (qkv | o | gate-up | down, the step's dequant). Beside them a plain
    device copy of the q_proj output size: the calibration kernel for the FETCH_SIZE /
    WRITE_SIZE counter runs. Returns a dict of achieved GB/s (algorithmic bytes / event time)."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(1)

    def weight(shape):
        w = (torch.randn(shape, generator=g, device=dev) * 0.02).half()
        return pkg.ops.NF4Weight(pkg.quant.quantize_nf4(w))

    qs = [weight((1536, 1536)) for _ in range(copies)]
    outs = [torch.empty((1536, 1536), device=dev, dtype=torch.float16) for _ in range(copies)]
    per_q = pkg.profiling._dequant_bytes([None] * 7 + [qs[0].blocks, 1, None, 64, 256,
                                                       2**63 - 1, 2**63 - 1])

    def timed(fn, n):
        for i in range(min(n, 4)):
            fn(i)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for i in range(n):
            fn(i)
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) * 1e-3 / n

    t_q = timed(lambda i: qs[i % copies].dequant_into(outs[i % copies]), copies * reps)
    layers = []
    for i in range(8):
        grp = lambda shapes: pkg.ops.NF4Group.of([weight(sh) for sh in shapes])  # noqa: E731
        layers.append([grp([(1536, 1536), (256, 1536), (256, 1536)]), weight((1536, 1536)),
                       grp([(8960, 1536), (8960, 1536)]), weight((1536, 8960))])
    per_layer = sum(pkg.profiling._dequant_bytes(
        [None] * 7 + [w.blocks, 1, None, 64, 256, getattr(w, "seg1", 2**63 - 1),
                      getattr(w, "seg2", 2**63 - 1)]) for w in layers[0])
    t_l = timed(lambda i: pkg.ops.dequant_many(layers[i % 8], dev), 8 * reps)
    src = torch.empty(1536 * 1536, device=dev, dtype=torch.float16).normal_()
    dst = torch.empty_like(src)
    t_c = timed(lambda i: dst.copy_(src), copies * reps)
    return {"q_proj_dequant_GBs": per_q / t_q / 1e9, "q_proj_bytes": per_q,
            "q_proj_us": t_q * 1e6, "layer_dequant_GBs": per_layer / t_l / 1e9,
            "layer_bytes": per_layer, "layer_us": t_l * 1e6,
            "copy_GBs": 2 * src.numel() * 2 / t_c / 1e9, "copies": copies}


def config4(pkg, reps=3):
    """BASELINE config 4 on the GPU: LM head loss over hidden [2048, 1536] (N(0, 1)) and the
    tied embedding [151936, 1536] (N(0, 0.02)), ~25 % of the labels ignored, with the hidden and
    embedding gradients: vocabulary pieces of 8192 (online softmax, head.chunked_head: logits,
    the dh accumulation, recomputed logits, dE; 4 products of 2 T V H flops) and whole rows
    (head.full_head: logits, G E, G^T h; 3 products)."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(4)
    T, V, H = 2048, 151936, 1536
    hn = torch.randn(T, H, generator=g, device=dev).half()
    E = (torch.randn(V, H, generator=g, device=dev) * 0.02).half()
    targets = torch.randint(0, V, (T,), generator=g, device=dev)
    targets[torch.rand(T, generator=g, device=dev) < 0.25] = -100
    denom = float((targets >= 0).sum())
    out = {}
    for name, fn, products in (("pieces", pkg.head.chunked_head, 4),
                               ("whole_rows", pkg.head.full_head, 3)):
        fn(hn, E, targets, denom)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            r = fn(hn, E, targets, denom)
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / reps
        flops = products * 2.0 * T * V * H
        out[name] = {"ms": dt * 1e3, "TFLOPs": flops / dt / 1e12, "loss": float(r.loss)}
    return out


def cpu_baseline(pkg, model, batch):
    """The CPU oracle step on a bounded sample: forward + autograd backward of embedding +
    2 layers + head, and of the head alone; a 28-layer step is head + 28 x layer."""
    from oracle import step as OS

    ids, mask, labels, denom, ntok, _ = batch
    threads = torch.get_num_threads()
    L = len(model.layers)
    gen = model.dropout.gen
    seed, offset = gen.initial_seed(), gen.get_offset()
    G = model.dropout.max_blocks * 256
    cpu2 = OS.CpuQwen2(model, layers=[0, 1])
    t0 = time.perf_counter()
    loss, _ = OS.forward_loss(cpu2, ids, mask, labels, denom, drop_seed=seed,
                              drop_offset=offset, drop_G=G, p=model.dropout_p, vec=4)
    loss.backward()
    t_two = time.perf_counter() - t0
    cpu0 = OS.CpuQwen2(model, layers=[])
    n = int(mask.sum())
    h = torch.randn(n, model.cfg.hidden_size, requires_grad=True)
    t0 = time.perf_counter()
    loss0, _ = OS.forward_loss(cpu0, ids, mask, labels, denom, first_layer_input=h)
    loss0.backward()
    t_head = time.perf_counter() - t0
    t_layer = max(t_two - t_head, 1e-9) / 2
    t_step = t_head + L * t_layer
    return {"value": ntok / t_step, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": (f"oracle.step (torch fp32 autograd) on {ntok} tokens: embedding + 2 of "
                       f"{L} layers + head fwd+bwd {t_two:.2f} s, head alone {t_head:.2f} s; "
                       f"step = head + {L} x layer = {t_step:.2f} s"),
            "cpu": _cpu_model()}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--policy", choices=("plan", "recompute", "keep"), default="plan",
                    help="which layers keep their intermediates for the backward: the "
                         "reference's memory-cap plan under this GPU's memory (default; every "
                         "layer keeps them on 288 GB), none (full per-layer recompute) or all")
    ap.add_argument("--recompute-steps", type=int, default=10,
                    help="also time this many steps with full per-layer recompute (0: skip)")
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--config1", action="store_true",
                    help="only the config-1 dequant measurement (and its copy calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus}: this build measures one GPU only (the path is "
              "data-parallel; multi-GPU runs are out of scope)", file=sys.stderr)
        sys.exit(2)
    pkg = importlib.import_module(PKG_NAME)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.config1:
        print(json.dumps({"config1": config1(pkg)}), flush=True)
        return
    torch.manual_seed(0)
    torch.cuda.manual_seed(0)
    cfg = pkg.engine.Qwen2Config(num_hidden_layers=args.layers)
    model = pkg.engine.random_qwen2(cfg, dev, seed=0)
    model.keep_all = {"plan": None, "recompute": False, "keep": True}[args.policy]
    trainer = Trainer(model)
    batches = make_batches(args.warmup + args.steps + 1, cfg.vocab_size, device=dev)
    print("[bench] model built; timing the projection GEMM solutions", file=sys.stderr,
          flush=True)
    # every step size config 5 can produce (4 rows of 256..1024 tokens), before any timing
    tune_s = model.tune_gemms(range(4 * 256, 4 * 1024 + pkg.gemm.BUCKET, pkg.gemm.BUCKET),
                              log=lambda m: print("[bench] " + m, file=sys.stderr, flush=True))
    print(f"[bench] GEMM tuning {tune_s:.1f} s; warmup {args.warmup}", file=sys.stderr,
          flush=True)
    for i in range(args.warmup):
        trainer.step(batches[i])
    torch.cuda.synchronize()
    print("[bench] timing", file=sys.stderr, flush=True)
    tokens = 0
    losses = []
    t0 = time.perf_counter()
    for i in range(args.warmup, args.warmup + args.steps):
        losses.append(trainer.step(batches[i]).detach())
        tokens += batches[i][4]
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    losses = [float(x) for x in losses]
    value = tokens / elapsed
    print(f"[bench] {args.steps} steps {elapsed:.3f} s, {value:.0f} tokens/s", file=sys.stderr,
          flush=True)
    kept = model.keep_plan(batches[-1][4])
    recompute = None
    if args.recompute_steps > 0 and model.keep_all is not False:
        # the same step with every layer recomputing its forward in backward
        saved, model.keep_all = model.keep_all, False
        for i in range(2):
            trainer.step(batches[i])
        torch.cuda.synchronize()
        rtok, t1 = 0, time.perf_counter()
        for i in range(args.recompute_steps):
            b = batches[(args.warmup + i) % (len(batches) - 1)]
            trainer.step(b)
            rtok += b[4]
        torch.cuda.synchronize()
        rel = time.perf_counter() - t1
        recompute = {"value": rtok / rel, "ms_per_step": 1000.0 * rel / args.recompute_steps,
                     "steps": args.recompute_steps}
        model.keep_all = saved
        print(f"[bench] full recompute: {recompute['value']:.0f} tokens/s", file=sys.stderr,
              flush=True)
    roof = measure_kernel(pkg, trainer, batches[-1], pkg.profiling.DOMINANT)
    result = {
        "metric": "train tokens/s (1.5B NF4 QLoRA step, 1 GPU); NF4 dequant HBM GB/s",
        "value": value, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": 1000.0 * elapsed / args.steps,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (random token ids, random-init Qwen2.5-1.5B NF4 weights)",
        "config": {"workload": "config 5: full Qwen2.5-1.5B NF4+LoRA training step",
                   "batch": "4 packed sequences, lengths U[256,1024]",
                   "tokens": tokens, "layers": args.layers, "parallelism": "single GPU",
                   "activations": (f"kept for the backward by {kept} of {args.layers} layers "
                                   "(the reference's memory-cap plan, engine.py:1626-1640, "
                                   "under this GPU's memory), with their dequantized weights "
                                   "(each NF4 weight dequantized once per step); the others "
                                   "recompute their forward")},
        "gemm_tuning_s": tune_s,
        "full_recompute": recompute,
        "loss_first_last": [losses[0], losses[-1]],
        "roofline": roof,
        "config1": config1(pkg),
        "config4": config4(pkg),
    }
    if not args.no_cpu:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(pkg, model, batches[-1])
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
