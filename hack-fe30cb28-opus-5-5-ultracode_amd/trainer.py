"""Hugging Face Trainer / TRL SFTTrainer drop-in: `trainer.compute_loss` served by the fused step.

Reference interface: solution/patch.py:268-347 (`fused_compute_loss`), 349-378 (its metric
flush) and 452-503 (`install`); the host offload and the Soup-specific patches there have no
counterpart (everything stays resident on one GPU).

`install(trainer)` builds the step over the trainer's PEFT 4-bit Qwen2 (`engine.from_peft`) and
puts a `FusedLoss` in place of `trainer.compute_loss`. A call goes to the fused step when the
batch is exactly the causal-LM triple (input_ids, attention_mask, labels), the model is in
training mode and the trainer uses its built-in loss (no `compute_loss_func`, no label
smoother); otherwise, and when the engine raises `UnsupportedBatch` (before it changed
anything), the trainer's own `compute_loss` gets the call with the inputs untouched.
`FusedLoss.last_refusal` names the reason of the last hand-back.

Loss normalisation is Hugging Face's (an interface, kept): the summed token loss divided by
`num_items_in_batch` when the model accepts loss kwargs and the trainer passed it, else by the
batch's supervised shifted labels; under `average_tokens_across_devices` the loss is multiplied
by the data-parallel degree, as Trainer.compute_loss does.

TRL's metrics (an interface, kept: `entropy` averaged over the packed tokens,
`mean_token_accuracy` over the supervised ones, the running `num_tokens`) are gathered without
stalling the GPU: each step's three sums are reduced on the device and copied into pinned host
memory behind an event, right after the forward is queued; `MetricsQueue.drain` waits for that
event only (not for the device) once backward is queued (callback `on_pre_optimizer_step`, or
`on_step_end` when no optimizer step ran), which is still before the optimizer step and the
log."""

import torch

from . import engine as E

BATCH_KEYS = ("input_ids", "attention_mask", "labels")
# keys Trainer may add to a training batch that the fused step does not read
PASSIVE_KEYS = frozenset({"_prediction_loss_only"})
_ATTR = "_qlora_fused_loss"  # the installed FusedLoss, on the trainer


def loss_denominator(trainer, labels, num_items_in_batch):
    """The divisor of the summed token loss, as Hugging Face's Trainer picks it: the count the
    trainer passes when the model takes loss kwargs, else the supervised shifted labels."""
    if num_items_in_batch is not None and getattr(trainer, "model_accepts_loss_kwargs", False):
        n = num_items_in_batch
    else:
        n = labels[..., 1:].ne(-100).sum()
    return float(n)


def device_average_factor(trainer, num_items_in_batch):
    """What Trainer multiplies the loss by under `average_tokens_across_devices` (the
    num_items_in_batch it divided by counts every data-parallel rank's tokens): the GPU count
    of a DataParallel run, else the processes over the tensor-parallel degree; 1 otherwise."""
    args = getattr(trainer, "args", None)
    if not (getattr(args, "average_tokens_across_devices", False)
            and getattr(trainer, "model_accepts_loss_kwargs", False)
            and num_items_in_batch is not None):
        return 1
    n_gpu = getattr(args, "n_gpu", 1)
    if n_gpu > 1:
        return n_gpu
    accel = getattr(trainer, "accelerator", None)
    procs = getattr(accel, "num_processes", 1)
    tp = getattr(getattr(accel, "parallelism_config", None), "tp_size", 1)
    return procs // tp


class MetricsQueue:
    """Per-step metric sums on their way from the device to the trainer's `_metrics`."""

    def __init__(self):
        self.pending = []  # (host or device tensor [3], event or None, packed token count)

    def push(self, packed, stats):
        """Queue the sums of one step: entropy over every packed token, correct predictions and
        supervised tokens (targets >= 0)."""
        with torch.no_grad():
            supervised = packed.targets.ge(0)
            sums = torch.stack([stats.entropy.float().sum(),
                                stats.correct.float().sum(),
                                supervised.float().sum()])
            event = None
            if sums.is_cuda:
                host = torch.empty((3,), dtype=torch.float32, pin_memory=True)
                host.copy_(sums, non_blocking=True)
                event = torch.cuda.Event()
                event.record()
                sums = host
        self.pending.append((sums, event, int(packed.n)))

    def drain(self, metrics):
        """Append every queued step's entropy and accuracy to `metrics` (TRL's train dict)."""
        while self.pending:
            sums, event, n_tok = self.pending.pop(0)
            if event is not None:
                event.synchronize()
            ent, right, sup = (float(x) for x in sums.tolist())
            metrics["entropy"].append(ent / n_tok if n_tok else 0.0)
            metrics["mean_token_accuracy"].append(right / sup if sup else 0.0)


class FusedLoss:
    """The callable installed as `trainer.compute_loss`."""

    def __init__(self, trainer, engine, original):
        self.trainer, self.engine, self.original = trainer, engine, original
        self.queue = MetricsQueue()
        self.last_refusal = None

    def refusal(self, model, inputs):
        """Why the fused step does not take this call (None: it does)."""
        t = self.trainer
        if not getattr(model, "training", False):
            return "the model is not in training mode"
        if not isinstance(inputs, dict):
            return "the inputs are not a dict"
        keys = set(inputs) - PASSIVE_KEYS
        if keys != set(BATCH_KEYS):
            return f"batch keys {sorted(keys)} are not {list(BATCH_KEYS)}"
        if getattr(t, "compute_loss_func", None) is not None:
            return "the trainer has a custom loss function"
        if getattr(t, "label_smoother", None) is not None:
            return "the trainer smooths labels"
        return None

    def _hand_back(self, reason, model, inputs, return_outputs, num_items_in_batch):
        self.last_refusal = reason
        return self.original(model, inputs, return_outputs=return_outputs,
                             num_items_in_batch=num_items_in_batch)

    def __call__(self, model, inputs, return_outputs=False, num_items_in_batch=None):
        reason = self.refusal(model, inputs)
        if reason is not None:
            return self._hand_back(reason, model, inputs, return_outputs, num_items_in_batch)
        ids, mask, labels = (inputs[k] for k in BATCH_KEYS)
        denom = loss_denominator(self.trainer, labels, num_items_in_batch)
        try:
            loss, packed, stats = self.engine.step(ids, mask, labels, denom)
        except E.UnsupportedBatch as exc:  # raised before the step changed anything
            return self._hand_back(str(exc), model, inputs, return_outputs, num_items_in_batch)
        self.last_refusal = None
        factor = device_average_factor(self.trainer, num_items_in_batch)
        if factor != 1:
            loss = loss * factor
        self._record(packed, stats)
        if return_outputs:
            from transformers.modeling_outputs import CausalLMOutputWithPast
            return loss, CausalLMOutputWithPast(loss=loss, logits=None)
        return loss

    def _record(self, packed, stats):
        metrics = getattr(self.trainer, "_metrics", None)
        if metrics is None:
            return
        train = metrics["train"]
        self.flush()  # an earlier micro-batch of this optimizer step (gradient accumulation)
        for key in ("entropy", "mean_token_accuracy"):  # TRL's key order in the log
            train.setdefault(key, [])
        # TRL's running count of trained tokens lives on the trainer (its own compute_loss adds
        # to it too, on the calls handed back)
        total = getattr(self.trainer, "_total_train_tokens", 0) + int(packed.n)
        self.trainer._total_train_tokens = total
        train["num_tokens"] = [total]
        self.queue.push(packed, stats)

    def flush(self):
        """Record the queued steps' entropy and accuracy in the trainer's metrics."""
        metrics = getattr(self.trainer, "_metrics", None)
        if metrics is not None:
            self.queue.drain(metrics["train"])


def row_losses(packed, stats):
    """Each batch row's mean token loss over its supervised tokens, and those tokens' counts
    (what the reference's rewind recorder takes, patch.py:372-378), from the packed targets:
    the head's per-token losses (in its supervised-first order `stats.order`) summed by row."""
    with torch.no_grad():
        rows = packed.row_of_token.index_select(0, stats.order)
        sums = torch.bincount(rows, weights=stats.tok_loss.double(), minlength=packed.rows)
        sup = packed.targets.index_select(0, stats.order).ge(0)
        counts = torch.bincount(rows[sup], minlength=packed.rows)
        means = sums / counts.clamp(min=1).double()
    return [float(x) for x in means.tolist()], [int(x) for x in counts.tolist()]


def _callback_base():
    try:
        from transformers import TrainerCallback
        return TrainerCallback
    except Exception:  # transformers absent: a plain base with the hooks
        return object


class FlushMetrics(_callback_base()):
    """Moves the queued metrics into the trainer's log once backward is queued."""

    def __init__(self, fused):
        self.fused = fused

    def on_pre_optimizer_step(self, args, state, control, **kwargs):
        self.fused.flush()

    def on_step_end(self, args, state, control, **kwargs):  # a step without an optimizer step
        self.fused.flush()


def install(trainer, engine=None):
    """Put the fused step in place of `trainer.compute_loss`. True when installed (now or
    before), False when the model is not one the step supports (the trainer is left as it
    was)."""
    if getattr(trainer, _ATTR, None) is not None:
        return True
    if engine is None:
        try:
            engine = E.from_peft(trainer.model)
        except E.UnsupportedModel:
            return False
    fused = FusedLoss(trainer, engine, trainer.compute_loss)
    setattr(trainer, _ATTR, fused)
    trainer.compute_loss = fused
    if hasattr(trainer, "add_callback"):
        trainer.add_callback(FlushMetrics(fused))
    return True


def installed(trainer):
    """The trainer's FusedLoss, or None."""
    return getattr(trainer, _ATTR, None)


__all__ = ["BATCH_KEYS", "FusedLoss", "FlushMetrics", "MetricsQueue", "device_average_factor",
           "install", "installed", "loss_denominator", "row_losses"]
