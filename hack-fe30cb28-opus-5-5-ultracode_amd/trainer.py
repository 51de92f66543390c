"""The trainer drop-in: Hugging Face Trainer / TRL SFTTrainer `compute_loss` replaced by the fused
step (the reference's patch.py:268-398 `fused_compute_loss`, `_flush_metrics`, `install`
452-503, without its host offload and Soup-specific patches).

`install(trainer)` builds the step over the trainer's PEFT 4-bit Qwen2 (`engine.from_peft`) and
swaps `trainer.compute_loss` for `fused_compute_loss`, which

- runs the fused step when the batch is a plain causal-LM batch (input_ids, attention_mask,
  labels) of a model in training mode and the trainer uses its default loss; otherwise, and on
  `UnsupportedBatch` (raised before anything changed), the original `compute_loss` runs;
- normalises the loss as HF does: the sum over the batch divided by `num_items_in_batch` when
  the model accepts loss kwargs, else the mean over supervised tokens; scaled by the number of
  processes under `average_tokens_across_devices`;
- records TRL's metrics (entropy, mean_token_accuracy, num_tokens) without stalling the GPU
  between forward and backward: the token count is a host number, entropy and accuracy are read
  once backward is queued (callback `on_pre_optimizer_step`), still before the optimizer step
  and the log, in TRL's key order.
"""

import types

import torch

from . import engine as E

_ENGINE_ATTR = "_qlora_engine"
_ORIGINAL_ATTR = "_qlora_original_compute_loss"
_PENDING_ATTR = "_qlora_pending_metrics"
BATCH_KEYS = ("input_ids", "attention_mask", "labels")


def _usable(trainer, model, inputs):
    return (getattr(trainer, _ENGINE_ATTR, None) is not None
            and getattr(model, "training", False)
            and isinstance(inputs, dict)
            and set(inputs) <= set(BATCH_KEYS) | {"_prediction_loss_only"}
            and all(k in inputs for k in BATCH_KEYS)
            and getattr(trainer, "compute_loss_func", None) is None
            and getattr(trainer, "label_smoother", None) is None)


def loss_denominator(trainer, labels, num_items_in_batch):
    """HF Trainer's normaliser: num_items_in_batch when the model takes loss kwargs, else the
    number of supervised (shifted) labels of the batch (patch.py:292-297)."""
    if getattr(trainer, "model_accepts_loss_kwargs", False) and num_items_in_batch is not None:
        denom = num_items_in_batch
    else:
        denom = (labels[:, 1:] != -100).sum()
    return float(denom.item() if torch.is_tensor(denom) else denom)


def fused_compute_loss(self, model, inputs, return_outputs=False, num_items_in_batch=None):
    """Trainer.compute_loss with the fused step (patch.py:268-347)."""
    engine = getattr(self, _ENGINE_ATTR, None)
    original = getattr(self, _ORIGINAL_ATTR)
    if not _usable(self, model, inputs):
        return original(model, inputs, return_outputs=return_outputs,
                        num_items_in_batch=num_items_in_batch)
    popped = {k: inputs.pop(k) for k in ("_prediction_loss_only",) if k in inputs}
    input_ids, attention_mask, labels = (inputs[k] for k in BATCH_KEYS)
    denom = loss_denominator(self, labels, num_items_in_batch)
    try:
        loss, packed, stats = engine.step(input_ids, attention_mask, labels, denom)
    except E.UnsupportedBatch:  # e.g. left padding: raised before the step changed anything
        inputs.update(popped)
        return original(model, inputs, return_outputs=return_outputs,
                        num_items_in_batch=num_items_in_batch)
    args = getattr(self, "args", None)
    if getattr(args, "average_tokens_across_devices", False) \
            and getattr(self, "model_accepts_loss_kwargs", False) \
            and num_items_in_batch is not None:
        accel = getattr(self, "accelerator", None)
        scale = getattr(accel, "num_processes", 1)
        pc = getattr(accel, "parallelism_config", None)
        if pc is not None:
            scale //= getattr(pc, "tp_size", 1)
        n_gpu = getattr(args, "n_gpu", 1)
        loss = loss * (scale if n_gpu <= 1 else n_gpu)
    metrics = getattr(self, "_metrics", None)
    if metrics is not None:
        flush_metrics(self)  # a previous micro-batch's, under gradient accumulation
        train = metrics["train"]
        train["entropy"], train["mean_token_accuracy"]  # noqa: B018 - TRL's key order
        self._total_train_tokens = getattr(self, "_total_train_tokens", 0) + int(packed.n)
        train["num_tokens"] = [self._total_train_tokens]
        setattr(self, _PENDING_ATTR, (packed, stats))
    if return_outputs:
        from transformers.modeling_outputs import CausalLMOutputWithPast
        return loss, CausalLMOutputWithPast(loss=loss, logits=None)
    return loss


def step_metrics(packed, stats):
    """(entropy averaged over the packed tokens, accuracy over the supervised ones) of a step,
    as TRL's SFTTrainer computes them from the logits (one device read)."""
    with torch.no_grad():
        valid = packed.targets >= 0
        ent, cor, cnt = torch.stack([stats.entropy.sum(), stats.correct.sum().float(),
                                     valid.sum().float()]).tolist()
    return ent / max(packed.n, 1), (cor / cnt if cnt > 0 else 0.0)


def row_losses(packed, stats, labels):
    """Per-row mean cross-entropy over the row's supervised tokens (the reference's rewind
    rows, patch.py:372-378) and the rows' supervised-token counts."""
    with torch.no_grad():
        totals = torch.zeros(packed.rows, device=stats.tok_loss.device, dtype=torch.float32)
        # tok_loss is in the head's row order (supervised first): stats.order maps it back
        totals.index_add_(0, packed.row_of_token.index_select(0, stats.order), stats.tok_loss)
        counts = (labels[:, 1:] != -100).sum(dim=1)
        means = totals / counts.clamp(min=1).to(totals.dtype)
    return [float(x) for x in means.tolist()], [int(x) for x in counts.tolist()]


def flush_metrics(trainer):
    """Record the queued micro-batch's entropy and accuracy (patch.py:350-370)."""
    pending = getattr(trainer, _PENDING_ATTR, None)
    if pending is None:
        return
    setattr(trainer, _PENDING_ATTR, None)
    entropy, accuracy = step_metrics(*pending)
    trainer._metrics["train"]["entropy"].append(entropy)
    trainer._metrics["train"]["mean_token_accuracy"].append(accuracy)


def _callback_base():
    try:
        from transformers import TrainerCallback
        return TrainerCallback
    except Exception:  # transformers absent: a plain base with the hooks
        return object


class FlushMetrics(_callback_base()):
    """Records the pending metrics once backward is queued, before the optimizer step."""

    def __init__(self, trainer):
        self.trainer = trainer

    def on_pre_optimizer_step(self, args, state, control, **kwargs):
        flush_metrics(self.trainer)

    def on_step_end(self, args, state, control, **kwargs):  # in case no optimizer step ran
        flush_metrics(self.trainer)


def install(trainer, engine=None):
    """Swap `trainer.compute_loss` for the fused step (patch.py:452-503); returns True when
    installed (or already), False when the model is not one the step supports."""
    if getattr(trainer, _ENGINE_ATTR, None) is not None:
        return True
    if engine is None:
        try:
            engine = E.from_peft(trainer.model)
        except E.UnsupportedModel:
            return False
    setattr(trainer, _ORIGINAL_ATTR, trainer.compute_loss)
    setattr(trainer, _ENGINE_ATTR, engine)
    trainer.compute_loss = types.MethodType(fused_compute_loss, trainer)
    if hasattr(trainer, "add_callback"):
        trainer.add_callback(FlushMetrics(trainer))
    return True
