"""The trainer drop-in's host logic (the reference's patch.py:268-398) against a stand-in engine
on the CPU: when the fused step runs and when the original compute_loss does, the loss
normaliser, the UnsupportedBatch fallback, the metrics and their deferred recording."""

import types

import pytest
import torch


class _Packed:
    def __init__(self, n, targets, rows, T):
        self.n, self.targets, self.rows, self.T = n, targets, rows, T
        self.tok = torch.arange(n)

    @property
    def row_of_token(self):
        return self.tok // self.T


class _Stats:
    pass


class _Engine:
    """Returns a loss that records the denominator it was given; raises UnsupportedBatch on
    request."""

    def __init__(self, pkg, fail=False):
        self.pkg, self.fail, self.calls = pkg, fail, []

    def step(self, ids, mask, labels, denom):
        if self.fail:
            raise self.pkg.engine.UnsupportedBatch("left padding")
        self.calls.append(denom)
        B, T = ids.shape
        n = int(mask.sum())
        # each real token's next-token label (-100 past the row's end), as the packing forms it
        nxt = torch.cat([labels[:, 1:], torch.full((B, 1), -100)], dim=1)
        targets = nxt[mask.bool()]
        packed = _Packed(n, targets, B, T)
        stats = _Stats()
        stats.entropy = torch.full((n,), 2.0)
        # the head's supervised-first order, its per-token losses 1, 2, ... in that order
        stats.order = torch.argsort(targets.lt(0).to(torch.int8), stable=True)
        stats.correct = torch.tensor([1, 0, 1, 1, 0, 0][:n], dtype=torch.int32)
        stats.tok_loss = torch.arange(1, n + 1, dtype=torch.float32) * \
            targets.index_select(0, stats.order).ge(0)
        loss = torch.tensor(3.0, requires_grad=True) * 1.0
        return loss, packed, stats


class _Trainer:
    def __init__(self):
        self.compute_loss_func = None
        self.label_smoother = None
        self.model_accepts_loss_kwargs = False
        self.args = types.SimpleNamespace(average_tokens_across_devices=False, n_gpu=1)
        self._metrics = {"train": {"entropy": [], "mean_token_accuracy": []}}
        self.callbacks = []
        self.original_calls = 0

    def compute_loss(self, model, inputs, return_outputs=False, num_items_in_batch=None):
        self.original_calls += 1
        return torch.tensor(-1.0)

    def add_callback(self, cb):
        self.callbacks.append(cb)


def _batch():
    ids = torch.tensor([[5, 6, 7, 8], [9, 10, 0, 0]])
    mask = torch.tensor([[1, 1, 1, 1], [1, 1, 0, 0]])
    labels = torch.tensor([[-100, 6, 7, 8], [-100, 10, -100, -100]])
    return {"input_ids": ids, "attention_mask": mask, "labels": labels}


def _install(pkg, engine):
    tr = _Trainer()
    assert pkg.trainer.install(tr, engine=engine)
    assert pkg.trainer.install(tr, engine=engine)  # idempotent
    assert len(tr.callbacks) == 1
    return tr


def test_fused_step_runs_and_normalises_like_hf(pkg):
    eng = _Engine(pkg)
    tr = _install(pkg, eng)
    model = types.SimpleNamespace(training=True)
    loss = tr.compute_loss(model, _batch())
    assert float(loss) == 3.0 and tr.original_calls == 0
    assert eng.calls == [4.0]  # supervised shifted labels: 6, 7, 8 and 10
    tr.model_accepts_loss_kwargs = True
    tr.compute_loss(model, _batch(), num_items_in_batch=torch.tensor(11))
    assert eng.calls[-1] == 11.0
    tr.compute_loss(model, _batch(), num_items_in_batch=None)
    assert eng.calls[-1] == 4.0


def test_original_compute_loss_when_not_usable(pkg):
    eng = _Engine(pkg)
    tr = _install(pkg, eng)
    train = types.SimpleNamespace(training=True)
    b = _batch()
    b["pixel_values"] = torch.zeros(1)
    assert float(tr.compute_loss(train, b)) == -1.0
    assert float(tr.compute_loss(types.SimpleNamespace(training=False), _batch())) == -1.0
    tr.compute_loss_func = lambda *a, **k: None
    assert float(tr.compute_loss(train, _batch())) == -1.0
    assert tr.original_calls == 3 and eng.calls == []


def test_unsupported_batch_falls_back_with_inputs_intact(pkg):
    tr = _install(pkg, _Engine(pkg, fail=True))
    b = _batch()
    b["_prediction_loss_only"] = True
    assert float(tr.compute_loss(types.SimpleNamespace(training=True), b)) == -1.0
    assert tr.original_calls == 1 and "_prediction_loss_only" in b


def test_metrics_recorded_after_backward_is_queued(pkg):
    tr = _install(pkg, _Engine(pkg))
    model = types.SimpleNamespace(training=True)
    tr.compute_loss(model, _batch())
    m = tr._metrics["train"]
    assert m["num_tokens"] == [6] and m["entropy"] == []  # deferred
    assert list(m) == ["entropy", "mean_token_accuracy", "num_tokens"]  # TRL's key order
    tr.callbacks[0].on_pre_optimizer_step(None, None, None)
    assert m["entropy"] == [2.0]
    # targets 6, 7, 8, -, 10, -: 4 supervised tokens, 3 of them right
    assert m["mean_token_accuracy"] == [pytest.approx(3 / 4)]
    tr.compute_loss(model, _batch())  # the next micro-batch flushes nothing new by itself
    assert m["num_tokens"] == [12] and len(m["entropy"]) == 1
    tr.callbacks[0].on_step_end(None, None, None)
    assert len(m["entropy"]) == 2
    tr.callbacks[0].on_step_end(None, None, None)  # nothing pending: no new entry
    assert len(m["entropy"]) == 2


def test_average_tokens_across_devices_scales_the_loss(pkg):
    tr = _install(pkg, _Engine(pkg))
    tr.model_accepts_loss_kwargs = True
    tr.args.average_tokens_across_devices = True
    tr.accelerator = types.SimpleNamespace(num_processes=4, parallelism_config=None)
    loss = tr.compute_loss(types.SimpleNamespace(training=True), _batch(), num_items_in_batch=8)
    assert float(loss) == 12.0


def test_row_losses(pkg):
    eng = _Engine(pkg)
    b = _batch()
    loss, packed, stats = eng.step(b["input_ids"], b["attention_mask"], b["labels"], 1.0)
    means, counts = pkg.trainer.row_losses(packed, stats)
    assert counts == [3, 1]  # supervised tokens of each row (its shifted labels)
    # head order: tokens 0, 1, 2, 4 (supervised), then 3, 5; losses 1, 2, 3, 4 then 0, 0
    assert means == pytest.approx([(1 + 2 + 3) / 3, 4.0])


def test_refusal_reasons_and_untouched_inputs(pkg):
    eng = _Engine(pkg)
    tr = _install(pkg, eng)
    fused = pkg.trainer.installed(tr)
    b = _batch()
    b["pixel_values"] = torch.zeros(1)
    tr.compute_loss(types.SimpleNamespace(training=True), b)
    assert "pixel_values" in fused.last_refusal and "pixel_values" in b
    b = _batch()
    b["_prediction_loss_only"] = False
    tr.compute_loss(types.SimpleNamespace(training=True), b)  # a passive key: fused step
    assert fused.last_refusal is None and b["_prediction_loss_only"] is False
    tr.label_smoother = object()
    tr.compute_loss(types.SimpleNamespace(training=True), _batch())
    assert fused.last_refusal == "the trainer smooths labels"
    assert len(eng.calls) == 1


def _fake_peft(r=16, HQ=12, HKV=2, D=128, H=1536):
    """The attribute paths engine.from_peft reads before it touches any weight (CPU tensors)."""
    NS = types.SimpleNamespace

    def proj(lora):
        m = NS(base_layer=NS(weight=None, bias=None))
        if lora:
            m.lora_A = {"default": NS(weight=torch.zeros(r, H))}
            m.lora_B = {"default": NS(weight=torch.zeros(HQ * D, r))}
            m.scaling = {"default": 2.0}
            m.lora_dropout = {"default": NS(p=0.05)}
            m.active_adapter = ["default"]
        return m

    layer = NS(self_attn=NS(q_proj=proj(True), k_proj=proj(False), v_proj=proj(True),
                            o_proj=proj(False)),
               mlp=NS(gate_proj=proj(False), up_proj=proj(False), down_proj=proj(False)),
               input_layernorm=NS(weight=None, variance_epsilon=1e-6),
               post_attention_layernorm=NS(weight=None, variance_epsilon=1e-6))
    config = NS(hidden_size=H, intermediate_size=4 * H, num_attention_heads=HQ,
                num_key_value_heads=HKV, head_dim=D, vocab_size=1024, rope_theta=1e6)
    causal = NS(model=NS(layers=[layer]), config=config)
    return NS(get_base_model=lambda: causal)


@pytest.mark.parametrize("kw", [{"r": 12}, {"r": 128}, {"HQ": 18, "HKV": 2},
                                {"HQ": 12, "HKV": 5}, {"D": 96}])
def test_from_peft_rejects_what_the_kernels_do_not_take(pkg, kw):
    """A LoRA rank outside 8/16/32/64, more than 8 q heads per kv head, head counts that do not
    divide, head_dim other than 64/128: UnsupportedModel (install then leaves the trainer on
    its own compute_loss) before any weight is read."""
    with pytest.raises(pkg.engine.UnsupportedModel):
        pkg.engine.from_peft(_fake_peft(**kw))
