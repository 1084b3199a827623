"""The QLoRA step replayed from HIP graphs (step_graph.GraphedTrainer) on a small tied Qwen2
(the parity model of test_gpu_step.py): against the same steps run eagerly with the same
fixed-shape packing (bit-identical losses and LoRA weights: the same kernels on the same shapes
in the same order), and against the eagerly packed patched step (the loss curve within the
north star's 0.5%). The token counts are chosen so that buckets repeat after other buckets ran,
one batch fills its bucket exactly (an empty pad sequence), one leaves a one-row pad sequence
(with 16-token buckets, the bench's default) and one is the largest batch. The per-token metrics
each replay leaves in patches.LAST_STEP must be that replay's, bit for bit."""

import pytest
import torch

from talm_amd import fused_head, patches, qlora_model, unpad
from talm_amd.step_graph import GraphedTrainer

pytestmark = pytest.mark.gpu

SEQ, VOCAB, WARM = 256, 1000, 2
# real tokens per step: eager warm-up, then 640 (no pad rows with 16- and 64-token buckets), 640,
# 300, 630, 1024 (the largest), 310, 607 (a one-row pad sequence with 16-token buckets)
LENGTHS = [(200, 100, 64, 256), (256, 130, 70, 90), (250, 150, 100, 140), (256, 128, 128, 128),
           (64, 100, 70, 66), (256, 200, 90, 84), (256, 256, 256, 256), (64, 64, 64, 118),
           (100, 200, 150, 157)]
BUCKETS = {16: [304, 320, 608, 640, 1024], 64: [320, 640, 1024]}


def _batch(step, lengths):
    g = torch.Generator().manual_seed(11 * 1000 + step)
    lengths = torch.tensor(lengths)
    ids = torch.randint(0, VOCAB, (len(lengths), SEQ), generator=g)
    mask = torch.arange(SEQ)[None, :] < lengths[:, None]
    labels = torch.where(mask, ids, torch.full_like(ids, -100))
    ids = torch.where(mask, ids, torch.zeros_like(ids))
    return {"input_ids": ids.cuda(), "attention_mask": mask.to(torch.int64).cuda(),
            "labels": labels.cuda()}


def _model():
    config = qlora_model.qwen2_config(vocab_size=VOCAB, hidden_size=512, intermediate_size=1024,
                                      num_hidden_layers=3, num_attention_heads=4,
                                      num_key_value_heads=2, head_dim=128)
    model = qlora_model.build_model(config, seed=3)
    with torch.no_grad():
        for p in qlora_model.lora_parameters(model):
            if p.abs().sum() == 0:
                p.normal_(0, 0.02)
    return model


def _metrics():
    m = patches.LAST_STEP[-1]
    return [t.detach().clone() for t in (m.token_loss, m.token_entropy, m.correct, m.labelled,
                                         m.argmax)]


def _penalize(model, weight, coeff=1e-2):
    """The loss plus coeff * |weight|^2 (a second autograd path to one LoRA weight, beside the
    q|k|v node's gradient), through a forward hook on the causal LM."""
    def hook(_module, _args, _kwargs, output):
        output.loss = output.loss + coeff * weight.float().square().sum()
        return output

    return model.register_forward_hook(hook, with_kwargs=True)


def _run(mode, monkeypatch, bucket=64, penalty=False):
    """mode: "graph" (GraphedTrainer), "static" (eager steps under the same fixed-shape packing)
    or "eager" (the patched step with host-list packing). Returns (losses, LoRA weights,
    (replays, buckets, direct gradient delivery) or None, per-step metrics of
    patches.LAST_STEP). penalty: a weight-norm term on one adapter weight in the loss."""
    steps = len(LENGTHS)
    model = _model()
    trainer = qlora_model.Trainer(model, steps=steps, fused_adapters=True)
    if penalty:
        _penalize(model, trainer.params[1])
    patches.apply()
    monkeypatch.setattr(fused_head, "VOCAB_CHUNK", 384)
    gt = GraphedTrainer(trainer, bucket=bucket, warm_steps=WARM) if mode == "graph" else None
    if mode == "static":
        from talm_amd.adapters import COPIES
        monkeypatch.setattr(COPIES, "in_place", True)
    losses, metrics = [], []
    try:
        batches = [_batch(i, lengths) for i, lengths in enumerate(LENGTHS)]
        for i in range(steps):
            ahead = batches[i + 1] if i + 1 < steps else None
            if mode == "graph":
                loss = gt.step(batches[i], ahead)
            elif mode == "static" and i >= WARM:
                nb = -(-sum(LENGTHS[i]) // bucket) * bucket
                with unpad.static_tokens(nb, max_pad=bucket):
                    loss = trainer.step(batches[i], ahead)
            else:
                loss = trainer.step(batches[i], ahead)
            losses.append(float(loss))
            metrics.append(_metrics())
        weights = [p.detach().clone() for p in trainer.params]
        info = None if gt is None else (gt.replays, sorted(gt.graphs), gt.direct_grads)
    finally:
        if gt is not None:
            gt.close()
        patches.unapply()
    del model, trainer, gt
    torch.cuda.empty_cache()
    return losses, weights, info, metrics


@pytest.mark.parametrize("bucket", [16, 64])
def test_graphed_step_matches_eager_static_step_bitwise(monkeypatch, bucket):
    print(f"[case] graphed step vs eager fixed-shape step (bitwise), bucket {bucket}", flush=True)
    ref_losses, ref_weights, _, ref_metrics = _run("static", monkeypatch, bucket)
    losses, weights, (replays, buckets, direct), metrics = _run("graph", monkeypatch, bucket)
    print(f"[graph] losses {losses}\n[static] losses {ref_losses}", flush=True)
    assert replays == len(LENGTHS) - WARM
    assert buckets == BUCKETS[bucket]
    assert direct, "the q|k|v nodes did not write every adapter gradient into its buffer"
    assert losses == ref_losses
    for w, r in zip(weights, ref_weights):
        assert torch.equal(w, r), (w - r).abs().max().item()
    names = ("token_loss", "token_entropy", "correct", "labelled", "argmax")
    for step, (got, ref) in enumerate(zip(metrics, ref_metrics)):
        for name, a, b in zip(names, got, ref):
            assert torch.equal(a, b), f"step {step}: LAST_STEP.{name} differs from the eager step"


def test_graphed_step_matches_eager_loss_curve(monkeypatch):
    print("[case] graphed step vs eager host-packed patched step (curve)", flush=True)
    ref_losses, _, _, _ = _run("eager", monkeypatch)
    losses, _, _, _ = _run("graph", monkeypatch, 16)
    print(f"[graph] losses {losses}\n[eager] losses {ref_losses}", flush=True)
    for a, b in zip(losses, ref_losses):
        assert abs(a - b) <= 5e-3 * abs(b), (losses, ref_losses)


def test_graphed_step_with_a_second_gradient_path_captures_the_general_way(monkeypatch):
    """A penalty on one LoRA weight in the loss reaches that weight through autograd as well as
    through the q|k|v node. Direct delivery would drop or stale-add that term, so the capture
    must notice it and fall back to zeroing and accumulating; the graphed run is then
    bit-identical to the eager fixed-shape run with the same penalty."""
    print("[case] graphed step vs eager fixed-shape step with a penalty on one LoRA weight",
          flush=True)
    ref_losses, ref_weights, _, _ = _run("static", monkeypatch, 16, penalty=True)
    losses, weights, (replays, _buckets, direct), _ = _run("graph", monkeypatch, 16,
                                                            penalty=True)
    print(f"[graph] losses {losses}\n[static] losses {ref_losses}", flush=True)
    assert replays == len(LENGTHS) - WARM
    assert not direct, "the capture kept direct delivery although autograd also fed a weight"
    assert losses == ref_losses
    for w, r in zip(weights, ref_weights):
        assert torch.equal(w, r), (w - r).abs().max().item()
