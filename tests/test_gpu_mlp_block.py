"""The MLP half of the decoder layer as one node (talm_amd/mlp_block.py) against the separate
nodes it replaces (NormNode + FusedMLP + NormNode).

- The fused launches: talm_splitk_add_rmsnorm on a split-K product's partials equals the
  product's own reduction followed by talm_rmsnorm's add forward, and talm_splitk_rmsnorm_bwd
  equals the reduction followed by its add backward (with and without the sum's gradient), bit
  for bit, for several part counts; the partials of talm_gemm_splitk_partials sum in part order
  to talm_gemm_splitk's output.
- The model: a small QLoRA model's loss and LoRA gradients with the block on and off are the
  same bits (the block runs on every layer, nothing falls back), and a few training steps of the
  graphed step track the eager curve.
"""

import pytest
import torch

from talm_amd import _ops, engaged, patches, qlora_model, state

pytestmark = pytest.mark.gpu

LAYERS = 3


@pytest.mark.parametrize("m,h,k,w_dtype", [(1367, 1536, 8960, torch.float32),
                                           (300, 512, 4096, torch.float32),
                                           (37, 256, 4096, torch.float16),
                                           (2048, 1536, 17920, torch.float32)])
def test_fused_norm_launches_equal_the_reduction_then_the_norm(m, h, k, w_dtype):
    _ops.load()
    n_parts = _ops.gemm_splitk_parts(m, h, k)
    print(f"[case] splitk norms m={m} h={h} k={k} parts={n_parts}", flush=True)
    g = torch.Generator().manual_seed(m + k)
    a = torch.randn(m, k, generator=g).half().cuda()
    b = (torch.randn(h, k, generator=g) * k ** -0.5).half().cuda()
    part = torch.full((n_parts, m, h), float("nan"), device="cuda")
    torch.ops.talm.gemm_splitk_partials(a, b, part)
    y = torch.empty(m, h, dtype=torch.float16, device="cuda")
    ws = torch.empty(_ops.gemm_splitk_workspace_bytes(m, h, k), dtype=torch.uint8, device="cuda")
    torch.ops.talm.gemm_splitk(a, b, y, ws)
    total = part[0].clone()
    for p in range(1, n_parts):
        total += part[p]
    assert torch.equal(total.half().view(torch.int16), y.view(torch.int16))
    resid = torch.randn(m, h, generator=g).cuda()
    w = (torch.rand(h, generator=g) + 0.5).to(w_dtype).cuda()
    eps = 1e-6
    outs = []
    for fused in (False, True):
        s = torch.empty(m, h, device="cuda")
        hh = torch.empty(m, h, dtype=torch.float16, device="cuda")
        xh = torch.empty_like(hh)
        r = torch.empty(m, device="cuda")
        if fused:
            torch.ops.talm.splitk_add_rmsnorm(part, resid, w, eps, s, hh, xh, r)
        else:
            torch.ops.talm.rmsnorm(resid, s, hh, xh, y, w, r, eps, 0)
        outs.append((s, hh, xh, r))
    for ref, got in zip(*outs):
        assert torch.equal(ref, got)
    _s, _h, xhat, rstd = outs[0]
    ds = torch.randn(m, h, generator=g).cuda()
    for with_ds in (True, False):
        grads = []
        for fused in (False, True):
            dx = torch.empty(m, h, device="cuda")
            db = torch.empty(m, h, dtype=torch.float16, device="cuda")
            q = ds if with_ds else None
            if fused:
                torch.ops.talm.splitk_rmsnorm_bwd(part, xhat, rstd, w, q, dx, db)
            else:
                torch.ops.talm.rmsnorm(dx, q, y, xhat, db, w, rstd, eps, 1)
            grads.append((dx, db))
        assert torch.equal(grads[0][0], grads[1][0]) and torch.equal(grads[0][1], grads[1][1])


def _model(seed=3):
    config = qlora_model.qwen2_config(vocab_size=1000, hidden_size=512, intermediate_size=4096,
                                      num_hidden_layers=LAYERS, num_attention_heads=4,
                                      num_key_value_heads=2, head_dim=128)
    model = qlora_model.build_model(config, seed=seed)
    with torch.no_grad():
        gen = torch.Generator(device="cuda").manual_seed(9)
        for p in qlora_model.lora_parameters(model):
            if p.abs().sum() == 0:
                p.copy_(0.02 * torch.randn(p.shape, generator=gen, device="cuda"))
    return model


def _forward_backward(model, batch):
    for p in qlora_model.lora_parameters(model):
        p.grad = None
    with torch.autocast("cuda", dtype=torch.float16):
        out = model(input_ids=batch["input_ids"], attention_mask=batch["attention_mask"],
                    labels=batch["labels"])
    out.loss.backward()
    return out.loss.detach().clone(), [p.grad.detach().clone()
                                       for p in qlora_model.lora_parameters(model)]


def test_block_equals_the_separate_nodes_bitwise(monkeypatch):
    print("[case] MLP block vs NormNode + FusedMLP + NormNode, small model", flush=True)
    model = _model()
    batch = qlora_model.make_batch(seed=5, step=0, vocab=1000, seq=256, lo=64, hi=256)
    patches.apply()
    try:
        engaged.reset()
        loss, grads = _forward_backward(model, batch)
        assert engaged.RAN["mlp_block"] == LAYERS and engaged.FELL_BACK["mlp_block"] == 0
        monkeypatch.setitem(state.DISABLED, "mlp_block", "switched off by the test")
        engaged.reset()
        ref_loss, ref_grads = _forward_backward(model, batch)
        assert engaged.RAN["mlp_block"] == 0 and engaged.RAN["fused_mlp"] == LAYERS
    finally:
        patches.unapply()
    assert torch.equal(loss, ref_loss), (float(loss), float(ref_loss))
    for got, want in zip(grads, ref_grads):
        assert torch.equal(got, want)
