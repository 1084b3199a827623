"""End-to-end parity of the patched QLoRA training step (every kernel of the package engaged)
with the unpatched eager path (transformers' Qwen2 + the 4-bit / LoRA layers' own forwards, the
padded batch, full logits and PyTorch's cross-entropy), on a small tied Qwen2 like the
reference's own parity run (solution/test_parity.py:22-38: vocabulary 1000, hidden 512,
3 layers, 4 query / 2 KV heads of 128, MLP 1024, NF4 double-quant base, LoRA r16/alpha32 on
q/v, fp16 autocast + GradScaler, AdamW). Bars: the loss curve within 0.5% at every step (the
north star), the first step's loss within 1e-3."""

import pytest
import torch

from talm_amd import engaged, fused_head, patches, qlora_model

pytestmark = pytest.mark.gpu


def _run(patched, steps, monkeypatch):
    config = qlora_model.qwen2_config(vocab_size=1000, hidden_size=512, intermediate_size=1024,
                                      num_hidden_layers=3, num_attention_heads=4,
                                      num_key_value_heads=2, head_dim=128)
    model = qlora_model.build_model(config, seed=3)
    # B starts non-zero (as the reference's parity run does) so step 0 exercises the adapters
    with torch.no_grad():
        for p in qlora_model.lora_parameters(model):
            if p.abs().sum() == 0:
                p.normal_(0, 0.02)
    trainer = qlora_model.Trainer(model, steps=steps, fused_adapters=patched)
    if patched:
        patches.apply()
        monkeypatch.setattr(fused_head, "VOCAB_CHUNK", 384)  # several slices of 1000 tokens
    losses = []
    try:
        batches = [qlora_model.make_batch(seed=5, step=step, vocab=1000, seq=256, lo=64, hi=256)
                   for step in range(steps)]
        for step in range(steps):
            ahead = batches[step + 1] if step + 1 < steps else None
            losses.append(float(trainer.step(batches[step], ahead)))
    finally:
        if patched:
            patches.unapply()
    return losses


@pytest.mark.parametrize("path", ["fused", "per_node", "lora_node"])
def test_patched_step_matches_eager_loss_curve(monkeypatch, path):
    """fused: every node of the package (the attention half and the MLP as one node each);
    per_node: q|k|v node + varlen attention + GroupLinear and the per-projection MLP with the
    in-place SwiGLU; lora_node: without the q|k|v node (SOLUTION_DISABLE_FUSED_PROJ=1), q_proj
    and v_proj run as the single-projection LoRA node and RoPE as its own kernel."""
    from talm_amd import fused_mlp, fused_proj

    print(f"[case] qlora step small model eager vs patched path={path}", flush=True)
    if path == "per_node":
        monkeypatch.setattr(fused_proj, "ATTN_BLOCK", False)
        monkeypatch.setattr(fused_mlp, "ENABLED", False)
    if path == "lora_node":
        monkeypatch.setenv("SOLUTION_DISABLE_FUSED_PROJ", "1")
    engaged.reset()
    eager = _run(False, 6, monkeypatch)
    assert engaged.RAN["fused_head"] == 0
    fused = _run(True, 6, monkeypatch)
    names = ["fused_head", "unpad", "group", "addnorm", "head", "varlen_attn", "attn_kernel",
             "attn_kernel_bwd", "adapter_adamw"]
    names += {"fused": ["fused_proj", "qkv_mfma", "qkv_mfma_bwd", "fused_mlp", "attn_block"],
              "per_node": ["fused_proj", "qkv_mfma", "qkv_mfma_bwd", "swiglu_inplace"],
              "lora_node": ["lora", "qkv_mfma", "qkv_mfma_bwd", "rope", "fused_mlp"]}[path]
    for name in names:
        assert engaged.RAN[name] > 0, f"{name} did not run"
    if path == "lora_node":
        assert engaged.RAN["fused_proj"] == 0 and engaged.RAN["attn_block"] == 0
    assert abs(fused[0] - eager[0]) <= 1e-3 * abs(eager[0]), (fused[0], eager[0])
    for a, b in zip(fused, eager):
        assert abs(a - b) <= 5e-3 * abs(b), (fused, eager)


def test_varlen_attention_matches_per_row_sdpa():
    """The one-launch variable-length attention (unpad.VarlenAttention on the HIP kernels)
    against PyTorch's causal SDPA per row with GQA (the reference's per-row semantics,
    solution/unpad.py:121-134) on the config-5 row lengths, on the q|k|v buffer's views: outputs
    and q/k/v gradients within one fp16 rounding of the largest magnitude (both sides round)."""
    import torch.nn.functional as F

    from talm_amd import unpad, workloads

    print("[case] varlen attention vs per-row sdpa", flush=True)
    lengths, cu = workloads.varlen_lengths(1005)
    n = int(cu[-1])
    g = torch.Generator().manual_seed(0)
    qkv = torch.randn(n, 2048, generator=g).half().cuda()
    gout = torch.randn(1, n, 12, 128, generator=g).half().cuda()
    bounds = [(int(cu[i]), int(cu[i + 1])) for i in range(len(lengths))]

    def views(x):
        return (x[:, :1536].view(1, n, 12, 128).transpose(1, 2),
                x[:, 1536:1792].view(1, n, 2, 128).transpose(1, 2),
                x[:, 1792:].view(1, n, 2, 128).transpose(1, 2))

    x1 = qkv.clone().requires_grad_()
    out1 = unpad.VarlenAttention.apply(*views(x1), cu.cuda(), int(lengths.max()), 128 ** -0.5)
    out1.backward(gout)
    x2 = qkv.clone().requires_grad_()
    q, k, v = views(x2)
    outs = [F.scaled_dot_product_attention(q[:, :, s:e], k[:, :, s:e], v[:, :, s:e],
                                           is_causal=True, enable_gqa=True) for s, e in bounds]
    out2 = torch.cat(outs, 2).transpose(1, 2)
    out2.backward(gout)
    for a, b in ((out1, out2), (x1.grad, x2.grad)):
        torch.testing.assert_close(a.float(), b.float(), rtol=2 ** -10,
                                   atol=2 ** -10 * float(b.abs().max()))


def test_fused_mlp_matches_per_projection_mlp(monkeypatch):
    """FusedMLP (one node, feature-major activations, gate|up and their input gradient as single
    GEMMs) against the per-projection path (GroupLinear x 3 + the in-place SwiGLU node) on the
    same packed layer: output and input gradient within fp16 rounding, on a token count that is
    not a multiple of 8 (the padded leading dimension), with the backward's gate|up span and its
    per-projection form (two GEMMs, the second accumulating: the weights "qgroup" gives once it
    is off)."""
    from talm_amd import fused_mlp, qgroup, state

    print("[case] fused mlp vs per-projection mlp", flush=True)
    config = qlora_model.qwen2_config(vocab_size=1000, hidden_size=512, intermediate_size=1024,
                                      num_hidden_layers=3, num_attention_heads=4,
                                      num_key_value_heads=2, head_dim=128)
    model = qlora_model.build_model(config, seed=4)
    layer = model.model.layers[0]
    patches.apply()
    try:
        qgroup.setup_layer(layer)
        group = layer._solution_layer_group
        assert group is not None
        g = torch.Generator("cpu").manual_seed(9)
        x0 = torch.randn(1, 333, 512, generator=g).half().cuda()
        dy = (torch.randn(1, 333, 512, generator=g) * 0.1).half().cuda()
        results = []
        for fused, split_bwd in ((False, False), (True, False), (True, True)):
            monkeypatch.setattr(fused_mlp, "ENABLED", fused)
            qgroup.release()
            group.begin_forward()
            x = x0.clone().requires_grad_()
            ran = engaged.RAN["fused_mlp"]
            y = layer.mlp(x)
            assert (engaged.RAN["fused_mlp"] > ran) == fused
            if split_bwd:  # the backward takes each projection's own dequantization
                monkeypatch.setitem(state.DISABLED, "qgroup", "test")
            y.backward(dy)
            monkeypatch.delitem(state.DISABLED, "qgroup", raising=False)
            results.append((y.detach().float(), x.grad.float()))
        for y, dx in results[1:]:
            torch.testing.assert_close(y, results[0][0], rtol=2e-3, atol=2e-3 * float(y.abs().max()))
            torch.testing.assert_close(dx, results[0][1], rtol=2e-3,
                                       atol=2e-3 * float(dx.abs().max()))
    finally:
        patches.unapply()


def test_attention_block_matches_per_node_attention(monkeypatch):
    """AttentionBlock (q|k|v + LoRA + RoPE, the packed rows' attention and o_proj as one node)
    against the per-node path (FusedProjections, VarlenAttention, GroupLinear) on one packed
    layer with ragged rows (one of a single token): output, input gradient and the LoRA
    gradients within fp16 rounding, with the backward's q|k|v span and with the backward taking
    each projection's own dequantization (what "qgroup" gives once it is off)."""
    from talm_amd import fused_proj, qgroup, state, unpad

    print("[case] attention block vs per-node attention", flush=True)
    config = qlora_model.qwen2_config(vocab_size=1000, hidden_size=512, intermediate_size=1024,
                                      num_hidden_layers=3, num_attention_heads=4,
                                      num_key_value_heads=2, head_dim=128)
    model = qlora_model.build_model(config, seed=6)
    layer = model.model.layers[0]
    attn = layer.self_attn
    lora = [p for p in attn.parameters() if p.requires_grad]
    assert len(lora) == 4
    with torch.no_grad():
        for p in lora:
            if p.abs().sum() == 0:
                p.normal_(0, 0.02)
    patches.apply()
    try:
        qgroup.setup_layer(layer)
        group = layer._solution_layer_group
        assert group is not None
        lengths = [120, 77, 1, 135]
        bounds, start = [], 0
        for n in lengths:
            bounds.append((start, start + n))
            start += n
        positions = torch.cat([torch.arange(n) for n in lengths])[None].cuda()
        g = torch.Generator("cpu").manual_seed(11)
        x0 = torch.randn(1, start, 512, generator=g).half().cuda()
        dy = (torch.randn(1, start, 512, generator=g) * 0.1).half().cuda()
        cos, sin = model.model.rotary_emb(x0.float(), positions)
        results = []
        for block, split_bwd in ((False, False), (True, False), (True, True)):
            monkeypatch.setattr(fused_proj, "ATTN_BLOCK", block)
            qgroup.release()
            group.begin_forward()
            x = x0.clone().requires_grad_()
            for p in lora:
                p.grad = None
            ran, fused = engaged.RAN["attn_block"], engaged.RAN["fused_proj"]
            with unpad.rows_context(bounds, device=x.device), \
                    torch.autocast("cuda", dtype=torch.float16):
                y, _ = attn(x, position_embeddings=(cos, sin), attention_mask=None)
            assert (engaged.RAN["attn_block"] > ran) == block
            assert engaged.RAN["fused_proj"] > fused
            if split_bwd:
                monkeypatch.setitem(state.DISABLED, "qgroup", "test")
            y.backward(dy)
            monkeypatch.delitem(state.DISABLED, "qgroup", raising=False)
            results.append([y.detach().float(), x.grad.float()] + [p.grad.float() for p in lora])
        for other in results[1:]:
            for a, b in zip(other, results[0]):
                torch.testing.assert_close(a, b, rtol=2e-3, atol=2e-3 * float(b.abs().max()))
    finally:
        patches.unapply()
