"""The adapters' device state: talm_lora_mirror (fp16 copies and the side-by-side transposes of
the q|k|v nodes' A matrices) against PyTorch's casts, bit for bit; talm_lora_adamw /
AdapterAdamW against torch.optim.AdamW (the reference's optimizer) step by step, with the
GradScaler's scale and inf flag on the device; the copies registry's refresh rules."""

import pytest
import torch

from talm_amd import adapters

pytestmark = pytest.mark.gpu


def _row(w, h_off, t_off=-1, ld_t=0, g=None, m=None, v=None):
    return [w.data_ptr(), w.numel(), w.shape[1], h_off, t_off, ld_t,
            0 if g is None else g.data_ptr(), 0 if m is None else m.data_ptr(),
            0 if v is None else v.data_ptr()]


def test_mirror_copies_and_transposes_bit_exact():
    print("[case] lora_mirror: copies + transposes vs torch casts", flush=True)
    g = torch.Generator().manual_seed(1)
    # odd shapes (element counts not multiples of 4), the adapters' shapes, values around the
    # fp16 rounding boundaries and its subnormal range
    shapes = [(3, 5), (16, 1536), (1536, 16), (256, 16), (16, 1536), (1, 7)]
    ws = [(torch.randn(*s, generator=g) * 10.0 ** torch.randint(-6, 3, s, generator=g)).cuda()
          for s in shapes]
    off, rows = 0, []
    h_offs = []
    for w in ws:
        h_offs.append(off)
        off += (w.numel() + 7) // 8 * 8
    t_off = off  # A^T of ws[1] and ws[4] side by side: [1536, 32]
    off += 1536 * 32
    for i, w in enumerate(ws):
        t = {1: t_off, 4: t_off + 16}.get(i, -1)
        rows.append(_row(w, h_offs[i], t, 32 if t >= 0 else 0))
    table = torch.tensor(rows, dtype=torch.int64).cuda()
    out = torch.full((off,), float("nan"), dtype=torch.float16, device="cuda")
    torch.ops.talm.lora_mirror(table, len(ws), max(w.numel() for w in ws), out)
    for w, h in zip(ws, h_offs):
        got = out[h:h + w.numel()].view(w.shape)
        assert torch.equal(got.view(torch.int16), w.to(torch.float16).view(torch.int16))
    want_t = torch.cat([ws[1], ws[4]], 0).t().to(torch.float16).contiguous()
    got_t = out[t_off:t_off + 1536 * 32].view(1536, 32)
    assert torch.equal(got_t.view(torch.int16), want_t.view(torch.int16))


@pytest.mark.parametrize("scaled", [False, True])
def test_adamw_matches_torch_adamw(scaled):
    print(f"[case] lora_adamw vs torch AdamW scaled={scaled}", flush=True)
    g = torch.Generator().manual_seed(2)
    shapes = [(16, 1536), (1536, 16), (16, 1536), (256, 16), (3, 5)]
    ref = [torch.randn(*s, generator=g).mul(0.05).cuda().requires_grad_() for s in shapes]
    ours = [p.detach().clone().requires_grad_() for p in ref]
    opt_ref = torch.optim.AdamW(ref, lr=3e-3, betas=(0.9, 0.99), eps=1e-6, weight_decay=0.1,
                                foreach=False, fused=False)
    copies = adapters.AdapterCopies()
    for p in ours:
        copies.half(p)
    copies.pair_t((ours[0], ours[2]))
    opt = adapters.AdapterAdamW(ours, lr=3e-3, betas=(0.9, 0.99), eps=1e-6, weight_decay=0.1,
                                copies=copies)
    scale = torch.tensor([1024.0], device="cuda")
    for step in range(5):
        grads = [torch.randn(*s, generator=g).cuda() for s in shapes]
        for p, q, gr in zip(ref, ours, grads):
            p.grad = gr.clone()
            q.grad = gr * 1024.0 if scaled else gr.clone()
        opt_ref.step()
        if scaled:
            opt.grad_scale = scale
            opt.found_inf = torch.zeros(1, device="cuda")
        opt.step()
        for p, q in zip(ref, ours):
            torch.testing.assert_close(q.detach(), p.detach(), rtol=1e-5, atol=1e-7)
        # the copies of the updated weights, made by the same launch
        for q in ours:
            assert torch.equal(copies.half(q).view(torch.int16),
                               q.detach().to(torch.float16).view(torch.int16))
        want_t = torch.cat([ours[0], ours[2]], 0).detach().t().to(torch.float16).contiguous()
        assert torch.equal(copies.pair_t((ours[0], ours[2])).view(torch.int16),
                           want_t.view(torch.int16))
    assert copies.adopted_by is opt


def test_adamw_skips_on_inf_and_keeps_step_count():
    print("[case] lora_adamw found_inf", flush=True)
    p = torch.randn(16, 64).cuda().requires_grad_()
    before = p.detach().clone()
    opt = adapters.AdapterAdamW([p], lr=1e-2, copies=adapters.AdapterCopies())
    p.grad = torch.ones_like(p)
    opt.found_inf = torch.ones(1, device="cuda")
    opt.step()
    del opt.found_inf
    assert torch.equal(p.detach(), before)
    steps = opt.param_groups[0]["_talm_steps"]
    assert float(steps.sum()) == 0.0
    opt.step()  # a real first step: t = 1
    assert not torch.equal(p.detach(), before)
    assert float(opt.state[p]["step"]) == 1.0


def test_copies_registry_refreshes_after_inplace_change():
    print("[case] adapter copies registry refresh", flush=True)
    copies = adapters.AdapterCopies()
    ws = [torch.randn(16, 256).cuda(), torch.randn(16, 256).cuda()]
    first = [copies.half(w) for w in ws]  # first use: standalone copies
    copies.pair_t(tuple(ws))
    second = [copies.half(w) for w in ws]  # laid out: views of one buffer
    assert second[0].data_ptr() != first[0].data_ptr()
    for w, h in zip(ws, second):
        assert torch.equal(h, w.to(torch.float16))
    with torch.no_grad():
        ws[0].mul_(2.0)  # version bump: the next use refreshes every copy in one launch
    third = copies.half(ws[0])
    assert torch.equal(third, ws[0].to(torch.float16))
    assert torch.equal(second[0], first[0])  # an earlier copy is never overwritten
    t = copies.pair_t(tuple(ws))
    assert torch.equal(t, torch.cat(ws, 0).t().to(torch.float16))


@pytest.mark.parametrize("case", ["clipped", "unclipped", "inf"])
def test_fused_tail_matches_unscale_clip_step(case):
    """AdapterAdamW.fused_tail (talm_lora_grad_norm + talm_lora_adamw_clipped) against
    GradScaler.unscale_ + clip_grad_norm_ + GradScaler.step + update on the same scaled
    gradients: the same total norm (to the norm's summation order), the same weights and moments
    after the step, the same scale after the update; with an inf gradient no weight moves and
    the scale backs off in both."""
    print(f"[case] fused optimizer tail: {case}", flush=True)
    g = torch.Generator().manual_seed(3)
    shapes = [(16, 1536), (1536, 16), (16, 1536), (256, 16)]
    size = {"clipped": 1.0, "unclipped": 1e-4, "inf": 1.0}[case]
    grads = [torch.randn(*s, generator=g).mul(size).cuda() for s in shapes]
    if case == "inf":
        grads[2][3, 7] = float("inf")
    runs = []
    for fused in (False, True):
        params = [torch.randn(*s, generator=torch.Generator().manual_seed(4 + i)).mul(0.05)
                  .cuda().requires_grad_() for i, s in enumerate(shapes)]
        opt = adapters.AdapterAdamW(params, lr=1e-3, weight_decay=0.01,
                                    copies=adapters.AdapterCopies())
        scaler = torch.amp.GradScaler("cuda", init_scale=2.0 ** 16)
        scaler.scale(torch.ones((), device="cuda"))  # the scale tensor exists, as after a step
        for p, gr in zip(params, grads):
            p.grad = gr * scaler.get_scale()
        if fused:
            norm = opt.fused_tail(scaler, 1.0)
            assert norm is not None
        else:
            scaler.unscale_(opt)
            norm = torch.nn.utils.clip_grad_norm_(params, 1.0)
            scaler.step(opt)
        scaler.update()
        runs.append((norm, [p.detach().clone() for p in params],
                     [opt.state[p]["exp_avg_sq"].clone() for p in params], scaler.get_scale()))
    (n0, w0, v0, s0), (n1, w1, v1, s1) = runs
    assert s0 == s1
    if case == "inf":
        assert not torch.isfinite(n1) or not torch.isfinite(n0)
        for a, b in zip(w0, w1):
            assert torch.equal(a, b)
        return
    assert abs(float(n1) - float(n0)) <= 1e-6 * float(n0)
    for a, b in zip(w0, w1):
        torch.testing.assert_close(b, a, rtol=1e-6, atol=1e-9)
    for a, b in zip(v0, v1):
        torch.testing.assert_close(b, a, rtol=1e-5, atol=1e-20)
