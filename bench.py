"""Benchmark of the MI355X QLoRA kernel set (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAME,...]

Default workload: configuration 5, the full QLoRA step (the JSON line's `value`, mean ms per
step). Then the kernel suite of configurations 1-4. Per kernel: the launches are captured in a
HIP graph of `--reps` back-to-back launches and the graph is replayed (>= 200 timed launches),
with HIP events recorded on the launch stream around each replay; the reported duration is the
median over the replays of the per-launch average, so it is the kernel's time, not Python's
launch overhead. The bandwidth-bound kernels read and write a rotating set of buffers whose total
footprint is more than twice the 256 MB last-level cache, so their GB/s are HBM rates, not cache
rates. Achieved throughput divides the ALGORITHMIC bytes (or FLOPs) of one launch, stated next to
each kernel below, by that duration.

The last line printed is one JSON object (the driver's contract); per-kernel results ride in
its "kernels" list.
"""

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, GB/s
FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, TFLOP/s
LLC_BYTES = 256 * 2**20    # MI355X last-level (Infinity) cache

METRIC = "QLoRA step ms (Qwen2.5-1.5B shape, B4xS512); kernel HBM GB/s & MFMA %"

# HBM-side bytes per launch of each suite kernel, measured offline: two rocprofv3 --pmc runs of
# this file's kernel suite (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each scaled by what the
# counter reads for the 512 MiB calibration copy (--only copy): FETCH x 2.000, WRITE x 1.000.
# Commands and per-dispatch tables: profiles/kernel_suite_config1-4_hbm_traffic.md. The head is
# one talm_head_ce call (all its dispatches). Re-measured whenever a kernel changes.
MEASURED_TRAFFIC = {
    "nf4_group_dequant": 118.0e6,
    "add_rmsnorm_fwd": 18.1e6,
    "add_rmsnorm_bwd": 18.1e6,
    "rope_inplace": 10.1e6,
    "swiglu_fwd": 110.1e6,
    "swiglu_bwd": 183.5e6,
    "attn_fwd": 14.1e6,
    "attn_bwd": 56.9e6,  # its three dispatches: dot, the dQ / dK / dV kernel, the reduction
    "nf4_gemm_gate_up_dx": 227.8e6,  # the dequant-GEMM and the reduction of its K parts
    "head_ce_fwd_bwd": 4329e6,
    "nf4_group_dequant_streaming": 118.3e6,
    "qkv_lora_fwd_n1312": 54.1e6 + 5.2e6,   # proj_ext + lora_down
    "qkv_lora_bwd_n1312": 57.9e6 + 12.1e6 + 5.2e6 + 13.6e6 + 4.8e6,  # + prep, lora_down, wgrad
}


def graph_time_ms(fn, steps, warmup, reps):
    """Duration (ms) of one fn(i) launch, i = 0 .. reps - 1 selecting the buffer set: `reps`
    launches captured in one graph, the graph replayed until at least `steps` launches are timed,
    each replay between two events on the capture stream. Returns (median over replays of the
    per-launch average, mean over all launches, launches timed)."""
    for i in range(max(1, warmup)):
        fn(i % reps)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        fn(0)  # first launch outside capture on the side stream
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(reps):
                fn(i)
    torch.cuda.synchronize()
    replays = max(3, math.ceil(steps / reps))
    graph.replay()
    torch.cuda.synchronize()
    events = [torch.cuda.Event(enable_timing=True) for _ in range(replays + 1)]
    with torch.cuda.stream(stream):
        events[0].record(stream)
        for r in range(replays):
            graph.replay()
            events[r + 1].record(stream)
    events[-1].synchronize()
    per = [events[r].elapsed_time(events[r + 1]) / reps for r in range(replays)]
    return statistics.median(per), sum(per) / replays, replays * reps


def rotation(bytes_per_set, cap=64):
    """How many buffer sets of `bytes_per_set` bytes rotate so that their footprint is more than
    twice the last-level cache (a set is then evicted before it is used again)."""
    return max(2, min(cap, math.ceil(2.2 * LLC_BYTES / bytes_per_set)))


def kernel_suite(args, only):
    from talm_amd import qgroup, rmsnorm, rope, swiglu, workloads

    dev = "cuda"
    results = []

    def record(name, timing, bytes_=None, flops=None, config="", sets=1):
        ms, mean_ms, count = timing
        entry = {"kernel": name, "config": config, "us": round(ms * 1e3, 3),
                 "us_mean": round(mean_ms * 1e3, 3), "launches": count, "buffer_sets": sets}
        if bytes_ is not None:
            gbs = bytes_ / (ms * 1e-3) / 1e9
            entry.update(bytes=int(bytes_), gbs=round(gbs, 1),
                         hbm_frac=round(gbs / HBM_PEAK_GBS, 4),
                         footprint_mb=round(sets * bytes_ / 1e6, 1))
        if flops is not None:
            tf = flops / (ms * 1e-3) / 1e12
            entry.update(flops=int(flops), tflops=round(tf, 1),
                         mfma_frac=round(tf / FP16_PEAK_TFLOPS, 4))
        results.append(entry)
        print(f"[bench] {json.dumps(entry)}", flush=True)

    def want(name):
        return not only or name in only

    def timed(fn, sets):
        # every buffer set is used the same number of times per replay
        reps = sets * max(1, math.ceil(args.reps / sets)) if sets > 1 else args.reps
        return graph_time_ms(lambda i: fn(i % sets), args.steps, args.warmup, reps)

    if "copy" in only:
        # calibration for the HBM byte counters: a plain 512 MiB device copy reads and writes
        # exactly 512 MiB per launch (run only when named explicitly)
        src = torch.empty(2**28, dtype=torch.float16, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        record("copy_512MiB", timed(lambda i: dst.copy_(src), 1), bytes_=2 * 2**29,
               config="calibration")
        del src, dst

    if want("ceilings"):
        # this build's own streaming probes (talm_amd/csrc/bench/stream.hip, libtalm_bench.so) on
        # the read / write mixes of the bandwidth-bound kernels, at their byte counts, cold
        # buffers rotated like theirs: 16-byte accesses, 64 items per wavefront and iteration,
        # ordinary accesses, non-temporal ones, non-temporal loads with ordinary stores, or
        # non-temporal loads with buffer stores carrying the nt and sc1 cache-policy bits, several
        # grid sizes; the best of each mix is what this chip sustains for it (the ceiling the
        # kernels are compared with)
        import ctypes

        from talm_amd import build as tbuild

        blib = ctypes.CDLL(str(tbuild.BENCH_LIB))
        blib.talm_bench_stream.argtypes = [ctypes.c_int] * 4 + [ctypes.c_void_p] * 6 + [
            ctypes.c_int64, ctypes.c_int, ctypes.c_void_p]
        n_nf4 = 46792704
        mixes = [  # name, what, reads, writes, write items per read item, items
            ("ceiling_fill_0r1w", "write-only, 93.6 MB (the NF4 output)", 0, 1, 1,
             2 * n_nf4 // 16),
            ("ceiling_nf4_1r4w", "23.4 MB read, 93.6 MB written (the grouped NF4 dequant's mix)",
             1, 1, 4, n_nf4 // 2 // 16),
            ("ceiling_copy_1r1w", "copy of 36.7 MB", 1, 1, 1, 2048 * 8960 * 2 // 16),
            ("ceiling_2r1w", "2 x 36.7 MB read, 36.7 MB written (the SwiGLU forward's mix)",
             2, 1, 1, 2048 * 8960 * 2 // 16),
            ("ceiling_3r2w", "3 x 36.7 MB read, 2 x 36.7 MB written (the SwiGLU backward's mix)",
             3, 2, 1, 2048 * 8960 * 2 // 16),
            ("ceiling_2r3w", "2 x 100 MB read, 3 x 100 MB written (the 28-layer stacked "
             "add+RMSNorm forward's mix)", 2, 3, 1, 32676 * 1536 * 2 // 16),
        ]
        for name, what, nr, nw, wr, items in mixes:
            items -= items % 128
            nbytes = 16 * items * (nr + nw * wr)
            k = rotation(nbytes)
            sets = [([torch.ones(items * 8, dtype=torch.int16, device=dev) for _ in range(nr)],
                     [torch.empty(items * 8 * wr, dtype=torch.int16, device=dev)
                      for _ in range(nw)]) for _ in range(k)]
            best, by_kind = None, {}
            for nt in (0, 1, 2, 6):
                for grid in (0, 1024, 2048, 4096):
                    def op(i, nt=nt, grid=grid):
                        srcs, dsts = sets[i]
                        ptrs = [t.data_ptr() for t in srcs] + [None] * (3 - nr)
                        outs = [t.data_ptr() for t in dsts] + [None] * (3 - nw)
                        stream = torch.cuda.current_stream().cuda_stream
                        st = blib.talm_bench_stream(nr, nw, wr, nt, *ptrs, *outs, items, grid,
                                                    stream)
                        if st != 0:
                            raise RuntimeError(f"talm_bench_stream {name}: status {st}")

                    timing = timed(op, k)
                    if best is None or timing[0] < best[0][0]:
                        best = (timing, nt, grid)
                    kind = {0: "plain", 1: "non-temporal", 2: "non-temporal loads",
                            6: "non-temporal loads, nt sc1 buffer stores"}[nt]
                    if kind not in by_kind or timing[0] < by_kind[kind][0]:
                        by_kind[kind] = (timing[0], grid)
            (timing, nt, grid) = best
            fracs = ", ".join(f"{kind} {nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS:.3f} (grid "
                              f"{g or 'one-shot'})" for kind, (ms, g) in by_kind.items())
            record(name, timing, bytes_=nbytes, sets=k,
                   config=f"{what}; best of 4 access kinds x 4 grids: {fracs}")
            del sets

    if want("nf4_group"):
        d = workloads.nf4_layer()
        n_rows = d["absmax8"].numel()
        # packed + absmax8 + absmax2 + offsets (7 x 4) + code + fp16 out
        algo = d["n"] // 2 + n_rows + 4 * d["absmax2"].numel() + 28 + 1024 + 2 * d["n"]
        k = rotation(algo)
        sets = [{key: d[key].to(dev) for key in ("packed", "absmax8", "code", "absmax2",
                                                  "offset2")} for _ in range(k)]
        outs = [torch.empty(d["n"], dtype=torch.float16, device=dev) for _ in range(k)]

        for name, streaming in (("nf4_group_dequant", False),
                                ("nf4_group_dequant_streaming", True)):
            def fn(i, streaming=streaming):
                t = sets[i]
                qgroup.launch(t["packed"], t["absmax8"], t["code"], t["absmax2"], t["offset2"],
                              None, outs[i], n_rows, 64, 256, streaming=streaming)

            record(name, timed(fn, k), bytes_=algo, sets=k,
                   config="1: Qwen2.5-1.5B layer, " + (
                       "non-temporal stores (talm_nf4_group_dequant_streaming)" if streaming else
                       "ordinary stores (the training step's: its GEMMs read the layer next)"))
        del sets, outs

    if want("nf4_gemm"):
        # the W4A16 dequant-GEMM on config 1's layer as the step runs it: the MLP's gate|up input
        # gradient dx = [dgate | dup] [W_gate; W_up] read as NF4 codes, at a step's token count
        from talm_amd import _ops

        d = workloads.nf4_layer()
        t = {key: d[key].to(dev) for key in ("packed", "absmax8", "code", "absmax2", "offset2")}
        scale = torch.empty(d["n"] // 64, dtype=torch.float32, device=dev)
        torch.ops.talm.nf4_block_scales(t["absmax8"], t["code"], t["absmax2"], t["offset2"], 256,
                                        scale)
        shapes = d["shapes"]
        e0 = sum(a * b for a, b in shapes[:4])  # gate's first weight
        rows, cols, n_tok = shapes[4][0] + shapes[5][0], shapes[4][1], 1312
        dy = torch.randn(n_tok, rows, generator=torch.Generator().manual_seed(5)).half().to(dev)
        dx = torch.empty(n_tok, cols, dtype=torch.float16, device=dev)
        ws = torch.empty(_ops.nf4_gemm_workspace_bytes(n_tok, rows, cols, True),
                         dtype=torch.uint8, device=dev)
        packed, sc = t["packed"][e0 // 2:], scale[e0 // 64:]

        def fn(i):
            torch.ops.talm.nf4_gemm(dy, packed, sc, rows, cols, True, 64, dx, ws)

        record("nf4_gemm_gate_up_dx", timed(fn, 1), flops=2.0 * n_tok * rows * cols,
               config=f"gate|up input gradient of the config-1 layer on its NF4 codes, "
                      f"{n_tok} tokens")
        del t, scale, dy, dx, ws

    d2 = workloads.norm_rope() if any(want(x) for x in ("addnorm_fwd", "addnorm_bwd", "rope",
                                                         "stacked", "attn")) else None
    # config 2's shapes, and (with "stacked") the 28 layers' rows in one launch: the per-launch
    # floor of these 10-18 MB kernels apart from their streaming rate
    norm_stacks = [st for st in (1, 28) if d2 is not None and (
        (st == 1 and (want("addnorm_fwd") or want("addnorm_bwd"))) or (st == 28 and want("stacked")))]
    rope_stacks = [st for st in (1, 28) if d2 is not None and (
        (st == 1 and want("rope")) or (st == 28 and want("stacked")))]
    for stack in norm_stacks:
        name_sfx = "" if stack == 1 else "_stacked28"
        n, hdim = d2["n"] * stack, 1536
        nbytes = 10 * n * hdim + 4 * n + 4 * hdim
        k = rotation(nbytes)
        w = d2["weight"].to(dev)

        def norm_set():
            x = d2["residual"].to(dev).repeat(stack, 1)
            br = d2["x"].to(dev).repeat(stack, 1)
            return {"x": x, "br": br, "total": torch.empty_like(x), "y": torch.empty_like(x),
                    "xhat": torch.empty_like(x),
                    "rstd": torch.empty(n, dtype=torch.float32, device=dev),
                    "dy": d2["dy"].to(dev).repeat(stack, 1), "ds": d2["ds"].to(dev).repeat(stack, 1),
                    "dx": torch.empty_like(x), "db": torch.empty_like(x)}

        sets = [norm_set() for _ in range(k)]

        def fwd(i):
            s_ = sets[i]
            rmsnorm.launch(s_["x"], w, s_["y"], s_["xhat"], s_["rstd"], 1e-6, 0, p=s_["br"],
                           q=s_["total"])

        def bwd(i):
            s_ = sets[i]
            rmsnorm.launch(s_["dx"], w, s_["dy"], s_["xhat"], s_["rstd"], 1e-6, 1, p=s_["db"],
                           q=s_["ds"])

        for i in range(k):
            fwd(i)
        cfg = f"2: N={d2['n']}" + ("" if stack == 1 else f" x 28 layers in one launch ({n} rows)")
        if want("addnorm_fwd") or stack > 1:
            record("add_rmsnorm_fwd" + name_sfx, timed(fwd, k), bytes_=nbytes, config=cfg, sets=k)
        if want("addnorm_bwd") or stack > 1:
            record("add_rmsnorm_bwd" + name_sfx, timed(bwd, k), bytes_=nbytes, config=cfg, sets=k)
        del sets

    for stack in rope_stacks:
        n = d2["n"] * stack
        nbytes = 8192 * n
        k = rotation(nbytes)

        def rope_set():
            qkv = torch.randn(n, 2048, device=dev).half()
            return (qkv[:, :1536].view(n, 12, 128), qkv[:, 1536:1792].view(n, 2, 128),
                    d2["cos"].to(dev).repeat(stack, 1), d2["sin"].to(dev).repeat(stack, 1))

        sets = [rope_set() for _ in range(k)]

        def fn(i):
            q, k_, cos, sin = sets[i]
            rope.rope_(q, k_, cos, sin, backward=False)

        cfg = f"2: N={d2['n']}" + ("" if stack == 1 else f" x 28 layers in one launch ({n} rows)")
        record("rope_inplace" + ("" if stack == 1 else "_stacked28"), timed(fn, k),
               bytes_=nbytes, config=cfg, sets=k)
        del sets

    if want("attn") and d2 is not None:
        # the varlen causal GQA attention of one layer at config 2's lengths, on q|k|v views of
        # one [N, 2048] buffer as in the step; algorithmic FLOPs over the causal pairs: 2 GEMMs
        # forward (S, P V), 5 backward (S, dP, dV, dQ, dK), 2 * Hq * D FLOP per pair and GEMM
        from talm_amd import _ops

        lengths, cu = d2["lengths"], d2["cu_seqlens"].to(dev)
        n, hq, hkv, hd = d2["n"], 12, 2, 128
        pairs = int(sum(int(x) * (int(x) + 1) // 2 for x in lengths))
        unit = 2.0 * hq * hd * pairs
        g = torch.Generator().manual_seed(5)
        qkv = torch.randn(n, 2048, generator=g).half().to(dev)
        dqkv = torch.empty_like(qkv)
        q = qkv[:, :1536].view(n, hq, hd)
        k = qkv[:, 1536:1792].view(n, hkv, hd)
        v = qkv[:, 1792:].view(n, hkv, hd)
        o = torch.empty(n, hq, hd, dtype=torch.float16, device=dev)
        lse = torch.empty(hq, n, dtype=torch.float32, device=dev)
        do = (0.1 * torch.randn(n, hq, hd, generator=g)).half().to(dev)
        ws = torch.empty(_ops.attn_bwd_workspace_bytes(n, hq), dtype=torch.uint8, device=dev)
        max_len, scale = int(lengths.max()), hd ** -0.5

        def fwd(i):
            torch.ops.talm.attn_fwd(q, k, v, cu, max_len, scale, o, lse)

        def bwd(i):
            torch.ops.talm.attn_bwd(q, k, v, o, do, lse, cu, max_len, scale,
                                    dqkv[:, :1536].view(n, hq, hd),
                                    dqkv[:, 1536:1792].view(n, hkv, hd),
                                    dqkv[:, 1792:].view(n, hkv, hd), ws)

        fwd(0)
        cfg = f"2: lengths {[int(x) for x in lengths]}, Hq 12, Hkv 2, D 128"
        record("attn_fwd", timed(fwd, 1), flops=2 * unit, config=cfg)
        record("attn_bwd", timed(bwd, 1), flops=5 * unit, config=cfg)

    if want("qkv"):
        # the fused q|k|v projection with the q and v LoRA adapters (r 16, scaling 2) and the
        # rotary embedding in place, as the step's attention block runs it (fused_proj.py):
        # forward = lora_down (t = x [A_q; A_v]^T) + proj_ext ([x | s t] [W | B]^T + b, RoPE);
        # backward = qkv_bwd_prep (RoPE-back, concatenation) + lora_down (u = s dy B) +
        # proj_ext (dX = [dcat | u] [W^T | A^T]^T) + lora_wgrad (dA = u^T x, dB = s dy^T t).
        # Algorithmic FLOPs: forward 2 N H (n_out + 32) + 2 N 16 (n_q + n_v); backward
        # 2 N (n_out + 32) H + 2 N 16 (n_q + n_v) (u) + 2 N 32 H (dA) + 2 N 16 (n_q + n_v) (dB)
        from talm_amd import fused_proj

        hdim, sizes, r = 1536, (1536, 256, 256), 16
        bounds = [0, 1536, 1792, 2048]
        n_out, n_qv = bounds[-1], sizes[0] + sizes[2]
        adapters = [(0, 2.0, 0.0), (2, 2.0, 0.0)]
        n_cfg2 = workloads.norm_rope()["n"] if d2 is None else d2["n"]
        for n in (n_cfg2, 1312):
            g = torch.Generator().manual_seed(17)
            x2 = torch.randn(n, hdim, generator=g).half().to(dev)
            w = (0.02 * torch.randn(n_out, hdim, generator=g)).half().to(dev)
            w_t = w.t().contiguous()
            bias = (0.02 * torch.randn(n_out, generator=g)).half().to(dev)
            halves = [((0.02 * torch.randn(r, hdim, generator=g)).half().to(dev),
                       (0.02 * torch.randn(sizes[seg], r, generator=g)).half().to(dev))
                      for seg, _s, _p in adapters]
            a_t = torch.cat([a for a, _b in halves], 0).t().contiguous()
            cos, sin = (t_.to(dev) for t_ in workloads.rope_cos_sin(torch.arange(n) % 512))
            state = {}

            def fwd(i):
                state["out"], state["t"] = fused_proj._mfma_forward(
                    x2, w, bias, bounds, adapters, halves, (cos, sin))

            fwd(0)
            dqkv = (0.1 * torch.randn(n, n_out, generator=g)).half().to(dev)
            grads = (dqkv[:, :1536], dqkv[:, 1536:1792], dqkv[:, 1792:])
            t = state["t"]
            rest = [t[:, :16], halves[0][0], halves[0][1], t[:, 16:], halves[1][0], halves[1][1]]
            outs = [torch.empty(r, hdim, dtype=torch.float32, device=dev),
                    torch.empty(sizes[0], r, dtype=torch.float32, device=dev),
                    torch.empty(r, hdim, dtype=torch.float32, device=dev),
                    torch.empty(sizes[2], r, dtype=torch.float32, device=dev)]

            def bwd(i):
                fused_proj._mfma_backward_core(grads, x2, rest, cos, sin, None, sizes, adapters,
                                               True, [True] * 4, a_t, outs, w_t)

            cfg = (f"q|k|v + LoRA r16 on q, v + RoPE, N={n} H=1536 (q 1536, k 256, v 256)")
            f_fwd = 2.0 * n * hdim * (n_out + 2 * r) + 2.0 * n * r * n_qv
            f_bwd = 2.0 * n * (n_out + 2 * r) * hdim + 4.0 * n * r * n_qv + 2.0 * n * 2 * r * hdim
            record(f"qkv_lora_fwd_n{n}", timed(fwd, 1), flops=f_fwd, config=cfg)
            record(f"qkv_lora_bwd_n{n}", timed(bwd, 1), flops=f_bwd, config=cfg)
            del x2, w, w_t, dqkv, state, outs

    if want("swiglu_fwd") or want("swiglu_bwd"):
        d3 = workloads.swiglu_inputs()
        n = d3["gate"].numel()
        for name, per_elem in (("swiglu_fwd", 6), ("swiglu_bwd", 10)):
            if not want(name):
                continue
            k = rotation(per_elem * n)
            sets = [{key: d3[key].to(dev) for key in ("gate", "up", "grad")} for _ in range(k)]
            for s_ in sets:
                s_["out"], s_["dgate"], s_["dup"] = (torch.empty_like(s_["gate"])
                                                     for _ in range(3))
            if name == "swiglu_fwd":
                def fn(i):
                    s_ = sets[i]
                    swiglu.swiglu_fwd(s_["gate"], s_["up"], s_["out"])
            else:
                def fn(i):
                    s_ = sets[i]
                    swiglu.swiglu_bwd(s_["grad"], s_["gate"], s_["up"], s_["dgate"], s_["dup"])
            record(name, timed(fn, k), bytes_=per_elem * n, config="3: [2048, 8960]", sets=k)
            del sets
    if want("head"):
        from talm_amd import _ops, fused_head

        d4 = workloads.head_inputs()
        targets = d4["targets"]
        labelled = targets >= 0
        n_lab = int(labelled.sum())
        order = torch.cat([torch.nonzero(labelled)[:, 0], torch.nonzero(~labelled)[:, 0]])
        h16 = d4["hidden"][order].contiguous().to(dev)
        w16 = d4["weight"].to(dev)
        tt = targets[order].contiguous().to(dev)
        n, hdim = h16.shape
        vocab = w16.shape[0]
        vchunk, group = fused_head.VOCAB_CHUNK, fused_head.GROUP
        outs = [torch.empty(n, dtype=torch.float32, device=dev),
                torch.empty(n, dtype=torch.float32, device=dev),
                torch.empty(n, dtype=torch.int32, device=dev),
                torch.empty(n, dtype=torch.int32, device=dev),
                torch.empty(n, hdim, dtype=torch.float16, device=dev)]
        ws = torch.empty(_ops.head_ce_workspace_bytes(n, hdim, vocab, vchunk, n_lab, group),
                         dtype=torch.uint8, device=dev)
        def fn(i):
            torch.ops.talm.head_ce(h16, w16, tt, vchunk, n_lab, group, *outs, ws)

        # compute-bound (the 467 MB weight streams from HBM on every call anyway): one set
        timing = graph_time_ms(fn, 200, 3, 10)
        flops = 2.0 * vocab * hdim * (n + n_lab)
        record("head_ce_fwd_bwd", timing, flops=flops,
               config=f"4: N={n} H={hdim} V={vocab} N_lab={n_lab} vchunk={vchunk}")
    return results


def run_steps(model, trainer, n_steps, seed, timed_from, before_timing=None):
    """Run n_steps optimizer steps; time steps [timed_from, n_steps) between two device syncs
    (`before_timing()` runs just before the first timed step). Returns (losses,
    ms_per_timed_step, peak_bytes)."""
    from talm_amd import qlora_model

    vocab = model.config.vocab_size
    batches = [qlora_model.make_batch(seed, i, vocab) for i in range(n_steps)]
    losses = []
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    t0 = None
    for i in range(n_steps):
        if i == timed_from:
            if before_timing is not None:
                before_timing()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
        losses.append(trainer.step(batches[i], batches[i + 1] if i + 1 < n_steps else None))
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / max(1, n_steps - timed_from)
    return [float(x) for x in losses], ms, torch.cuda.max_memory_allocated()


def step_workload(args):
    """Configuration 5: the full QLoRA step of the Qwen2.5-1.5B-shaped model, patched
    (every kernel of the package), and the unpatched eager path for the loss curve."""
    from talm_amd import engaged, patches, qlora_model

    n_steps = args.warmup + args.steps
    out = {}
    for mode in ("patched", "eager") if not args.no_eager else ("patched",):
        torch.cuda.empty_cache()
        model = qlora_model.build_model(seed=1)
        trainer = qlora_model.Trainer(model, steps=n_steps, fused_adapters=mode == "patched")
        runner, prepare, graphed = trainer, None, None
        if mode == "patched":
            patches.apply()
            engaged.reset()
            if not args.no_graph:
                from talm_amd.step_graph import GraphedTrainer

                # forward + backward replayed from one HIP graph per 16-token bucket; every
                # bucket of the workload's token range (4 rows of 128..512) is captured before
                # the timed steps, as the reference warms its kernels up before training
                graphed = runner = GraphedTrainer(trainer, bucket=16,
                                                  warm_steps=max(1, min(args.warmup, 2)))
                prepare = lambda: graphed.prepare(4 * 128, 4 * 512)  # noqa: E731
        try:
            losses, ms, peak = run_steps(model, runner, n_steps, seed=7,
                                         timed_from=max(args.warmup, 1 if graphed else 0),
                                         before_timing=prepare)
        finally:
            if mode == "patched":
                ran = dict(engaged.RAN)
                patches.unapply()
            if graphed is not None:
                graph_info = {"graphs": len(graphed.graphs), "replays": graphed.replays,
                              "capture_s": round(graphed.capture_seconds, 2),
                              "bucket": graphed.bucket}
                graphed.close()
        out[mode] = {"losses": losses, "ms_per_step": ms, "peak_bytes": peak}
        if mode == "patched":
            out[mode]["engaged"] = ran
            if graphed is not None:
                out[mode]["hip_graph"] = graph_info
        print(f"[bench] step {mode}: {ms:.2f} ms/step, peak {peak / 2**30:.2f} GiB, "
              f"loss {losses[0]:.4f} -> {losses[-1]:.4f}", flush=True)
        del model, trainer
    return out


def cpu_host():
    """Core counts and CPU model of the host the CPU baseline ran on."""
    model = ""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"threads": torch.get_num_threads(), "cpu_count": os.cpu_count(),
            "affinity": len(os.sched_getaffinity(0)), "cpu_model": model}


def cpu_model_from(model):
    """The QLoRA model moved to the host for the reference's CPU eager path: fp32 compute, the
    tied embedding in fp32, the 4-bit layers dequantizing with the oracle's PyTorch CPU
    restatement of bitsandbytes' dequantize_4bit (the product has no CPU path)."""
    from oracle import nf4 as nf4_oracle
    from talm_amd import nf4_linear

    model = model.to("cpu")
    embed = model.model.embed_tokens
    embed.weight.data = embed.weight.data.float()
    for module in model.modules():
        if isinstance(module, nf4_linear.Linear4bit):
            module.compute_dtype = torch.float32
            if module.bias is not None:
                module.bias.data = module.bias.data.float()
    nf4_linear.dequantize_4bit = nf4_oracle.dequant_state_torch
    return model


def cpu_baseline_step(n_timed=2, seed=7):
    """The reference's CPU eager path, measured: the unpatched QLoRA step of configuration 5
    (the same Qwen2.5-1.5B-shaped model and B4 x S512 batches as the GPU runs) in fp32 PyTorch
    on the host cores — per projection NF4 dequantization + F.linear, PEFT's LoRA, transformers'
    SDPA attention on the padded batch, full logits and cross-entropy, backward, clipping and
    AdamW — 1 warm-up step, then `n_timed` timed steps (the planned "2-step CPU sample")."""
    from talm_amd import nf4_linear, qlora_model

    real_dequant = nf4_linear.dequantize_4bit
    torch.cuda.empty_cache()
    model = cpu_model_from(qlora_model.build_model(seed=1))
    try:
        params = qlora_model.lora_parameters(model)
        opt = torch.optim.AdamW(params, lr=2e-4, weight_decay=0.01)
        vocab = model.config.vocab_size
        times, tokens, losses = [], 0, []
        for i in range(1 + n_timed):
            # the warm-up step (thread pools, allocator) runs on one short row
            batch = qlora_model.make_batch(seed, i, vocab, device="cpu") if i else \
                qlora_model.make_batch(seed, i, vocab, batch=1, seq=128, lo=64, hi=128,
                                       device="cpu")
            t0 = time.perf_counter()
            out = model(**batch)
            out.loss.backward()
            torch.nn.utils.clip_grad_norm_(params, 1.0)
            opt.step()
            opt.zero_grad(set_to_none=True)
            dt = time.perf_counter() - t0
            losses.append(out.loss.item())
            print(f"[bench] cpu step {i}: {dt:.2f} s, loss {losses[-1]:.4f}", flush=True)
            if i > 0:
                times.append(dt)
                tokens += int(batch["attention_mask"].sum())
    finally:
        nf4_linear.dequantize_4bit = real_dequant
    del model
    host = cpu_host()
    ms = 1e3 * sum(times) / len(times)
    return {"value": round(ms, 1), "unit": "ms/step", "cores": host["threads"], "kind": "port",
            "sample": f"{n_timed} timed steps (after a 1-row warm-up step) of the unpatched "
                      f"config-5 QLoRA step in fp32 PyTorch CPU eager (B4 x S512 padded, "
                      f"{tokens} real tokens in the timed steps; bitsandbytes' dequantize_4bit "
                      f"as the oracle's PyTorch restatement), losses "
                      f"{', '.join(f'{x:.4f}' for x in losses[1:])}",
            "host": host, "step_seconds": [round(t, 2) for t in times]}


def cpu_baseline_nf4(seconds):
    """The C oracle of the grouped NF4 dequant (one thread) on the config-1 layer, repeated for
    about `seconds`; weights per second."""
    from oracle import nf4 as nf4_oracle
    from talm_amd import workloads

    d = workloads.nf4_layer()
    args = [d[k].numpy() for k in ("packed", "absmax8", "code", "absmax2", "offset2")]
    t0 = time.perf_counter()
    reps = 0
    while True:
        nf4_oracle.group_dequant(*args)
        reps += 1
        if time.perf_counter() - t0 > seconds:
            break
    dt = time.perf_counter() - t0
    return {"value": round(reps * d["n"] / dt / 1e9, 4), "unit": "Gweights/s", "cores": 1,
            "kind": "port",
            "sample": f"{reps} x config-1 layer ({d['n']} weights), C oracle, 1 thread, {dt:.1f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--only", default="")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--workload", choices=("step", "kernels"), default="step")
    ap.add_argument("--no-eager", action="store_true", help="skip the eager loss-curve run")
    ap.add_argument("--no-graph", action="store_true",
                    help="run the patched step eagerly (no HIP graph replay)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: every box of this build has a single MI355X and "
              "the kernel set runs unsharded (its multi-GPU sharding is a design, not code).",
              file=sys.stderr)
        sys.exit(2)
    torch.cuda.set_device(0)
    only = {s for s in args.only.split(",") if s}
    if args.workload == "step":
        # defaults: 64 steps, the first 2 untimed (the reference times steps 3-64)
        if "--steps" not in sys.argv:
            args.steps = 62
        if "--warmup" not in sys.argv:
            args.warmup = 2
    step = step_workload(args) if args.workload == "step" else None
    kernel_args = args if step is None else argparse.Namespace(
        **{**vars(args), "steps": 200, "warmup": 10})
    kernels = kernel_suite(kernel_args, only)
    measured = [e for e in kernels if not e["kernel"].startswith("ceiling_")]
    dominant = max(measured, key=lambda e: e["us"]) if measured else None
    line_roofline = None
    traffic = MEASURED_TRAFFIC.get(dominant["kernel"]) if dominant is not None else None
    if dominant is not None and "tflops" in dominant:
        line_roofline = {"kernel": dominant["kernel"], "bound": "mfma",
                         "achieved": dominant["tflops"], "peak": FP16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": dominant["mfma_frac"], "traffic": traffic}
    elif dominant is not None:
        line_roofline = {"kernel": dominant["kernel"], "bound": "hbm",
                         "achieved": dominant["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": dominant["hbm_frac"], "traffic": traffic}
    line = {"metric": METRIC, "value": None, "unit": "ms", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": None, "higher_is_better": False,
            "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
            "config": {"workload": "kernel suite (configs 1-4)"}}
    if step is not None:
        p = step["patched"]
        line.update(value=round(p["ms_per_step"], 3), ms_per_step=round(p["ms_per_step"], 3))
        line["config"] = {"workload": "config 5: QLoRA step, Qwen2.5-1.5B shape (28 layers, "
                                      "NF4 double-quant base, LoRA r16/a32 on q,v), B4 x S512 "
                                      "varlen (lengths U[128,512]), fp16 autocast, AdamW",
                          "global_batch": 4, "seq_len": 512, "parallelism": "none (1 GPU)"}
        line["peak_hbm_gib"] = round(p["peak_bytes"] / 2**30, 3)
        line["loss_first_last"] = [round(p["losses"][0], 5), round(p["losses"][-1], 5)]
        if "eager" in step:
            e = step["eager"]
            rel = [abs(a - b) / abs(b) for a, b in zip(p["losses"], e["losses"])]
            line["eager_ms_per_step"] = round(e["ms_per_step"], 3)
            line["eager_peak_hbm_gib"] = round(e["peak_bytes"] / 2**30, 3)
            line["loss_curve_max_rel_diff"] = round(max(rel), 6)
            line["loss_curve_mean_rel_diff"] = round(sum(rel) / len(rel), 6)
        line["engaged"] = {k: v for k, v in sorted(p["engaged"].items()) if v}
        if "hip_graph" in p:  # engaged counts: eager warm-up steps and graph captures
            line["hip_graph"] = p["hip_graph"]
    line["kernels"] = kernels
    if line_roofline is not None:
        line["roofline"] = line_roofline
    if args.cpu_seconds > 0:
        line["cpu_baseline"] = (cpu_baseline_step() if step is not None
                                else cpu_baseline_nf4(args.cpu_seconds))
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
