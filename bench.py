"""Benchmark of the MI355X QLoRA kernel set (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAME,...]

Per kernel: K timed launches after W warm-up launches. The launches are
captured once in a HIP graph of `--reps` back-to-back launches and the graph is replayed, with
HIP events recorded on the launch stream around the replays, so the average duration is the
kernel's, not Python's launch overhead. Achieved throughput divides the ALGORITHMIC bytes (or
FLOPs) of one launch, stated next to each kernel below, by that average duration.

The last line printed is one JSON object (the driver's contract); per-kernel results ride in
its "kernels" list.
"""

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, GB/s
FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, TFLOP/s

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
    "swiglu_bwd": 183.6e6,
    "head_ce_fwd_bwd": 4546e6,
}


def graph_time_ms(fn, steps, warmup, reps):
    """Average duration (ms) of one fn() launch: `reps` launches captured in one graph,
    replayed until `steps` launches are timed."""
    for _ in range(max(1, warmup)):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        fn()  # first launch outside capture on the side stream
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(reps):
                fn()
    torch.cuda.synchronize()
    replays = max(1, steps // reps)
    graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / (replays * reps), replays * reps


def kernel_suite(args, only):
    from talm_amd import qgroup, rmsnorm, rope, swiglu, workloads

    dev = "cuda"
    results = []

    def record(name, ms, count, bytes_=None, flops=None, config=""):
        entry = {"kernel": name, "config": config, "us": round(ms * 1e3, 3), "launches": count}
        if bytes_ is not None:
            gbs = bytes_ / (ms * 1e-3) / 1e9
            entry.update(bytes=int(bytes_), gbs=round(gbs, 1),
                         hbm_frac=round(gbs / HBM_PEAK_GBS, 4))
        if flops is not None:
            tf = flops / (ms * 1e-3) / 1e12
            entry.update(flops=int(flops), tflops=round(tf, 1),
                         mfma_frac=round(tf / FP16_PEAK_TFLOPS, 4))
        results.append(entry)
        print(f"[bench] {json.dumps(entry)}", flush=True)

    def want(name):
        return not only or name in only

    if "copy" in only:
        # calibration for the HBM byte counters: a plain 512 MiB device copy reads and writes
        # exactly 512 MiB per launch (run only when named explicitly)
        src = torch.empty(2**28, dtype=torch.float16, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        ms, cnt = graph_time_ms(lambda: dst.copy_(src), args.steps, args.warmup, args.reps)
        record("copy_512MiB", ms, cnt, bytes_=2 * 2**29, config="calibration")
        del src, dst

    if want("nf4_group"):
        d = workloads.nf4_layer()
        t = {k: d[k].to(dev) for k in ("packed", "absmax8", "code", "absmax2", "offset2")}
        out = torch.empty(d["n"], dtype=torch.float16, device=dev)
        n_rows = d["absmax8"].numel()

        def fn():
            qgroup.launch(t["packed"], t["absmax8"], t["code"], t["absmax2"], t["offset2"],
                          None, out, n_rows, 64, 256)

        ms, cnt = graph_time_ms(fn, args.steps, args.warmup, args.reps)
        # packed + absmax8 + absmax2 + offsets(7 x 4) + code + fp16 out
        algo = d["n"] // 2 + n_rows + 4 * t["absmax2"].numel() + 28 + 1024 + 2 * d["n"]
        record("nf4_group_dequant", ms, cnt, bytes_=algo, config="1: Qwen2.5-1.5B layer")

    d2 = workloads.norm_rope() if (want("addnorm_fwd") or want("addnorm_bwd")
                                   or want("rope")) else None
    if d2 is not None and (want("addnorm_fwd") or want("addnorm_bwd")):
        n, hdim = d2["n"], 1536
        x, br, w = d2["residual"].to(dev), d2["x"].to(dev), d2["weight"].to(dev)
        total = torch.empty_like(x)
        y = torch.empty_like(x)
        xhat = torch.empty_like(x)
        rstd = torch.empty(n, dtype=torch.float32, device=dev)
        dy, ds = d2["dy"].to(dev), d2["ds"].to(dev)
        dx = torch.empty_like(x)
        db = torch.empty_like(x)

        def fwd():
            rmsnorm.launch(x, w, y, xhat, rstd, 1e-6, 0, p=br, q=total)

        def bwd():
            rmsnorm.launch(dx, w, dy, xhat, rstd, 1e-6, 1, p=db, q=ds)

        fwd()
        if want("addnorm_fwd"):
            ms, cnt = graph_time_ms(fwd, args.steps, args.warmup, args.reps)
            record("add_rmsnorm_fwd", ms, cnt, bytes_=10 * n * hdim + 4 * n + 4 * hdim,
                   config=f"2: N={n}")
        if want("addnorm_bwd"):
            ms, cnt = graph_time_ms(bwd, args.steps, args.warmup, args.reps)
            record("add_rmsnorm_bwd", ms, cnt, bytes_=10 * n * hdim + 4 * n + 4 * hdim,
                   config=f"2: N={n}")

    if d2 is not None and want("rope"):
        n = d2["n"]
        qkv = torch.randn(n, 2048, device=dev).half()
        q = qkv[:, :1536].view(n, 12, 128)
        k = qkv[:, 1536:1792].view(n, 2, 128)
        cos, sin = d2["cos"].to(dev), d2["sin"].to(dev)

        def fn():
            rope.rope_(q, k, cos, sin, backward=False)

        ms, cnt = graph_time_ms(fn, args.steps, args.warmup, args.reps)
        record("rope_inplace", ms, cnt, bytes_=8192 * n, config=f"2: N={n}")

    if want("swiglu_fwd") or want("swiglu_bwd"):
        d3 = workloads.swiglu_inputs()
        gate, up, grad = (d3[k].to(dev) for k in ("gate", "up", "grad"))
        out = torch.empty_like(gate)
        dgate, dup = torch.empty_like(gate), torch.empty_like(up)
        n = gate.numel()
        if want("swiglu_fwd"):
            ms, cnt = graph_time_ms(lambda: swiglu.swiglu_fwd(gate, up, out), args.steps,
                                    args.warmup, args.reps)
            record("swiglu_fwd", ms, cnt, bytes_=6 * n, config="3: [2048, 8960]")
        if want("swiglu_bwd"):
            ms, cnt = graph_time_ms(lambda: swiglu.swiglu_bwd(grad, gate, up, dgate, dup),
                                    args.steps, args.warmup, args.reps)
            record("swiglu_bwd", ms, cnt, bytes_=10 * n, config="3: [2048, 8960]")
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
        wt = fused_head.transpose_weight(w16)  # built once per frozen weight, outside the timing

        def fn():
            torch.ops.talm.head_ce(h16, w16, wt, tt, vchunk, n_lab, group, *outs, ws)

        ms, cnt = graph_time_ms(fn, max(10, args.steps // 20), args.warmup, 4)
        flops = 2.0 * vocab * hdim * (n + n_lab)
        record("head_ce_fwd_bwd", ms, cnt, flops=flops,
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


def cpu_baseline_step(seconds):
    """The reference's eager path on the host cores, bounded: one decoder layer of the QLoRA
    model (fp32, forward + backward) on a config-5 token count, timed and scaled to 28 layers,
    plus the head + cross-entropy oracle on a row sample scaled to the token count."""
    import numpy as np

    from oracle import head as head_oracle
    from talm_amd import qlora_model

    torch.manual_seed(0)
    n_tok = 1280  # 4 rows of 128-512 tokens: the mean of config 5
    cfg = qlora_model.qwen2_config(num_hidden_layers=1)
    from transformers.models.qwen2.modeling_qwen2 import Qwen2DecoderLayer, Qwen2RotaryEmbedding

    layer = Qwen2DecoderLayer(cfg, 0).float()
    rot = Qwen2RotaryEmbedding(cfg)
    x = torch.randn(1, n_tok, cfg.hidden_size, requires_grad=True)
    pos = torch.arange(n_tok)[None]
    pe = rot(x, pos)
    mask = torch.full((n_tok, n_tok), float("-inf")).triu(1)[None, None]
    t0 = time.perf_counter()
    reps = 0
    while True:
        y = layer(x, attention_mask=mask, position_embeddings=pe, position_ids=pos)
        y.float().sum().backward()
        reps += 1
        if time.perf_counter() - t0 > seconds / 2:
            break
    layer_ms = (time.perf_counter() - t0) * 1e3 / reps
    rows = 16
    rng = np.random.default_rng(0)
    h = rng.standard_normal((rows, cfg.hidden_size)).astype(np.float16)
    w = (rng.standard_normal((cfg.vocab_size, cfg.hidden_size)) * 0.02).astype(np.float16)
    t = rng.integers(0, cfg.vocab_size, rows)
    t1 = time.perf_counter()
    head_oracle.head_ce(h, w, t, vchunk=8192)
    head_ms = (time.perf_counter() - t1) * 1e3 * n_tok / rows
    threads = torch.get_num_threads()
    return {"value": round(28 * layer_ms + head_ms, 1), "unit": "ms/step (estimated)",
            "cores": threads, "kind": "port",
            "sample": f"1 Qwen2.5-1.5B decoder layer fwd+bwd in fp32 PyTorch CPU eager on "
                      f"{n_tok} tokens ({reps} reps, {layer_ms:.0f} ms) x 28 layers + the head/CE "
                      f"oracle on {rows} rows x full vocabulary scaled to {n_tok} rows "
                      f"({head_ms:.0f} ms); {threads} threads, {os.cpu_count()} CPUs visible"}


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
    dominant = max(kernels, key=lambda e: e["us"]) if kernels else None
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
        line["cpu_baseline"] = (cpu_baseline_step(args.cpu_seconds) if step is not None
                                else cpu_baseline_nf4(args.cpu_seconds))
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
