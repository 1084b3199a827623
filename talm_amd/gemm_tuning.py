"""A measured hipBLASLt solution table for the decoder's fp16 GEMMs (o_proj, gate|up, down).

hipBLASLt's heuristic picks one solution per shape from its own model; for the few products a
Qwen2.5-1.5B training step runs, every supported solution can simply be timed. `tune()` times
them (torch.ops.talm.gemm_tune) for each product form at token counts in buckets of 128, and
writes the winners that beat the heuristic's choice by at least 3 % to gemm_algos.json next to
this file; `load()` (called by `apply()`) installs that table into torch.ops.talm.gemm /
gemm_ex, which fall back to the heuristic for every product the table does not name or whose
named solution hipBLASLt rejects for the exact shape. The table is only used with the hipBLASLt
version and GPU architecture it was measured on. SOLUTION_DISABLE_GEMM_TABLE=1 leaves it out.

The reference runs these products through PyTorch's F.linear / mm (bitsandbytes dequant, then
cuBLAS) with cuBLAS's own heuristic (solution/lora.py:151-231, solution/__init__.py:229-408).

    python -m talm_amd.gemm_tuning --out talm_amd/gemm_algos.json   # on the GPU
"""

import argparse
import json
import os
from pathlib import Path

import torch

from . import _ops  # noqa: F401 - registers torch.ops.talm

TABLE = Path(__file__).resolve().parent / "gemm_algos.json"
BUCKET = 128
N_MAX = 2176
GAIN = 0.97
HIDDEN, INTER = 1536, 8960


def product_forms():
    """(name, trans_a, trans_b, m, k, lda, ldb, ldd) of each hipBLASLt product of a step, in the
    column-major terms of gemm_ex (n = token count)."""
    h, i = HIDDEN, INTER
    return (
        ("o_fwd", 1, 0, h, h, h, h, h),
        ("o_dx", 0, 0, h, h, h, h, h),
        ("gate_up_fwd", 1, 0, 2 * i, h, h, h, 2 * i),
        ("down_fwd", 1, 0, h, i, i, i, h),
        ("down_dx", 0, 0, i, h, i, h, i),
        ("gate_up_dx", 0, 0, h, 2 * i, h, 2 * i, h),
        # the input gradients in the forward's form, on the group's transposed weights
        ("down_dx_t", 1, 0, i, h, h, h, i),
        ("gate_up_dx_t", 1, 0, h, 2 * i, 2 * i, 2 * i, h),
    )


def _arch():
    return torch.cuda.get_device_properties(0).gcnArchName.split(":")[0]


def tune(reps=20, n_max=N_MAX, bucket=BUCKET, log=print):
    """Time every supported solution of each product form at the middle of each token bucket;
    return the table (a JSON-able dict)."""
    device = torch.device("cuda", 0)
    g = torch.Generator(device).manual_seed(0)
    rows, report = [], []
    for name, ta, tb, m, k, lda, ldb, ldd in product_forms():
        for lo in range(bucket, n_max, bucket):
            hi = lo + bucket
            n = lo + bucket // 2
            a = torch.randn((m if ta else k) * lda, device=device, generator=g).half()
            b = torch.randn((k if tb else n) * ldb, device=device, generator=g).half()
            d = torch.empty(n * ldd, device=device, dtype=torch.float16)
            best, best_us, heur, heur_us = torch.ops.talm.gemm_tune(
                a, ta, b, tb, d, m, n, k, lda, ldb, ldd, reps).tolist()
            report.append({"form": name, "n": n, "best": int(best), "best_us": best_us,
                           "heuristic": int(heur), "heuristic_us": heur_us})
            log(f"{name:12s} n={n:5d} best {int(best):7d} {best_us:8.2f} us   "
                f"heuristic {int(heur):7d} {heur_us:8.2f} us")
            if best >= 0 and (heur_us < 0 or best_us < GAIN * heur_us) and int(best) != int(heur):
                rows.append([ta, tb, m, k, lo, hi, int(best)])
    return {"hipblaslt": int(torch.ops.talm.gemm_lib_version()), "arch": _arch(), "rows": rows,
            "measured": report}


def load(path=TABLE):
    """Install the table when it was measured with this hipBLASLt and architecture; an empty
    table (hipBLASLt's heuristic for every product) otherwise. Returns the number of rows."""
    rows = []
    if os.environ.get("SOLUTION_DISABLE_GEMM_TABLE") != "1" and Path(path).exists():
        table = json.loads(Path(path).read_text())
        if table.get("hipblaslt") == int(torch.ops.talm.gemm_lib_version()) \
                and table.get("arch") == _arch():
            rows = table["rows"]
    t = torch.tensor(rows, dtype=torch.int64).reshape(-1, 7)
    torch.ops.talm.gemm_algo_table(t)
    return len(rows)


def main(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--out", default=str(TABLE))
    parser.add_argument("--reps", type=int, default=20)
    args = parser.parse_args(argv)
    table = tune(reps=args.reps, log=lambda s: print(s, flush=True))
    Path(args.out).write_text(json.dumps(table, indent=1) + "\n")
    print(f"{len(table['rows'])} rows -> {args.out}", flush=True)


if __name__ == "__main__":
    main()
