"""The QLoRA training step replayed from HIP graphs, one graph per token bucket.

`qlora_model.Trainer.step` issues about 900 kernels per step from Python: autograd nodes, module
calls and the C++ op layer's launches. On MI355X that took about 21 ms of host time per step,
against about 20 ms of GPU time, so the host set the step time and no faster kernel could lower
it. `GraphedTrainer` captures the forward and backward of the step once per bucket of
`bucket` packed tokens and then replays it, one graph launch per step:

- the batch is packed on the device into exactly `n_bucket` rows (`unpad.static_tokens`, read
  by the causal-LM patch): the real tokens first, as in eager packing, then a pad sequence
  labelled -100 that attends only to itself. Its loss and every gradient through it are exactly
  zero, so the step computes the same values as the eager packing of the same batch. The only
  difference is rounding where a library GEMM picks another algorithm for the larger row count;
- the head takes every row as a gradient row, with no labelled-first count read on the host;
- the batch tensors are copied into the static input buffers the graph reads;
- the LoRA gradients live in one set of buffers shared by every graph, so 97 buckets hold one
  gradient set, not 97. The q|k|v nodes write each adapter weight's gradient straight into its
  buffer (`fused_proj.GRAD_INTO`: one contribution per weight and backward, so the buffers need
  no clearing and autograd adds nothing: about 230 fill and add launches fewer per step). That
  holds only if those nodes are a weight's ONLY contribution. The capture watches for any other:
  a weight no node wrote, a weight two nodes wrote (the second write would drop the first), or
  autograd accumulating into a weight's buffer (another path to the weight, such as a penalty
  term on it in the loss: it would add onto the buffer's stale contents). On any of them the
  bucket, and every later one, is captured again the general way: the graph zeroes the buffers
  (fill kernels) and the backward accumulates into them. They are handed to the parameters after
  each replay.

The optimizer tail stays eager: GradScaler unscale and update, clipping, `AdapterAdamW` and the
learning-rate schedule. It is about ten launches, and their host cost overlaps the graph's GPU
time. `AdapterAdamW` rewrites the adapters' fp16 copies in place (`COPIES.in_place`), at the
address the captured forward reads. The graphs share one memory pool and run one at a time on
one stream. A tensor a replay leaves behind (loss, gradients) is read before the next replay.

Capture needs a warmed-up trainer (`warm_steps` eager steps: optimizer state, GradScaler
scale, the head's transposed weight, hipBLASLt plans). `prepare(lo, hi)` captures every bucket
of a token range ahead of time, like the reference's kernel warm-up (solution/warmup.py); a
bucket met for the first time is captured on the spot.
"""

import time

import torch

from . import fused_proj, patches, unpad
from .adapters import COPIES, AdapterAdamW

_BATCH_KEYS = ("input_ids", "attention_mask", "labels")


class GraphedTrainer:
    """Wraps a `qlora_model.Trainer` whose optimizer is `AdapterAdamW` and whose model runs the
    patched path (`apply()`): `step(batch, next_batch)` as the trainer's, replayed from graphs."""

    def __init__(self, trainer, bucket=16, warm_steps=2):
        if not isinstance(trainer.opt, AdapterAdamW):
            raise ValueError("GraphedTrainer: the trainer's optimizer must be AdapterAdamW")
        if bucket < 1:
            raise ValueError(f"GraphedTrainer: bucket {bucket}")
        self.trainer = trainer
        self.bucket = int(bucket)
        self.warm_steps = int(warm_steps)
        self.steps = 0
        self.static = None
        self.graphs = {}           # bucket -> (graph, loss, gradients, per-token metrics)
        self.pool = None
        self.grads = None          # the LoRA gradient buffers every graph writes
        self.direct_grads = True   # the nodes write them (False: zero, then accumulate)
        self.capture_seconds = 0.0
        self.replays = 0
        COPIES.in_place = True

    # -- batches ----------------------------------------------------------------------------------
    def n_tokens(self, batch):
        """Real tokens of a right-padded batch: from the statistics `unpad.prefetch` copied to the
        host a step ahead, or one host sync for a batch that was not prefetched."""
        mask, labels = batch["attention_mask"], batch["labels"]
        values = unpad.take_prefetched(mask, labels)
        if values is None:
            values = unpad._row_values(mask).tolist()
        return int(sum(values[:mask.shape[0]]))

    def bucket_of(self, n_tokens):
        return max(self.bucket, -(-int(n_tokens) // self.bucket) * self.bucket)

    def _stage(self, batch):
        if self.static is None:
            self.static = {k: torch.empty_like(batch[k]) for k in _BATCH_KEYS}
        for k in _BATCH_KEYS:
            dst, src = self.static[k], batch[k]
            if src.shape != dst.shape or src.dtype != dst.dtype or src.device != dst.device:
                raise ValueError(f"GraphedTrainer: batch '{k}' {tuple(src.shape)} {src.dtype} "
                                 f"differs from the captured {tuple(dst.shape)} {dst.dtype}")
            dst.copy_(src, non_blocking=True)

    # -- graphs -----------------------------------------------------------------------------------
    def capture(self, n_bucket):
        """Capture the forward + backward of a step packed into `n_bucket` rows."""
        t = self.trainer
        if self.static is None or self.steps < self.warm_steps:
            raise RuntimeError("GraphedTrainer: capture after the warm-up steps")
        n_bucket = int(n_bucket)
        b, s = self.static["attention_mask"].shape
        if n_bucket % self.bucket or not 0 < n_bucket < b * s + self.bucket:
            raise ValueError(f"GraphedTrainer: bucket {n_bucket} for a [{b}, {s}] batch")
        start = time.perf_counter()
        held = [p.grad for p in t.params]
        if self.grads is None:  # outside the graphs' pool: they outlive every capture
            self.grads = [torch.zeros_like(p) for p in t.params]
        for p, g in zip(t.params, self.grads):
            p.grad = g
        graph = torch.cuda.CUDAGraph()
        direct = self.direct_grads
        accumulated, hooks = set(), []
        if direct:
            fused_proj.GRAD_INTO.update((id(p), (p, g)) for p, g in zip(t.params, self.grads))
            fused_proj.GRAD_WRITTEN.clear()
            fused_proj.GRAD_TWICE.clear()
            # host-side callbacks (they record, they launch nothing): autograd is about to
            # accumulate a gradient into a parameter's .grad, i.e. some contribution did not
            # come through direct delivery (a node that delivered directly hands autograd an
            # undefined gradient, which reaches the hook as None)
            hooks = [p.register_hook(lambda g, i=id(p): None if g is None else accumulated.add(i))
                     for p in t.params]
        try:
            # the pad sequence is shorter than one bucket step (a full bucket when no token is
            # real)
            with unpad.static_tokens(n_bucket, max_pad=self.bucket):
                with torch.cuda.graph(graph, pool=self.pool):
                    if not direct:
                        for g in self.grads:
                            g.zero_()
                    with torch.autocast("cuda", dtype=torch.float16):
                        out = t.model(**self.static)
                    t.backward(out.loss)
        finally:
            fused_proj.GRAD_INTO.clear()
            for h in hooks:
                h.remove()
        if self.pool is None:
            self.pool = graph.pool()
        if direct and (any(id(p) not in fused_proj.GRAD_WRITTEN for p in t.params)
                       or fused_proj.GRAD_TWICE or accumulated):
            # some gradient went through autograd into an uncleared buffer, or one weight got two
            # direct writes: capture this bucket (and every later one) the general way. The
            # discarded graph is the only user of the memory pool when no other graph was kept:
            # the pool then goes with it, and the next capture starts a new one
            if not self.graphs:
                self.pool = None
            del graph, out
            self.direct_grads = False
            for p, g in zip(t.params, held):
                p.grad = g
            self.capture_seconds += time.perf_counter() - start
            return self.capture(n_bucket)
        # the backward wrote or accumulated into the shared buffers in place (autograd replaces
        # a parameter's .grad only when it cannot add into it)
        if any(p.grad is not g for p, g in zip(t.params, self.grads)):
            raise RuntimeError("GraphedTrainer: the backward did not accumulate into the shared "
                               "gradient buffers")
        grads = self.grads
        for p, g in zip(t.params, held):
            p.grad = g
        # the per-token metrics (patches.LAST_STEP) this graph writes on every replay: kept with
        # the graph, so their memory stays this graph's (no other capture in the shared pool
        # reuses it) and a replay of this bucket can hand them out again
        metrics = patches.LAST_STEP[-1] if patches.LAST_STEP else None
        entry = (graph, out.loss.detach(), grads, metrics)
        self.graphs[n_bucket] = entry
        self.capture_seconds += time.perf_counter() - start
        return entry

    def prepare(self, lo_tokens, hi_tokens):
        """Capture every bucket that a batch of lo_tokens..hi_tokens real tokens can fall in."""
        for nb in range(self.bucket_of(lo_tokens), self.bucket_of(hi_tokens) + 1, self.bucket):
            if nb not in self.graphs:
                self.capture(nb)

    def close(self):
        """Drop the graphs and their pool; the adapters' copies go back to fresh buffers."""
        self.graphs.clear()
        self.pool = None
        self.grads = None
        self.static = None
        COPIES.in_place = False

    # -- the step ---------------------------------------------------------------------------------
    def step(self, batch, next_batch=None):
        """One optimizer step; returns the loss tensor (not synchronized)."""
        t = self.trainer
        if self.steps < self.warm_steps:
            loss = t.step(batch, next_batch)
            self._stage(batch)
            self.steps += 1
            return loss
        n = self.n_tokens(batch)
        if next_batch is not None:
            unpad.prefetch(next_batch["attention_mask"], next_batch["labels"])
        self._stage(batch)
        nb = self.bucket_of(n)
        entry = self.graphs.get(nb) or self.capture(nb)
        graph, loss, grads, metrics = entry
        graph.replay()
        self.replays += 1
        patches.LAST_STEP.clear()
        if metrics is not None:
            patches.LAST_STEP.append(metrics)
        for p, g in zip(t.params, grads):
            p.grad = g
        t.optimizer_tail()
        self.steps += 1
        return loss.clone()
