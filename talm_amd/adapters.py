"""The LoRA adapters' per-step device state: fp16 images of the fp32 adapter weights for the
MFMA kernels, and the AdamW step that keeps them current (§8 (f) 4 of the reference's plan:
solution/lora.py:57-137 keeps the fp16 copies; the reference leaves the optimizer to PyTorch).

`AdapterCopies` lays every registered fp32 weight's fp16 copy out in one flat fp16 buffer, and
for the q|k|v nodes with two adapters also A^T = [A_q^T | A_v^T] ([hidden, 32], the B operand of
the extra reduction step of the backward dX GEMM, which the node would otherwise build with a
concatenation and a transposed copy per layer and step). `talm_lora_mirror` writes all of them
in one launch into a fresh buffer — at the first use after an optimizer step or after a weight
changed (its storage or version counter), so copies saved by an earlier forward for its backward
stay as they were. A weight or pair seen for the first time is copied on its own with PyTorch
ops and joins the layout at the next refresh.

`AdapterAdamW` is AdamW (decoupled weight decay, bias-corrected moments) over the adapters in one
`talm_lora_adamw` launch per parameter group, which also writes the next forward's copies: the
post-step refresh disappears. It takes torch.amp.GradScaler's scale and inf flag on the device
(`_step_supports_amp_scaling`, as PyTorch's fused optimizers), so a step needs no host sync.
"""

import weakref

import torch

from . import _ops  # noqa: F401 - registers torch.ops.talm.*
from .engaged import RAN

_ALIGN = 8            # copies start on 16-byte boundaries
_COLS = 9             # int64 entries per tensor in the device table


def _key(param):
    return param.data_ptr(), param._version


def _pad(n):
    return (n + _ALIGN - 1) // _ALIGN * _ALIGN


class AdapterCopies:
    def __init__(self):
        self.params = []        # weakrefs to the registered fp32 weights, in registration order
        self.index = {}         # id(weight) -> registration position
        self.pairs = []         # tuples of positions whose transposes share one block
        self.pair_index = {}    # tuple of ids -> position in `pairs`
        self.layout = None      # (h_off per weight, (t_off, ld_t) per weight, size) of `buffer`
        self.table = None       # device int64 [weights, 9] of `layout` (optimizer columns 0)
        self.buffer = None      # flat fp16: copies of the current layout
        self.keys = []          # per weight: the key its copy in `buffer` was made from
        # id(weight) or pair ids -> (weakref(s), key(s), copy) made outside a layout; the
        # weakrefs tell a live weight from a freed one whose id and storage a new one reuses
        self.loose = {}
        self.adopted_by = None  # the optimizer whose step wrote `buffer`
        # rewrite `buffer` in place instead of a fresh buffer per refresh / optimizer step: for a
        # step replayed from a HIP graph, whose forward reads the copies at the address it was
        # captured with. The caller guarantees that every backward reading the copies has run
        # before the next optimizer step (a training loop does).
        self.in_place = False

    # -- registration and layout ------------------------------------------------------------
    def _position(self, param):
        pos = self.index.get(id(param))
        if pos is None or self.params[pos]() is not param:
            pos = len(self.params)
            self.params.append(weakref.ref(param))
            self.index[id(param)] = pos
            self.layout = None
        return pos

    def _alive(self):
        return all(ref() is not None for ref in self.params)

    def _build_layout(self, device):
        if not self._alive():  # a weight was freed: start the registry over
            live = [ref for ref in self.params if ref() is not None]
            pair_ids = [tuple(id(self.params[p]()) for p in pair) for pair in self.pairs
                        if all(self.params[p]() is not None for p in pair)]
            self.params, self.index = live, {id(ref()): i for i, ref in enumerate(live)}
            self.pairs = [tuple(self.index[i] for i in ids) for ids in pair_ids]
            self.pair_index = {ids: k for k, ids in enumerate(pair_ids)}
        weights = [ref() for ref in self.params]
        h_off, size = [], 0
        for w in weights:
            h_off.append(size)
            size += _pad(w.numel())
        t_of = [(-1, 0)] * len(weights)
        for pair in self.pairs:
            width = sum(weights[p].shape[0] for p in pair)
            col = 0
            for p in pair:
                t_of[p] = (size + col, width)
                col += weights[p].shape[0]
            size += _pad(weights[pair[0]].shape[1] * width)
        rows = [[w.data_ptr(), w.numel(), w.shape[1], h, t, ld, 0, 0, 0]
                for w, h, (t, ld) in zip(weights, h_off, t_of)]
        self.table = torch.tensor(rows, dtype=torch.int64).to(device)
        self.layout = (h_off, t_of, size)

    def entries(self, params):
        """(h_off, t_off, ld_t) of each weight in the current layout (-1: not laid out)."""
        h_off, t_of, _size = self.layout
        out = []
        for p in params:
            pos = self.index.get(id(p))
            if pos is None or pos >= len(h_off) or self.params[pos]() is not p:
                out.append((-1, -1, 0))
            else:
                out.append((h_off[pos], t_of[pos][0], t_of[pos][1]))
        return out

    def max_numel(self):
        return max((ref().numel() for ref in self.params), default=0)

    # -- the copies -----------------------------------------------------------------------------
    @torch.no_grad()
    def refresh(self, device):
        if self.layout is None or not self._alive():
            self._build_layout(device)
        buffer = self.reusable(device)
        torch.ops.talm.lora_mirror(self.table, len(self.params), self.max_numel(), buffer)
        self.adopt(buffer, None)
        RAN["lora_cast"] += 1

    def reusable(self, device):
        """The buffer the next copies go to: the current one in place mode when it has the
        layout's size, else a fresh one."""
        size = max(self.layout[2], 1)
        b = self.buffer
        if self.in_place and b is not None and b.numel() == size and b.device == device:
            return b
        return torch.empty(size, dtype=torch.float16, device=device)

    def adopt(self, buffer, optimizer):
        """`buffer` holds the copies of the current layout, made from the weights as they are."""
        self.buffer = buffer
        self.keys = [_key(ref()) for ref in self.params]
        self.loose = {}
        self.adopted_by = optimizer

    def invalidate(self, optimizer=None, *_args, **_kwargs):
        if optimizer is not None and optimizer is self.adopted_by:
            self.adopted_by = None  # its step wrote the copies
            return
        if self.in_place:
            self.keys = []  # stale: the next use rewrites the same buffer
        else:
            self.buffer = None
        self.loose = {}

    def _current(self, pos, param):
        return (self.buffer is not None and self.layout is not None and pos < len(self.keys)
                and self.keys[pos] == _key(param))

    def _known(self, param):
        pos = self.index.get(id(param))
        return pos is not None and self.params[pos]() is param

    def half(self, param):
        """fp16 copy of an fp32 weight (rows x cols, contiguous)."""
        known = self._known(param)
        pos = self._position(param)
        if known and not self._current(pos, param):
            self.refresh(param.device)  # one launch for every registered weight
        if self._current(pos, param):
            h_off = self.layout[0][pos]
            return self.buffer[h_off:h_off + param.numel()].view(param.shape)
        key = _key(param)
        hit = self.loose.get(id(param))
        if hit is None or hit[0]() is not param or hit[1] != key:
            hit = (weakref.ref(param), key, param.detach().to(torch.float16))
            self.loose[id(param)] = hit
        return hit[2]

    def pair_t(self, params):
        """[cols, sum of rows] fp16: the weights' transposes side by side (A^T of a q|k|v node's
        adapters, each A [16, cols])."""
        known = all(self._known(p) for p in params)
        positions = tuple(self._position(p) for p in params)
        ids = tuple(id(p) for p in params)
        k = self.pair_index.get(ids)
        if k is not None and self.pairs[k] != positions:  # ids of freed weights, reused
            k = None
        if k is None or not known:
            if k is None:
                self.pair_index[ids] = len(self.pairs)
                self.pairs.append(positions)
            self.layout = None
        else:
            if not all(self._current(pos, p) for pos, p in zip(positions, params)):
                self.refresh(params[0].device)
            t_off, width = self.layout[1][positions[0]]
            if t_off >= 0 and all(self._current(pos, p) for pos, p in zip(positions, params)):
                cols = params[0].shape[1]
                return self.buffer[t_off:t_off + cols * width].view(cols, width)
        keys = tuple(_key(p) for p in params)
        hit = self.loose.get(ids)
        if hit is None or any(r() is not p for r, p in zip(hit[0], params)) or hit[1] != keys:
            hit = (tuple(weakref.ref(p) for p in params), keys,
                   torch.cat([p.detach() for p in params], 0).t().to(torch.float16).contiguous())
            self.loose[ids] = hit
        return hit[2]


COPIES = AdapterCopies()


class AdapterAdamW(torch.optim.Optimizer):
    """AdamW on fp32 CUDA parameters in one `talm_lora_adamw` launch per parameter group, writing
    the fp16 copies of `COPIES` for the next forward in the same pass."""

    _step_supports_amp_scaling = True

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2,
                 copies=COPIES):
        if not 0.0 <= lr or not 0.0 < eps or not all(0.0 <= b < 1.0 for b in betas):
            raise ValueError(f"AdapterAdamW: lr {lr}, betas {betas}, eps {eps}")
        super().__init__(params, dict(lr=lr, betas=tuple(betas), eps=eps,
                                      weight_decay=weight_decay))
        self.copies = copies
        for group in self.param_groups:
            for p in group["params"]:
                if not (p.is_cuda and p.dtype == torch.float32 and p.is_contiguous()
                        and p.dim() == 2):
                    raise ValueError("AdapterAdamW: 2-D contiguous fp32 CUDA parameters")
        self._pinned = {}

    def _state(self, group, params, device):
        steps = group.get("_talm_steps")
        if steps is None:
            steps = torch.zeros(2, dtype=torch.float32, device=device)
            group["_talm_steps"], group["_talm_flip"] = steps, 0
        for p in params:
            st = self.state[p]
            if "exp_avg" not in st:
                st["exp_avg"] = torch.zeros_like(p)
                st["exp_avg_sq"] = torch.zeros_like(p)
        return steps

    def _table(self, key, rows, device):
        """Device int64 [rows, 9] uploaded from pinned host memory: two host / device pairs per
        group used in turn, a host array rewritten only after its previous upload is done."""
        st = self._pinned.get(key)
        n = len(rows)
        if st is None or st["host"][0].shape[0] != n:
            st = {"host": [torch.empty(n, _COLS, dtype=torch.int64, pin_memory=True)
                           for _ in range(2)],
                  "dev": [torch.empty(n, _COLS, dtype=torch.int64, device=device)
                          for _ in range(2)],
                  "event": [None, None], "next": 0}
            self._pinned[key] = st
        i = st["next"]
        st["next"] = 1 - i
        if st["event"][i] is not None:
            st["event"][i].synchronize()
        st["host"][i].numpy()[:] = rows
        st["dev"][i].copy_(st["host"][i], non_blocking=True)
        event = torch.cuda.Event()
        event.record()
        st["event"][i] = event
        return st["dev"][i]

    def _group_launch_args(self, gi, group, params, buffer):
        """(table, n, max_numel, step_in, step_out, buffer) of one group's launch: the device
        table of its tensors (weight, sizes, copy offsets, gradient, moments) and the step
        counters; the adapters' copy layout is built on first use."""
        copies = self.copies
        device = params[0].device
        if copies.layout is None or not copies._alive():
            copies._build_layout(device)
        if buffer is None:
            buffer = copies.reusable(device)
        steps = self._state(group, params, device)
        rows = []
        for p, (h, t, ld) in zip(params, copies.entries(params)):
            g = p.grad
            if g.dtype != torch.float32 or not g.is_contiguous() or g.shape != p.shape:
                raise ValueError("AdapterAdamW: gradients must be contiguous fp32")
            st = self.state[p]
            rows.append([p.data_ptr(), p.numel(), p.shape[1], h, t, ld, g.data_ptr(),
                         st["exp_avg"].data_ptr(), st["exp_avg_sq"].data_ptr()])
        table = self._table(gi, rows, device)
        flip = group["_talm_flip"]
        return (table, len(params), max(p.numel() for p in params), steps[flip:flip + 1],
                steps[1 - flip:2 - flip], buffer)

    def _after_group(self, group, params, step_out):
        group["_talm_flip"] = 1 - group["_talm_flip"]
        for p in params:
            self.state[p]["step"] = step_out
        RAN["adapter_adamw"] += 1

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        grad_scale = getattr(self, "grad_scale", None)
        found_inf = getattr(self, "found_inf", None)
        copies = self.copies
        registered = {id(ref()) for ref in copies.params if ref() is not None}
        covered = set()
        buffer = None
        for gi, group in enumerate(self.param_groups):
            params = [p for p in group["params"] if p.grad is not None]
            if not params:
                continue
            table, n, max_numel, step_in, step_out, buffer = self._group_launch_args(
                gi, group, params, buffer)
            covered.update(id(p) for p in params)
            beta1, beta2 = group["betas"]
            torch.ops.talm.lora_adamw(table, n, max_numel, float(group["lr"]), beta1, beta2,
                                      group["eps"], group["weight_decay"], step_in, step_out,
                                      grad_scale, found_inf, buffer)
            self._after_group(group, params, step_out)
        if buffer is not None and registered and registered <= covered:
            copies.adopt(buffer, self)
        return loss

    @torch.no_grad()
    def fused_tail(self, scaler, max_norm):
        """`scaler.unscale_(self)`, `clip_grad_norm_(params, max_norm)` and `scaler.step(self)`
        in three launches (talm_lora_grad_norm, talm_lora_adamw_clipped): the gradients are not
        rewritten, the step reads them unscaled and clipped as those calls would leave them, and
        is skipped when one is not finite. The scaler is left as `scaler.step` leaves it (this
        step's inf flag recorded, ready for `scaler.update()`). Returns the gradients' total
        norm (a device scalar), or None when it does not apply (one parameter group, every
        parameter with a gradient, an enabled scaler that has scaled this step's loss and not
        yet unscaled): the caller then runs the three calls."""
        from torch.amp.grad_scaler import OptState

        if len(self.param_groups) != 1 or not scaler.is_enabled():
            return None
        scale = getattr(scaler, "_scale", None)
        states = getattr(scaler, "_per_optimizer_states", None)
        if scale is None or states is None or states[id(self)]["stage"] is not OptState.READY:
            return None
        group = self.param_groups[0]
        params = list(group["params"])
        if not params or any(p.grad is None for p in params):
            return None
        copies = self.copies
        registered = {id(ref()) for ref in copies.params if ref() is not None}
        table, n, max_numel, step_in, step_out, buffer = self._group_launch_args(
            0, group, params, None)
        device = params[0].device
        ws = torch.empty(_ops.lora_grad_norm_workspace_bytes(n, max_numel), dtype=torch.uint8,
                         device=device)
        stats = torch.empty(4, dtype=torch.float32, device=device)
        torch.ops.talm.lora_grad_norm(table, n, max_numel, scale.reshape(1), float(max_norm), ws,
                                      stats)
        beta1, beta2 = group["betas"]
        torch.ops.talm.lora_adamw_clipped(table, n, max_numel, float(group["lr"]), beta1, beta2,
                                          group["eps"], group["weight_decay"], step_in, step_out,
                                          stats[0:1], stats[1:3], buffer)
        self._after_group(group, params, step_out)
        if registered and registered <= {id(p) for p in params}:
            copies.adopt(buffer, self)
            copies.adopted_by = None  # what the step's post hook (`invalidate`) would leave
        self._opt_called = True  # an optimizer step ran (the schedule's order check)
        state = states[id(self)]
        state["found_inf_per_device"] = {device: stats[0:1]}
        state["stage"] = OptState.STEPPED
        RAN["fused_tail"] += 1
        return stats[3]
