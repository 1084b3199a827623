"""A static check of LDS read results in gfx950 assembly (test infrastructure).

A `ds_read*` writes its destination VGPRs when the LDS returns the data, some cycles after the
instruction issues; the hardware does not interlock on them. Code must execute an
`s_waitcnt lgkmcnt(N)` that covers the read before any instruction touches those registers. The
compiler inserts such waits for the reads it emits itself. The attention kernels also issue
reads through inline assembly that the compiler does not track: they are waited for explicitly,
and nothing may read or move their destination registers before that wait, not even a copy made
by the register allocator.

`violations(body)` scans a kernel body in program order. It keeps the outstanding LGKM operations
(LDS and scalar-memory loads) and retires them at each `s_waitcnt lgkmcnt(N)`: LDS operations
return in order, so an LDS read is complete once more than N LDS operations were issued from it
on; scalar loads may return out of order and are retired only by `lgkmcnt(0)`. Any other
instruction that names a VGPR / AGPR of a read still outstanding is reported. The scan is linear
(labels do not reset the state), so it is conservative at control-flow joins.
"""

import re

_REG = re.compile(r"\b([va])(?:\[(\d+):(\d+)\]|(\d+)\b)")
_WAIT = re.compile(r"\bs_waitcnt\b(.*)")
_LGKM = re.compile(r"lgkmcnt\((\d+)\)")


def _regs(text):
    out = set()
    for kind, lo, hi, one in _REG.findall(text):
        if one:
            out.add((kind, int(one)))
        else:
            out.update((kind, r) for r in range(int(lo), int(hi) + 1))
    return out


def _instructions(body):
    for line in body.splitlines():
        line = line.split(";", 1)[0].strip()
        if not line or line.startswith(".") or line.endswith(":"):
            continue
        yield line


def violations(body):
    """[(instruction index, instruction, the read it touches)] for one kernel body."""
    pending = []  # [kind ("ds" | "smem"), registers written, instruction text]
    found = []
    for i, ins in enumerate(_instructions(body)):
        op = ins.split(None, 1)[0]
        wait = _WAIT.match(ins)
        if wait:
            m = _LGKM.search(wait.group(1))
            if m is not None:
                n = int(m.group(1))
                if n == 0:
                    pending = []
                else:
                    keep = []
                    for j, entry in enumerate(pending):
                        later_ds = sum(1 for e in pending[j:] if e[0] == "ds")
                        if entry[0] == "smem" or later_ds <= n:
                            keep.append(entry)
                    pending = keep
            continue
        operands = ins[len(op):]
        touched = _regs(operands)
        for kind, regs, text in pending:
            if kind == "ds" and regs & touched:
                found.append((i, ins, text))
        if op.startswith("ds_"):
            dest = set()
            if op.startswith(("ds_read", "ds_load")) or "_rtn_" in op:
                dest = _regs(operands.split(",", 1)[0])
            pending.append(("ds", dest, ins))
        elif op.startswith("s_load") or op.startswith("s_buffer_load"):
            pending.append(("smem", set(), ins))
    return found


_VM = re.compile(r"vmcnt\((\d+)\)")


def drained_prefetches(body):
    """[(instruction index, LDS read, the wait before it)] where a vmcnt wait forces a
    direct-to-LDS load (`buffer_load_* ... lds`) issued since the last `s_barrier` to complete
    before an LDS read of the same window.

    A ring keeps the next tile's direct-to-LDS loads in flight while the wavefront reads the
    current tile; the waits it needs sit before the barrier that publishes a tile. A compiler
    that cannot tell the slot being filled from the slot being read inserts a vmcnt wait right
    before the reads instead, which waits for the prefetch too (the ring then runs one memory
    round trip per tile). Vector-memory operations complete in order (on gfx9 vmcnt counts loads
    and stores), so `s_waitcnt vmcnt(N)` completes all but the newest N: it drains the window's
    first prefetch when N is below the number of vector-memory operations issued since it.
    Linear scan: a barrier ends the window, labels do not."""
    found = []
    since_dma = None  # vector-memory operations issued since the window's first prefetch
    drained = None
    for i, ins in enumerate(_instructions(body)):
        op = ins.split(None, 1)[0]
        if op == "s_barrier":
            since_dma = drained = None
        elif op.startswith(("buffer_", "global_", "flat_")) and not op.startswith(
                ("buffer_wbl2", "buffer_inv", "buffer_gl")):
            if since_dma is None and op.startswith("buffer_load") and ins.rstrip().endswith(" lds"):
                since_dma = 0
            if since_dma is not None:
                since_dma += 1
        elif op == "s_waitcnt" and since_dma is not None:
            m = _VM.search(ins)
            if m is not None and int(m.group(1)) < since_dma:
                drained = ins
        elif op.startswith(("ds_read", "ds_load")) and drained is not None:
            found.append((i, ins, drained))
    return found


def kernel_bodies(asm_text, pattern):
    """{symbol: body} of the kernels whose mangled names match `pattern`."""
    bodies = re.findall(r"^(_Z\w+):[^\n]*\n(.*?)^\.Lfunc_end", asm_text, flags=re.S | re.M)
    return {name: body for name, body in bodies if re.search(pattern, name)}
