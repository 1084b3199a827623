"""Which fast paths ran: host-side counters only (no sync, no kernel), after the reference's
solution/engaged.py:65-68 (`RAN`, `FELL_BACK`, `ON`) and its one-line summary (:128-146)."""

from collections import Counter

RAN = Counter()
FELL_BACK = Counter()
ON = set()


def line():
    """`[solution] engaged: name=ran/fallbacks ...` for every installed component."""
    names = sorted(ON | set(RAN) | set(FELL_BACK))
    parts = [f"{name}={RAN[name]}/{FELL_BACK[name]}" for name in names]
    return "[solution] engaged: " + " ".join(parts)


def reset():
    RAN.clear()
    FELL_BACK.clear()
