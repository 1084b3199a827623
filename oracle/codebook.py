"""The NF4 level table from its published construction (test infrastructure).

The 16 NormalFloat levels are the ones hard-coded in the reference (solution/qgroup.py:60-63,
solution/nf4_dequant.py:32-35). QLoRA (Dettmers et al., 2023, section 3 and appendix E) builds
them from quantiles of N(0, 1): 8 positive quantiles at probabilities evenly spaced from
0.9677083 down to 0.5 (exclusive), 7 negative ones likewise, and an exact zero, normalized so
that the largest magnitude is 1. `nf4_levels_from_quantiles` restates that construction in
float64; the tests check the hard-coded table against it.

The second-level code table of the double quantization (bitsandbytes' dynamic map) is not part
of the oracle: it is an input of every kernel and of every oracle function, written once as the
committed fixture tests/golden/dynamic_map.txt by tests/golden/make_golden.py, which runs
bitsandbytes' published create_dynamic_map.
"""

import numpy as np

NF4_LEVELS = np.array([
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0], dtype=np.float32)


def nf4_levels_from_quantiles(offset=0.9677083):
    """QLoRA's NF4 construction in float64 (7 negative quantiles, 0, 8 positive, max-normalized)."""
    from scipy.stats import norm

    positive = norm.ppf(np.linspace(offset, 0.5, 9)[:-1])
    negative = -norm.ppf(np.linspace(offset, 0.5, 8)[:-1])
    values = np.sort(np.concatenate([positive, [0.0], negative]))
    return values / values.max()
