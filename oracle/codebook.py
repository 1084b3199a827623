"""The two NF4 tables from their published constructions (test infrastructure).

- The 16 NormalFloat levels are the ones hard-coded in the reference (solution/qgroup.py:60-63,
  solution/nf4_dequant.py:32-35). QLoRA (Dettmers et al., 2023, section 3 and appendix E)
  builds them from quantiles of N(0, 1): 8 positive quantiles at probabilities evenly spaced
  from 0.9677083 down to 0.5 (exclusive), 7 negative ones likewise, and an exact zero, normalized
  so that the largest magnitude is 1. `nf4_levels_from_quantiles` restates that construction in
  float64; the tests check the hard-coded table against it.
- The second-level code table of the double quantization is bitsandbytes' dynamic map
  (`create_dynamic_map(signed=True)`, Dettmers et al., 8-bit optimizers, 2022: dynamic tree
  quantization): for each of 7 decades 10^(i-6), i = 0..6, the midpoints of 2^i + 1 points evenly
  spaced on [0.1, 1] times the decade, both signs, plus 0 and 1, sorted. The reference only
  passes that table through (solution/qgroup.py:82, :161); bitsandbytes itself is not vendored
  in the reference tree, so these values are parity unpinned. They are an input of the kernels.
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


def dynamic_map(signed=True, max_exponent_bits=7, total_bits=8):
    """bitsandbytes' dynamic map (the double-quant code table), float32 [256], sorted."""
    data = []
    non_sign_bits = total_bits - 1
    for i in range(max_exponent_bits):
        items = 2 ** (i + non_sign_bits - max_exponent_bits) + 1 if signed \
            else 2 ** (i + non_sign_bits - max_exponent_bits + 1) + 1
        boundaries = np.linspace(0.1, 1, items, dtype=np.float32)
        means = (boundaries[:-1] + boundaries[1:]) / np.float32(2.0)
        decade = np.float32(10.0 ** (-(max_exponent_bits - 1) + i))
        data += list((decade * means).astype(np.float32))
        if signed:
            data += list((-decade * means).astype(np.float32))
    data += [0.0, 1.0]
    data += [0.0] * (2 ** total_bits - len(data))
    return np.sort(np.array(data, dtype=np.float32))
