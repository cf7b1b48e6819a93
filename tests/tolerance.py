"""Per-element comparison against the oracle, in bf16 units in the last place of the oracle's value (shared by the
GPU parity tests)."""
import numpy as np


def bf16_ulp(v):
    """The bf16 ulp at each |v|: 2^(e - 7) for 2^e <= |v| < 2^(e+1) (v = 0 counts as the smallest normal)."""
    a = np.maximum(np.abs(np.asarray(v, np.float64)), 2.0 ** -126)
    return np.exp2(np.floor(np.log2(a)) - 7)


def ulp_profile(got, want):
    """(fraction within 1 ulp, within 2 ulps, within 4 ulps, largest distance in ulps) of got against want."""
    d = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64)) / bf16_ulp(want)
    return float((d <= 1).mean()), float((d <= 2).mean()), float((d <= 4).mean()), float(d.max())


def per_element_ok(got, want, frac2):
    """True when at least frac2 of the elements lie within 2 bf16 ulps of the oracle's; also the profile."""
    prof = ulp_profile(got, want)
    return prof[1] >= frac2, prof
