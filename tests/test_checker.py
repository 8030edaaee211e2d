"""The fp16-output error check of the random sweep (workload.fp16_output_errors), pinned on the
CPU: correctly rounded fp16 answers pass at any magnitude, and a plausible wrong answer fails."""
import numpy as np

import workload as kvc


def _ref(seed=0):
    g = np.random.default_rng(seed)
    r = g.normal(0.0, 1.0, 20000)
    r[::97] *= 150.0  # outlier-dominated outputs, up to a few hundred
    return r


def _passes(out, ref):
    _, _, excess, mean_excess = kvc.fp16_output_errors(out, ref)
    return excess <= 0.0 and mean_excess <= 2e-4


def test_half_ulp_matches_fp16_spacing():
    x = np.array([0.3, 0.75, 1.0, 1.9, 3.0, 100.0, 162.7, 1000.0])
    spacing = np.abs(np.nextafter(x.astype(np.float16), np.float16(np.inf)).astype(np.float64) -
                     x.astype(np.float16).astype(np.float64))
    assert np.allclose(kvc.fp16_half_ulp(x), spacing / 2)


def test_correctly_rounded_answers_pass():
    r = _ref()
    assert np.abs(r).max() > 200  # the flat 2e-3 bar fails these: their fp16 spacing is 0.125-0.25
    out = r.astype(np.float16)
    assert np.abs(out.astype(np.float64) - r).max() > 2e-3
    assert _passes(out, r)
    # a small fp32 error before the rounding (it can flip the rounding of values near a midpoint)
    assert _passes((r * (1 + 2e-6) + 1e-4).astype(np.float16), r)


def test_wrong_answers_fail():
    r = _ref(1)
    assert not _passes((r * 1.01).astype(np.float16), r)  # 1 % off
    assert not _passes((r + 3e-3).astype(np.float16), r)  # above the max-abs bound near 0
    small = np.random.default_rng(2).normal(0.0, 0.3, 20000)
    biased = (small + 3e-4).astype(np.float16)  # every element within 2e-3, the mean 3e-4 off
    assert kvc.fp16_output_errors(biased, small)[2] <= 0.0
    assert not _passes(biased, small)
