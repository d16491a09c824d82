"""Deciding, before a run, whether a comparison can see an int8
requantization flip.

Two evaluations of the fp32 glue that differ only by fp32 rounding (the
device's fp32 matrix cores against the oracle's fp64, or the reference's own
fp32 order against either) quantize to the same int8 values wherever no
quantizer argument lies within their difference of a rounding boundary.  The
oracle records the smallest such margin of a pass (Oracle.track_margins);
against the bound below it decides the bar of the comparison:

* flip-free (margin > MARGIN_BOUND): the results agree to fp32 rounding;
* otherwise: a flip may move this random model's outputs by the flip level.

EPS_F32 bounds the difference of two fp32-evaluated inputs of a quantizer,
relative to the row's largest magnitude: 1e-6, eight times the largest such
difference measured on the paths compared here (1.5e-7 of the largest
value).  A quantizer argument t = |v| * 127 / amax then moves by at most
254 EPS_F32 (v and amax each by EPS_F32 * amax), plus the fp32 rounding of
v * inv on both sides (2 * 127 * 2**-24).
"""

from __future__ import annotations

import numpy as np

EPS_F32 = 1e-6
MARGIN_BOUND = 254 * EPS_F32 + 2 * 127 * 2.0 ** -24


def flip_free(oracle) -> bool:
    """True when the oracle's pass since track_margins() has no quantizer
    argument within MARGIN_BOUND of a rounding boundary."""
    return oracle.min_margin() > MARGIN_BOUND


def clear_argmax(logits: np.ndarray, rel: float) -> bool:
    """True when the top logit leads the runner-up by more than 2 * rel of the
    largest magnitude: a perturbation of at most rel of that magnitude on
    every logit cannot change the argmax."""
    top2 = np.sort(np.asarray(logits, np.float64))[-2:]
    return float(top2[1] - top2[0]) > 2.0 * rel * float(np.abs(logits).max())


def tracked(oracle, fn, *args, **kwargs):
    """fn(*args, **kwargs) with the oracle's margins tracked; returns
    (result, smallest margin of the pass)."""
    oracle.track_margins()
    try:
        out = fn(*args, **kwargs)
        return out, oracle.min_margin()
    finally:
        oracle.margins = None
