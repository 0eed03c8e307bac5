"""Closeness of a GPU output to the oracle's bf16 output, with a record of every check.

The north-star tolerance is ``max|y - y_ref| <= 2e-2`` and
``mean|y - y_ref| / mean|y_ref| <= 5e-3``.  One departure from max-abs is
admitted, because no FP32 summation order other than the oracle's can avoid it:
a route's result passes three bf16 roundings (its down projection, its bf16
weighting, the route sum) and the layer adds two more (``x bf16(2.5)``, ``+
shared``).  When the kernel's FP32 sum and the oracle's land on opposite sides
of a bf16 rounding boundary, the element moves by one bf16 ulp at that point;
where the output's ulp exceeds max-abs (|y| >= 4 for one ulp, |y| >= 2 when two
roundings flip the same element) such a *rounding flip* breaks max-abs by
itself.  ``check`` admits flips only up to a per-call bound on their count and
their size in bf16 ulps of the oracle's value; every call is recorded, and
``tests/conftest.py`` prints the records at the end of the session, so the
measured flip counts stand in the test output beside the bounds they met.
"""

from __future__ import annotations

import os
from typing import NamedTuple

import numpy as np

MAX_ABS = 2e-2
MEAN_REL = 5e-3
FLIP_ULPS = 1        # default: an admitted flip moves an element by at most one bf16 ulp
FLIP_FRACTION = 1e-4  # default: at most this share of the elements (rounded down) may carry one
# The whole layer bf16(bf16(routed x 2.5) + shared): a one-ulp flip of the routed
# sum R moves 2.5 R by 2.5 ulps of R, which rounds to 1 or 2 ulps of
# bf16(2.5 R); a flip of the shared expert's output and the final rounding add
# one each -- at most 4 ulps of the largest magnitude on the element's path.
# Measured: 3 ulps (T=2048), 4 (T=8192 Zipf); 1.3e-4 (T=2048), 2.8e-4 (T=8192
# Zipf) and 3.3e-4 (decode, 2 of 6144) of the elements.
LAYER_FLIP_ULPS = 4
LAYER_FLIP_FRACTION = 4e-4


def layer_max_flips(elements: int) -> int:
    """Flips admitted in a whole-layer check of this many elements (at least 4)."""
    return max(4, int(LAYER_FLIP_FRACTION * elements))

RECORDS: list[tuple[str, str, "Closeness", int, float]] = []


class Closeness(NamedTuple):
    elements: int
    max_abs: float
    mean_rel: float
    unequal: int      # elements that differ from the oracle at all
    flips: int        # elements beyond max-abs: admitted rounding flips
    flip_ulps: float  # the largest flip in bf16 ulps of the oracle's value (0 without flips)


def bf16_ulp(values) -> np.ndarray:
    """One bf16 unit in the last place at |values| (8 significant bits)."""
    mag = np.maximum(np.abs(np.asarray(values, np.float64)), 2.0**-126)
    return np.exp2(np.floor(np.log2(mag)) - 7)


def measure(got, ref, max_abs: float = MAX_ABS, magnitude=None) -> Closeness:
    """``magnitude``: per element, the largest bf16-rounded value on its path
    (the oracle's ``return_route_max`` / ``return_magnitude``); a flip is
    measured in ulps of ``max(|ref|, magnitude)``, since a one-ulp flip of an
    intermediate is many ulps of an output that cancels to a smaller value."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    diff = np.abs(got - ref)
    rel = float(diff.mean() / max(np.abs(ref).mean(), 1e-30)) if diff.size else 0.0
    over = diff > max_abs
    flips = int(over.sum())
    scale = np.abs(ref) if magnitude is None else np.maximum(np.abs(ref), np.asarray(magnitude, np.float64))
    flip_ulps = float((diff[over] / bf16_ulp(scale[over])).max()) if flips else 0.0
    return Closeness(int(diff.size), float(diff.max()) if diff.size else 0.0, rel, int((diff != 0).sum()),
                     flips, flip_ulps)


def _current_test() -> str:
    name = os.environ.get("PYTEST_CURRENT_TEST", "?")
    return name.split("::", 1)[-1].rsplit(" ", 1)[0]


def check(got, ref, *, label: str = "", max_abs: float = MAX_ABS, mean_rel: float = MEAN_REL,
          flip_ulps: float = FLIP_ULPS, max_flips: int | None = None, magnitude=None) -> Closeness:
    """Assert the north-star tolerance with at most ``max_flips`` rounding flips
    (default ``FLIP_FRACTION`` of the elements, rounded down) of at most
    ``flip_ulps`` bf16 ulps each (of ``max(|ref|, magnitude)``); record and
    return the measurement."""
    got = np.asarray(got, np.float64)
    assert np.all(np.isfinite(got)), "non-finite output"
    c = measure(got, ref, max_abs, magnitude)
    allowed = int(FLIP_FRACTION * c.elements) if max_flips is None else int(max_flips)
    RECORDS.append((_current_test(), label, c, allowed, float(flip_ulps)))
    assert c.flips <= allowed, f"{c.flips} elements beyond max-abs {max_abs} (admitted: {allowed}); {c}"
    assert c.flip_ulps <= flip_ulps, f"a rounding flip of {c.flip_ulps:.2f} bf16 ulps (admitted: {flip_ulps}); {c}"
    assert c.mean_rel <= mean_rel, f"mean-rel {c.mean_rel:.3e} > {mean_rel}; {c}"
    return c


def summary_lines() -> list[str]:
    if not RECORDS:
        return []
    lines = [f"{len(RECORDS)} closeness checks against the oracle (max-abs {MAX_ABS}, mean-rel {MEAN_REL}); "
             "flips = elements beyond max-abs (bound), largest in bf16 ulps (bound)"]
    total = sum(r[2].elements for r in RECORDS)
    flips = sum(r[2].flips for r in RECORDS)
    unequal = sum(r[2].unequal for r in RECORDS)
    lines.append(f"  all checks: {total} elements, {unequal} not bit-equal ({unequal / max(total, 1):.2e}), "
                 f"{flips} flips ({flips / max(total, 1):.2e})")
    for test, label, c, allowed, ulps in RECORDS:
        lines.append(f"  {test}{' ' + label if label else ''}: n={c.elements} max-abs={c.max_abs:.3e} "
                     f"mean-rel={c.mean_rel:.2e} unequal={c.unequal} flips={c.flips} (<= {allowed}) "
                     f"max-flip={c.flip_ulps:.2f} ulp (<= {ulps:g})")
    return lines
