"""Selection checks that allow exactly the ambiguity the arithmetic admits.

Test infrastructure only (see oracle/__init__.py).

A kernel score is an fp32 dot product (some summation order) optionally
rounded to the activation dtype, times the scale, rounded again
(oracle.exact.emulate_scores).  The exact dot ``dot64`` is known, and any
fp32 summation of D products differs from it by at most
delta = (D + 4) * 2**-24 * sum|q_i k_i|.  Every kernel score therefore lies
in [emulate(dot64 - delta), emulate(dot64 + delta)] (rounding is monotone).

For a top-k over a row of such intervals:
  * an index is certainly selected when fewer than k other indices can
    reach its lower end;
  * it is certainly not selected when at least k indices are surely above
    its upper end.
The kernel's set must contain the first group and lie inside the
complement of the second.  Rows where both groups coincide (no interval
straddles the boundary) are "determined" and compared bit-exactly; with
the separated synthetic scores (gap > 1e-3) that is almost every row.
"""

from __future__ import annotations

import numpy as np

from . import exact

U32 = 2.0 ** -24


def score_interval(q: np.ndarray, keys: np.ndarray, scaling: float, dtype: str, rounding: str):
    """(lo, hi) kernel-score bounds, [B, Hq, Q, T] each."""
    groups = q.shape[1] // keys.shape[1]
    dot = exact.grouped_dots(q, keys, groups)
    mag = exact.grouped_dots(q, keys, groups, absolute=True)
    delta = (q.shape[-1] + 4) * U32 * mag
    if rounding == "fp32":
        lo = (dot - delta).astype(np.float32).astype(np.float64) * scaling
        hi = (dot + delta).astype(np.float32).astype(np.float64) * scaling
        lo = lo - np.abs(lo) * 2 * U32
        hi = hi + np.abs(hi) * 2 * U32
        return lo, hi
    # Round outward to fp32 first so the dtype rounding brackets the kernel.
    lo32 = np.nextafter((dot - delta).astype(np.float32), np.float32(-np.inf))
    hi32 = np.nextafter((dot + delta).astype(np.float32), np.float32(np.inf))
    return (exact.emulate_scores(lo32, scaling, dtype), exact.emulate_scores(hi32, scaling, dtype))


def row_bands(lo: np.ndarray, hi: np.ndarray, k: int):
    """(certainly selected, possibly selected) index sets of one row's top-k."""
    n = lo.size
    k = min(k, n)
    his = np.sort(hi)
    reach = n - np.searchsorted(his, lo, side="left") - 1  # others whose hi >= my lo
    must = set(np.nonzero(reach < k)[0].tolist())
    los = np.sort(lo)
    above = n - np.searchsorted(los, hi, side="right")  # indices whose lo > my hi
    may = set(np.nonzero(above < k)[0].tolist())
    return must, may


def check_topk(got: set, lo_rows: np.ndarray, hi_rows: np.ndarray, k: int) -> float:
    """Assert ``got`` is the union of the rows' top-k within the bands.

    Returns the fraction of rows whose selection is fully determined.
    """
    must_all, may_all, determined = set(), set(), 0
    for lo, hi in zip(lo_rows, hi_rows):
        must, may = row_bands(lo, hi, k)
        determined += must == may
        must_all |= must
        may_all |= may
    missing = sorted(must_all - got)
    extra = sorted(got - may_all)
    assert not missing, f"{len(missing)} certainly-selected indices missing, e.g. {missing[:8]}"
    assert not extra, f"{len(extra)} indices outside the possible set, e.g. {extra[:8]}"
    return determined / max(1, len(lo_rows))


# ------------------------------------------------- telemetry score intervals

def _dtype_step(r: float, dtype: str, down: bool) -> float:
    """The dtype value next to the dtype value ``r``, below it (or above)."""
    if dtype == "float32":
        return float(np.nextafter(np.float32(r), np.float32(-np.inf if down else np.inf)))
    if dtype == "float16":
        return float(np.nextafter(np.float16(r), np.float16(-np.inf if down else np.inf)))
    # bfloat16: step the upper 16 bits of the fp32 pattern
    if r == 0.0:
        tiny = 2.0 ** -133
        return -tiny if down else tiny
    u = int(np.float32(r).view(np.uint32))
    u += (-0x10000 if down else 0x10000) * (1 if r > 0 else -1)
    return float(np.uint32(u).view(np.float32))


def dtype_floor(x: float, dtype: str) -> float:
    """The largest dtype value <= x."""
    r = float(exact.round_to_dtype(np.array([x]), dtype)[0])
    return _dtype_step(r, dtype, True) if r > x else r


def dtype_ceil(x: float, dtype: str) -> float:
    """The smallest dtype value >= x."""
    r = float(exact.round_to_dtype(np.array([x]), dtype)[0])
    return _dtype_step(r, dtype, False) if r < x else r


def max_band(lo: np.ndarray, hi: np.ndarray) -> tuple[float, float]:
    """Interval of the largest of scores that lie in [lo_i, hi_i]."""
    return float(np.max(lo)), float(np.max(hi))


def mean_band(lo: np.ndarray, hi: np.ndarray, dtype: str, rounding: str) -> tuple[float, float]:
    """Interval of a computed mean of scores in [lo_i, hi_i].

    The reference takes ``scores.mean()`` of a dtype tensor (a float
    accumulation, rounded to the dtype); the kernels sum in fp32 per row and
    in fp64 across rows, then round to the dtype.  Any fp32 summation of n
    terms errs by at most (n + 2) * 2**-24 * sum |s_i|, and rounding to the
    dtype (or to fp32, when scores are fp32) in any direction stays within
    the neighbouring values, so both lie in the returned interval."""
    n = lo.size
    err = (n + 2) * U32 * float(np.maximum(np.abs(lo), np.abs(hi)).sum()) / n
    a, b = float(lo.mean()) - err, float(hi.mean()) + err
    out = dtype if rounding == "activation" else "float32"
    return dtype_floor(a, out), dtype_ceil(b, out)
