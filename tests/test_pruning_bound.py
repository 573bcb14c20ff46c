"""The page score bounds of the pruned fine scan, checked by brute force on
the CPU: every token's score, as the scan computes it (an fp32 dot product
in some summation order, then the score rounding), must lie between the
scores of the page's lower and upper bound.

The bounds are the ones the coarse scan writes: around the dtype summary s
of a page row (the fp64 mean rounded to fp32, then to the dtype) with the
radius rad = max |k - s| and |s| recorded at eviction,

    q.s +- (|q| rad 1.0001 + 1e-4 |q| (|s| + rad)),

widened by 1e-4 relative for the fp32 rounding of the dot products.  The
summation orders tried here (sequential, pairwise, chunked by lanes) stand
for the kernels' FMA chains and cross-lane sums; the cases include head dims
up to 512, the three dtypes, tight clusters (where the radius term is small
and the margin matters most) and wide pages.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle.exact import round_to_dtype as round_to

pytestmark = pytest.mark.filterwarnings("ignore::RuntimeWarning")


def dot_orders(q: np.ndarray, k: np.ndarray) -> list[np.float32]:
    """fp32 dot products of q (D,) with the rows of k (T, D) in several orders."""
    q32, k32 = q.astype(np.float32), k.astype(np.float32)
    prod = (k32 * q32).astype(np.float32)  # exact for 16-bit inputs
    out = []
    # sequential
    acc = np.zeros(k.shape[0], dtype=np.float32)
    for d in range(k.shape[1]):
        acc = (acc + prod[:, d]).astype(np.float32)
    out.append(acc)
    # numpy's pairwise sum in fp32
    out.append(prod.sum(axis=1, dtype=np.float32))
    # lanes of 8, then a tree over the lanes (the VALU scan's chunks)
    lanes = prod.reshape(k.shape[0], -1, 8).sum(axis=2, dtype=np.float32)
    while lanes.shape[1] > 1:
        if lanes.shape[1] % 2:
            lanes = np.concatenate([lanes, np.zeros((lanes.shape[0], 1), np.float32)], axis=1)
        lanes = (lanes[:, 0::2] + lanes[:, 1::2]).astype(np.float32)
    out.append(lanes[:, 0])
    return out


def score_of(dot: np.ndarray, scale: float, dtype: str) -> np.ndarray:
    """The scan's score: the dot rounded to the dtype, times scale, rounded again."""
    if dtype == "float32":
        return (dot.astype(np.float32) * np.float32(scale)).astype(np.float32)
    return round_to(round_to(dot.astype(np.float64), dtype).astype(np.float32) * np.float32(scale), dtype)


def page_bounds(q: np.ndarray, k: np.ndarray, dtype: str) -> tuple[float, float]:
    """(lower, upper) bound of the fp32 dot of q with any row of the page k."""
    mean32 = k.astype(np.float64).mean(axis=0).astype(np.float32)
    s = mean32 if dtype == "float32" else round_to(mean32.astype(np.float64), dtype).astype(np.float32)
    diff = (k.astype(np.float32) - s).astype(np.float32)
    rad = np.float32(np.sqrt(np.max((diff.astype(np.float32) ** 2).sum(axis=1, dtype=np.float32))))
    sn = np.float32(np.sqrt((s * s).sum(dtype=np.float32)))
    qs = np.float32((q.astype(np.float32) * s).sum(dtype=np.float32))
    qn = np.float32(np.sqrt((q.astype(np.float32) ** 2).sum(dtype=np.float32)))
    w = np.float32(qn * rad * np.float32(1.0001) + np.float32(1e-4) * qn * (sn + rad))
    return float(qs - w), float(qs + w)


CASES = [
    # head dim, dtype, cluster spread, centroid norm scale
    (64, "bfloat16", 0.3, 1.0),
    (96, "float16", 0.3, 1.0),
    (128, "bfloat16", 0.01, 4.0),   # tight cluster: the radius term is small
    (128, "float32", 0.001, 8.0),
    (256, "bfloat16", 1.0, 0.5),    # wide page
    (512, "bfloat16", 0.02, 3.0),
    (512, "float16", 0.05, 1.0),
]


@pytest.mark.parametrize("D,dtype,spread,norm", CASES)
def test_token_scores_lie_within_the_page_bounds(D, dtype, spread, norm):
    rng = np.random.default_rng(D + int(spread * 1000))
    scale = 1.0 / np.sqrt(D)
    for trial in range(20):
        c = rng.normal(0.0, norm, D)
        k = c + spread * rng.normal(0.0, 1.0, (128, D))
        if trial % 5 == 4:
            k[rng.integers(0, 128)] *= 3.0  # one outlier token far from the mean
        q = c * rng.uniform(-2, 2) + rng.normal(0.0, 0.5, D)
        if dtype != "float32":
            k = round_to(k, dtype)
            q = round_to(q, dtype)
        lo, hi = page_bounds(q, k, dtype)
        s_lo = score_of(np.array([lo], np.float32), scale, dtype)[0]
        s_hi = score_of(np.array([hi], np.float32), scale, dtype)[0]
        for dots in dot_orders(q, k):
            scores = score_of(dots, scale, dtype)
            assert scores.max() <= s_hi, (trial, float(scores.max()), float(s_hi))
            assert scores.min() >= s_lo, (trial, float(scores.min()), float(s_lo))


def test_bounds_are_not_vacuous_for_clustered_pages():
    """On a clustered page far from the query the upper bound stays well below
    a near page's lower bound, which is what lets the scan skip it."""
    rng = np.random.default_rng(7)
    D = 128
    c_near, c_far = rng.normal(0, 1, D), rng.normal(0, 1, D)
    q = round_to(c_near + rng.normal(0, 0.1, D), "bfloat16")
    near = round_to(c_near + 0.3 * rng.normal(0, 1, (128, D)), "bfloat16")
    far = round_to(c_far + 0.3 * rng.normal(0, 1, (128, D)), "bfloat16")
    assert page_bounds(q, far, "bfloat16")[1] < page_bounds(q, near, "bfloat16")[0]


@pytest.mark.parametrize("D,dtype", [(128, "float32"), (512, "float32"), (256, "bfloat16"), (512, "float16")])
def test_bounds_hold_where_cauchy_schwarz_is_tight(D, dtype):
    """Tokens displaced from the mean along q make the radius term exact, so
    only the 1e-4 margin absorbs the fp32 rounding of the dot products."""
    rng = np.random.default_rng(100 + D)
    scale = 1.0 / np.sqrt(D)
    for trial in range(40):
        c = rng.normal(0.0, 2.0, D)
        q = rng.normal(0.0, 1.0, D) + c
        if dtype != "float32":
            q = round_to(q, dtype)
        qhat = q / np.linalg.norm(q)
        k = np.repeat(c[None, :], 128, axis=0)
        k += 1e-3 * rng.normal(0.0, 1.0, (128, D))
        t = rng.uniform(0.5, 4.0)
        k[0] = c + t * qhat   # the farthest token, along +q
        k[1] = c - t * qhat   # and along -q
        if dtype != "float32":
            k = round_to(k, dtype)
        lo, hi = page_bounds(q, k, dtype)
        s_lo = score_of(np.array([lo], np.float32), scale, dtype)[0]
        s_hi = score_of(np.array([hi], np.float32), scale, dtype)[0]
        for dots in dot_orders(q, k):
            scores = score_of(dots, scale, dtype)
            assert scores.max() <= s_hi, (trial, float(scores.max()), float(s_hi))
            assert scores.min() >= s_lo, (trial, float(scores.min()), float(s_lo))
