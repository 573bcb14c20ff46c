"""How far each disagreement between two top-k selections lies from the boundary.

Test infrastructure only (see oracle/__init__.py).

The parity rule for the retrieval's indices: selected page and token ids
must agree wherever the scores are separated by more than 1e-3.  For one
row of scores s (one arithmetic) and a top-k, let t_k and t_k1 be the k-th
and (k+1)-th largest values.  The distance of entry i from the boundary is

    gap_i = max(s_i - t_k1, t_k - s_i)

the smallest change of s_i alone that moves i across the boundary: an entry
inside the top k leaves it only by falling below t_k1, an entry outside it
enters only by rising above t_k (with ties, both terms are 0 for an entry
equal to a tied boundary value).  With k >= n every entry is selected and
the gap is infinite.

Two arithmetics are scored (the reference's scores are dtype-rounded, so a
boundary that is wide in float64 can be an exact tie in the dtype, and the
other way round near a rounding step):
  * ``s64``: q.k * scaling in float64 (closed form);
  * ``semu``: the dot product rounded once to fp32, then the reference's
    dtype rounding (kiv/cold_store.py:206-208, 333-335) via
    oracle.exact.emulate_scores.
An id on which the two selections disagree breaks the rule only when its gap
exceeds the tolerance in both.
"""

from __future__ import annotations

import numpy as np

from . import exact

TOL = 1e-3


def boundary_values(scores: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """(t_k, t_k1) per row of ``scores`` [R, n]; t_k1 = -inf when k >= n."""
    s = np.asarray(scores, dtype=np.float64)
    R, n = s.shape
    k = min(k, n)
    srt = -np.sort(-s, axis=1)
    tk = srt[:, k - 1]
    tk1 = srt[:, k] if k < n else np.full(R, -np.inf)
    return tk, tk1


def boundary_gaps(scores: np.ndarray, k: int) -> np.ndarray:
    """gap_i of every entry of every row: [R, n] (inf where k >= n)."""
    s = np.asarray(scores, dtype=np.float64)
    tk, tk1 = boundary_values(s, k)
    return np.maximum(s - tk1[:, None], tk[:, None] - s)


def scores_both(q: np.ndarray, keys: np.ndarray, scaling: float, dtype: str) -> tuple[np.ndarray, np.ndarray]:
    """(s64, semu) of q [B, Hq, Q, D] against keys [B, Hkv, T, D]: [B, Hq, Q, T] each."""
    groups = q.shape[1] // keys.shape[1]
    s64 = exact.scores64(q, keys, scaling, groups)
    semu = exact.emulate_scores(exact.dots32(q, keys, groups), scaling, dtype)
    return s64, semu


def _stats(got: set, ref: set, g64: np.ndarray, gemu: np.ndarray, ids: list) -> dict:
    both = np.minimum(g64, gemu) if len(ids) else np.zeros(0)
    return {
        "got": len(got), "ref": len(ref), "differ": len(ids),
        "max_gap64": float(g64.max()) if len(ids) else 0.0,
        "max_gap_emu": float(gemu.max()) if len(ids) else 0.0,
        "max_gap_min": float(both.max()) if len(ids) else 0.0,
        "violations": [int(i) for i, m in zip(ids, both) if m > TOL],
    }


def topk_differences(got: set, ref: set, s64_row: np.ndarray, semu_row: np.ndarray, k: int) -> dict:
    """One row's top-k: ``got`` and ``ref`` index sets (into the row) against
    the row's scores in both arithmetics.

    Returns counts, the largest gaps among the differing indices, and the
    indices whose gap exceeds TOL in both arithmetics ("violations")."""
    g64 = boundary_gaps(s64_row[None, :], k)[0]
    gemu = boundary_gaps(semu_row[None, :], k)[0]
    ids = sorted(got ^ ref)
    idx = np.array(ids, dtype=np.int64)
    return _stats(got, ref, g64[idx], gemu[idx], ids)


def union_differences(got: set, ref: set, s64_rows: np.ndarray, semu_rows: np.ndarray, k: int,
                      ref_rows: list[set]) -> dict:
    """The union over rows of per-row top-k (the coarse page union).

    ``ref_rows``: the reference's per-row selections.  A page only in
    ``got`` was selected for some row that the reference did not select it
    for (it selected it for none), so its gap is the smallest over all rows
    of min(gap64, gap_emu).  A page only in ``ref`` was selected by the
    reference in each row of ``ref_rows`` holding it, and ``got`` selected
    it nowhere, so each of those rows had to be near its boundary: its gap
    is the largest over those rows of min(gap64, gap_emu)."""
    g64 = boundary_gaps(s64_rows, k)
    gemu = boundary_gaps(semu_rows, k)
    gmin = np.minimum(g64, gemu)
    ids = sorted(got ^ ref)
    v64, vemu, vmin = [], [], []
    for p in ids:
        if p in got:
            r = int(np.argmin(gmin[:, p]))
        else:
            rows = [r for r, sel in enumerate(ref_rows) if p in sel]
            r = rows[int(np.argmax(gmin[rows, p]))]
        v64.append(g64[r, p])
        vemu.append(gemu[r, p])
        vmin.append(gmin[r, p])
    out = _stats(got, ref, np.array(v64), np.array(vemu), ids)
    out["max_gap_min"] = float(max(vmin)) if ids else 0.0
    out["violations"] = [int(p) for p, m in zip(ids, vmin) if m > TOL]
    return out
