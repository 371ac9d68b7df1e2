"""Shared test helpers: tolerances and metrics of the parity contract."""
import numpy as np

# outputs within rel_l2 <= 5e-3 and max-abs <= 2e-2 of the
# reference CPU path; routing ids (and here also weights) bit-exact.
REL_L2_TOL = 5e-3
MAX_ABS_TOL = 2e-2


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def max_abs(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def subsample(ids, seq, n, seed=7):
    """Seeded token subsample that always includes tokens routed to the most
    and the least loaded experts (BASELINE.md CPU-baseline plan)."""
    if seq <= n:
        return np.arange(seq, dtype=np.int32)
    counts = np.bincount(ids.ravel(), minlength=ids.max() + 1)
    live = np.nonzero(counts)[0]
    most, least = live[np.argmax(counts[live])], live[np.argmin(counts[live])]
    must = {int(np.nonzero((ids == most).any(1))[0][0]), int(np.nonzero((ids == least).any(1))[0][0])}
    rng = np.random.default_rng(seed)
    rest = [t for t in rng.permutation(seq) if t not in must][: n - len(must)]
    return np.array(sorted(must | set(int(t) for t in rest)), dtype=np.int32)
