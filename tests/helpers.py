"""Shared test helpers: golden fixtures, independent CTC checks, comparisons."""
from __future__ import annotations

from itertools import product
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden" / "golden.npz"
FIELDS = ("labels", "scores", "status", "objective", "stitched", "repair_passes", "repaired_frames",
          "shortcut_stats", "routing_stats", "reuse_stats")


def golden_cases():
    """(name, emissions[T,V], targets, blank, labels, scores) from golden.npz."""
    z = np.load(GOLDEN, allow_pickle=False)
    cases = []
    e_off = y_off = t_off = 0
    for i, name in enumerate(z["names"]):
        T, V, U = int(z["frames"][i]), int(z["vocab"][i]), int(z["tokens"][i])
        e = z["emissions"][e_off:e_off + T * V].reshape(T, V)
        y = z["targets"][y_off:y_off + U]
        cases.append((str(name), e, y, int(z["blanks"][i]), z["labels"][t_off:t_off + T],
                      z["scores"][t_off:t_off + T]))
        e_off += T * V
        y_off += U
        t_off += T
    return cases


def collapse(labels, blank):
    labels = np.asarray(labels)
    if labels.size == 0:
        return labels
    keep = np.r_[True, labels[1:] != labels[:-1]]
    out = labels[keep]
    return out[out != blank]


def dp_optimum(values, targets, blank):
    """float64 CTC Viterbi optimum, written independently of the oracle
    (the reference's tests/test_core.py:11-26 uses the same check)."""
    states = np.full(2 * len(targets) + 1, blank)
    states[1::2] = targets
    previous = np.full(len(states), -np.inf)
    previous[:2] = values[0, states[:2]]
    for frame in values[1:]:
        current = np.full_like(previous, -np.inf)
        for s, label in enumerate(states):
            incoming = [previous[s]]
            if s:
                incoming.append(previous[s - 1])
            if s > 1 and label != blank and label != states[s - 2]:
                incoming.append(previous[s - 2])
            current[s] = max(incoming) + frame[label]
        previous = current
    return max(previous[-2:]) if len(previous) > 1 else previous[-1]


def exhaustive_best(values, targets, blank):
    """Best score over every legal label path, by enumeration (tiny inputs)."""
    T, V = values.shape
    best = -np.inf
    tokens = list(targets)
    for path in product(range(V), repeat=T):
        if list(collapse(path, blank)) == tokens:
            best = max(best, float(values[np.arange(T), path].astype(np.float64).sum()))
    return best


def split(flat, lengths):
    return np.split(np.asarray(flat), np.cumsum(lengths)[:-1])


def assert_same(actual: dict, expected: dict, fields=FIELDS, where=""):
    for f in fields:
        a, e = np.asarray(actual[f]), np.asarray(expected[f])
        assert a.shape == e.shape, f"{where}{f}: shape {a.shape} != {e.shape}"
        if a.dtype.kind == "f":
            ok = np.array_equal(a.view(np.int32 if a.dtype == np.float32 else np.int64),
                                e.astype(a.dtype).view(np.int32 if a.dtype == np.float32 else np.int64))
        else:
            ok = np.array_equal(a, e)
        if not ok:
            bad = np.flatnonzero((a != e).reshape(-1) if a.dtype.kind != "f" else
                                 (a.view(np.int32) != e.astype(a.dtype).view(np.int32)).reshape(-1))
            raise AssertionError(f"{where}{f}: {bad.size} mismatches, first at {bad[:5].tolist()}: "
                                 f"{a.reshape(-1)[bad[:5]].tolist()} vs {e.reshape(-1)[bad[:5]].tolist()}")
