"""Token spans (the reference README's "Converting frame labels to timestamps",
README.md:509-517, stated only in prose): the oracle restatement pinned by
known answers written from that prose and by an independent groupby
formulation on random paths."""
from __future__ import annotations

from itertools import groupby

import numpy as np

from oracle import oracle as O


def groupby_spans(path, blank):
    """Independent formulation: itertools.groupby over (label) runs."""
    out, t = [], 0
    for label, run in groupby(path):
        n = len(list(run))
        if label != blank:
            out.append((t, t + n))
        t += n
    return out


def test_known_answers_from_the_readme_rule():
    # blank 0: runs 1-1 | 2-2-2 | 2 (a blank between the two 2-runs keeps them separate)
    path = np.array([0, 1, 1, 0, 2, 2, 2, 0, 0, 2])
    got = O.token_spans(path, [10], [3], np.array([0]), 0)
    assert got.tolist() == [[1, 3], [4, 7], [9, 10]]
    # no leading blank, blank id 5
    path = np.array([3, 3, 5, 4])
    assert O.token_spans(path, [4], [2], np.array([0]), 5).tolist() == [[0, 2], [3, 4]]
    # adjacent different tokens without a blank are two runs
    path = np.array([1, 2, 2])
    assert O.token_spans(path, [3], [2], np.array([0]), 0).tolist() == [[0, 1], [1, 3]]


def test_failed_records_and_padding():
    labels = np.array([-1, -1, -1, 0, 4, 4, 0])
    got = O.token_spans(labels, [3, 4], [2, 2], np.array([4, 0]), 0)
    assert got.tolist() == [[-1, -1], [-1, -1], [1, 3], [-1, -1]]  # record-relative frames; one run for two tokens
    assert O.token_spans(labels[3:], [4], [0], np.array([0]), 0).shape == (0, 2)


def test_random_paths_match_groupby():
    rng = np.random.default_rng(3)
    lengths, tokens, blanks, paths = [], [], [], []
    for _ in range(200):
        T = int(rng.integers(1, 60))
        blank = int(rng.integers(0, 4))
        path = rng.integers(0, 4, T)
        runs = groupby_spans(path.tolist(), blank)
        lengths.append(T); tokens.append(len(runs)); blanks.append(blank); paths.append(path)
    got = O.token_spans(np.concatenate(paths), lengths, tokens, np.zeros(len(paths), np.int32), blanks)
    want = [s for p, b in zip(paths, blanks) for s in groupby_spans(p.tolist(), b)]
    assert got.tolist() == [list(s) for s in want]
