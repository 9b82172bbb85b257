"""GPU parity for the path walk's edge cases (trace_path in ffa_kernels.hip).

The walk resolves 64-frame batches either frame by frame in groups of 8
(dense paths) or by runs of unchanged states (sparse paths, chosen per batch
from how far the previous batch moved), from an eight-word window of
backpointers per frame that a batch may leave. These records steer the path
through every switch: long stays followed by a stretch that moves two states
per frame (skip transitions between distinct tokens), the reverse, a record
where every frame moves, stays longer than a batch, and paths that cross the
window within one batch. Labels, scores and every other output must equal the
CPU oracle bit for bit, in both modes (optimized mode also walks the chunk
DPs and the repair DPs, which start at a > 0).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import fast_forced_aligner as ffa
from fast_forced_aligner import workloads
from helpers import FIELDS, assert_same
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _steered(rng, segments, V=32, boost=9.0):
    """Emissions whose best path follows `segments`: (label, frames) pairs in
    order, each label's frames one after another. Returns emissions, targets
    (the non-blank labels in order) and the frame labels."""
    labels = np.concatenate([np.full(n, lab, np.int64) for lab, n in segments])
    logits = rng.standard_normal((labels.size, V)).astype(np.float32)
    logits[np.arange(labels.size), labels] += np.float32(boost)
    targets = np.array([lab for lab, _ in segments if lab != 0], np.int64)
    return workloads._log_softmax(logits), targets, labels


def _distinct(rng, count, V=32):
    """`count` tokens in 1..V-1, no two neighbours equal (so skips are legal)."""
    out = [int(rng.integers(1, V))]
    while len(out) < count:
        t = int(rng.integers(1, V))
        if t != out[-1]:
            out.append(t)
    return out


def _records():
    rng = np.random.default_rng(64)
    recs = []
    # long stays, then one frame per token with no blank between them (two
    # states per frame), then long stays again
    toks = _distinct(rng, 70)
    recs.append([(toks[0], 300)] + [(t, 1) for t in toks[1:-1]] + [(toks[-1], 300)])
    # dense first, then a 700-frame blank stay and a short tail
    toks = _distinct(rng, 90)
    recs.append([(t, 1) for t in toks[:80]] + [(0, 700)] + [(t, 3) for t in toks[80:]])
    # every frame moves: tokens one frame each, blanks one frame between
    toks = _distinct(rng, 200)
    seg = []
    for t in toks:
        seg += [(t, 1), (0, 1)]
    recs.append(seg)
    # stays longer than a batch between short dense bursts (window crossings)
    toks = _distinct(rng, 150)
    seg, i = [], 0
    while i < len(toks):
        seg += [(t, 1) for t in toks[i:i + 25]] + [(0, 97)]
        i += 25
    recs.append(seg)
    # very sparse: 3 tokens over 5,000 frames
    toks = _distinct(rng, 3)
    recs.append([(0, 1500), (toks[0], 1000), (0, 10), (toks[1], 1490), (toks[2], 1000)])
    out = []
    for seg in recs:
        e, y, labels = _steered(rng, seg)
        out.append((e, y, labels))
    return out


@pytest.mark.parametrize("mode", ["conventional", "optimized"])
def test_path_walk_switches_and_window_crossings(mode):
    recs = _records()
    es = [e for e, _, _ in recs]
    ys = [y for _, y, _ in recs]
    print(f"trace edge cases, {mode}: T = {[e.shape[0] for e in es]}", flush=True)
    got = ffa.align([torch.from_numpy(e).cuda() for e in es], [torch.from_numpy(y).cuda() for y in ys],
                    mode=mode)
    got = {f: getattr(got, f).cpu().numpy() for f in FIELDS}
    want = O.align(es, ys, mode=mode, threads=8)
    assert_same(got, want, where=f"trace {mode} ")
    # the steering worked: every record's best path is the planted one
    offset = 0
    for e, _, labels in recs:
        np.testing.assert_array_equal(got["labels"][offset:offset + e.shape[0]], labels)
        offset += e.shape[0]
