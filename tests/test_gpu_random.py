"""Seeded randomized parity sweep: the operator (all ten outputs) against the
CPU oracle with the same options, on batches drawn to cross every launch form
of this build in turn.

Each seed draws a batch and a knob vector:
* records of seven kinds: peaky, peaky with flat noisy spans, integer ties,
  flat (near-tie) rows, tight (T = U + repeats), infeasible (one frame short)
  and empty targets, with a blank id per record;
* vocabularies from 4 to 1,024 (the greedy fast path, the general greedy path,
  LDS-staged and gathered DP rows);
* lengths below 2,048 frames (one launch with the fused tail, or two for more
  than 1,024 chunks) or past it (the split tail);
* chunk_frames 32..256, repair rounds 0..2, budget, overlap and frontier reuse
  on or off, mode 1 or 2, and conventional mode.
The reference operator accepts every such knob vector (alignment.cu:919-941).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import fast_forced_aligner as ffa
import repair_cases as RC
from fast_forced_aligner import workloads
from helpers import FIELDS, assert_same
from oracle import oracle as O

pytestmark = pytest.mark.gpu
KINDS = ("peaky", "spans", "ties", "flat", "tight", "infeasible", "empty")


def _targets(rng, U, vocab):
    return rng.choice(vocab, U).astype(np.int64)


def _record(rng, kind, V, blank, t_lo, t_hi):
    vocab = np.array([v for v in range(V) if v != blank])
    if kind == "empty":
        T = int(rng.integers(t_lo, t_hi))
        return workloads._log_softmax(rng.standard_normal((T, V)).astype(np.float32) * 2), np.zeros(0, np.int64)
    if kind in ("tight", "infeasible"):
        U = int(rng.integers(1, max(2, t_hi // 4)))
        y = _targets(rng, U, vocab)
        R = int((y[1:] == y[:-1]).sum())
        T = U + R if kind == "tight" else max(1, U + R - 1)
        if kind == "tight":
            return workloads.peaky(rng, y, T, V, blank), y
        return workloads._log_softmax(rng.standard_normal((T, V)).astype(np.float32)), y
    T = int(rng.integers(t_lo, t_hi))
    U = max(1, T // int(rng.integers(3, 7)))
    y = _targets(rng, U, vocab)
    R = int((y[1:] == y[:-1]).sum())
    if U + R > T:
        y = y[: max(1, T // 3)]
    if kind == "ties":
        return rng.integers(-3, 1, (T, V)).astype(np.float32), y
    if kind == "flat":
        return workloads._log_softmax((0.01 * rng.standard_normal((T, V))).astype(np.float32)), y
    e = workloads.peaky(rng, y, T, V, blank)
    if kind == "spans":
        for _ in range(int(rng.integers(1, 4))):
            w = int(rng.integers(10, 120))
            s = int(rng.integers(0, max(1, T - w)))
            e[s:s + w] = workloads._log_softmax(2 * rng.standard_normal((min(w, T - s), V)).astype(np.float32))
    return e, y


def _draw(seed):
    rng = np.random.default_rng(9000 + seed)
    V = int(rng.choice([4, 8, 12, 32, 33, 64, 300, 1024]))
    long_form = seed % 4 == 3
    t_lo, t_hi = (1800, 2700) if long_form else (20, 1900)
    count = int(rng.integers(2, 6 if long_form else 20))
    es, ys, blanks = [], [], []
    for _ in range(count):
        blank = int(rng.integers(0, V)) if rng.random() < 0.3 else 0
        kind = str(rng.choice(KINDS, p=[0.3, 0.25, 0.1, 0.1, 0.1, 0.05, 0.1]))
        e, y = _record(rng, kind, V, blank, t_lo, t_hi)
        es.append(e)
        ys.append(y)
        blanks.append(blank)
    knobs = dict(chunk_frames=int(rng.choice([32, 64, 128, 128, 128, 256])),
                 repair_rounds=int(rng.choice([0, 1, 2, 2])),
                 repair_budget_frames=int(rng.choice([0, 512, 512])),
                 overlap_fallback=bool(rng.random() < 0.7), frontier_reuse=bool(rng.random() < 0.8),
                 mode=int(rng.choice([1, 2, 2, 2])))
    if seed % 5 == 4:
        knobs.update(mode=0, repair_budget_frames=0, overlap_fallback=False, frontier_reuse=False)
    return es, ys, blanks, RC.knob_vector(**knobs)


def _op(es, ys, blanks, k):
    ffa.load_extension()
    e = [torch.from_numpy(x).cuda() for x in es]
    y = [torch.from_numpy(x).cuda() for x in ys]
    with torch.inference_mode():
        tensors, lengths = torch.ops.fast_forced_aligner_cuda.align(
            e, y, list(blanks), k["chunk_frames"], k["mode"], k["threads"], k["repair_rounds"],
            k["optimization_pass"], k["variant"], k["repair_budget_frames"], k["repair_threads"],
            k["compact_alphabet"], k["parallel_traceback"], k["overlap_fallback"], k["trace_min_frames"],
            k["repair_min_frames"], k["frontier_reuse"], k["frontier_min_frames"], None, True)
    out = {f: t.cpu().numpy() for f, t in zip(FIELDS, tensors)}
    out["lengths"] = tuple(int(x) for x in lengths)
    return out


@pytest.mark.parametrize("seed", range(48))
def test_random_batch_matches_the_oracle(seed):
    es, ys, blanks, knobs = _draw(seed)
    print(f"random seed {seed}: B={len(es)} V={es[0].shape[1]} T_max={max(e.shape[0] for e in es)} "
          f"knobs={ {k: knobs[k] for k in ('mode', 'chunk_frames', 'repair_rounds', 'repair_budget_frames')} }",
          flush=True)
    got = _op(es, ys, blanks, knobs)
    want = O.align(es, ys, blank_id=blanks, options=RC.oracle_options(knobs), threads=8)
    assert got["lengths"] == want["lengths"]
    assert_same(got, want, where=f"seed {seed} ")
