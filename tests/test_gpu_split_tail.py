"""GPU parity for the split tail (batches whose longest record has 2,048 frames
or more, optimized mode with repair rounds).

There the tail kernel plans the first repair round and stops; one workgroup
per (chunk slot, record) then runs that round's repair interval, or the
record's early fallback, in parallel, and the record's last workgroup to
finish carries on with the later rounds and the seam check. These batches
make many short noisy spans, so each record has several first-round
intervals: records that stitch after one round, a record that needs the
second round, records that run out of rounds and fall back, a record the
budget preflight sends to the early fallback, and short records that share
the batch. All ten outputs must equal the CPU oracle bit for bit. The
reference launches its repair recurrence over the same (chunk, record) grid
once per round, with plan_repairs and validate_seams as one-thread kernels
around it (alignment.cu:727-764).
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


def _long_form(rng, frames, tokens, vocab=32, noise=0.05, span=(40, 120)):
    """Peaky emissions of a random CTC path with `noise` of the frames in flat
    spans of `span` frames (the label's boost removed), placed at random."""
    y = rng.integers(1, vocab, size=tokens).astype(np.int64)
    labels = workloads.ctc_frame_labels(rng, y, frames, 0)
    logits = rng.standard_normal((frames, vocab), dtype=np.float32)
    boost = np.full(frames, 8.0, dtype=np.float32)
    flat, done = int(noise * frames), 0
    while done < flat:
        w = int(min(rng.integers(span[0], span[1] + 1), flat - done))
        start = int(rng.integers(0, frames - w))
        boost[start:start + w] = 0.0
        done += w
    logits[np.arange(frames), labels] += boost
    return workloads._log_softmax(logits), y


def _batch(seed, specs):
    rng = np.random.default_rng(seed)
    es, ys = zip(*[_long_form(rng, *s) for s in specs])
    return list(es), list(ys)


def _run(es, ys, knobs=None):
    ffa.load_extension()
    e = [torch.from_numpy(x).cuda() for x in es]
    y = [torch.from_numpy(x).cuda() for x in ys]
    if knobs is None:
        got = ffa.align(e, y, mode="optimized")
        got = {f: getattr(got, f).cpu().numpy() for f in FIELDS}
        want = O.align(es, ys, mode="optimized", threads=8)
        return got, want
    k = knobs
    with torch.inference_mode():
        tensors, _ = torch.ops.fast_forced_aligner_cuda.align(
            e, y, [0] * len(es), k["chunk_frames"], k["mode"], k["threads"], k["repair_rounds"],
            k["optimization_pass"], k["variant"], k["repair_budget_frames"], k["repair_threads"],
            k["compact_alphabet"], k["parallel_traceback"], k["overlap_fallback"], k["trace_min_frames"],
            k["repair_min_frames"], k["frontier_reuse"], k["frontier_min_frames"], None, True)
    got = {f: t.cpu().numpy() for f, t in zip(FIELDS, tensors)}
    want = O.align(es, ys, blank_id=[0] * len(es), options=RC.oracle_options(k), threads=8)
    return got, want


def test_widest_transcripts_stitch_after_one_round():
    """Two 12,000-frame records of 3,600 tokens (7,201 states: the K = 32 DP
    function): about 60 flat spans each, every first-round interval repaired
    in its own workgroup, both records stitched."""
    es, ys = _batch(1, [(12000, 3600)] * 2)
    print("split tail: 2 x 12000 frames, 3600 tokens", flush=True)
    got, want = _run(es, ys)
    assert_same(got, want, where="split K32 ")
    assert (got["repair_passes"] == 1).all() and (got["stitched"] == 1).all()
    assert (got["repaired_frames"] > 1000).all()


def test_bench_shaped_long_form():
    """Four 30,000-frame records of 9,000 tokens with 5% of the frames flat in
    short spans: the long-form workload the split tail was built for."""
    es, ys = _batch(7, [(30000, 9000)] * 4)
    print("split tail: 4 x 30000 frames, 9000 tokens", flush=True)
    got, want = _run(es, ys)
    assert_same(got, want, where="split long-form ")
    assert (got["stitched"] == 1).all()


MIXED = [(8000, 500, 8, 0.08)] * 4 + [(1500, 300, 8, 0.05), (2100, 200, 8, 0.0)]


def test_mixed_outcomes_in_one_batch():
    """Six K = 8 records: two repair rounds that do not stitch (fallback), one
    that stitches in round two, one the budget preflight routes to the early
    fallback, a 1,500-frame record below the gating thresholds and a clean
    record with nothing to repair."""
    es, ys = _batch(2, MIXED)
    print("split tail: mixed outcomes", flush=True)
    got, want = _run(es, ys)
    assert_same(got, want, where="split mixed ")
    assert got["routing_stats"][:, 0].tolist().count(2) >= 1  # an early fallback
    assert (got["repair_passes"] == 2).sum() >= 2
    assert got["repair_passes"][5] == 0


SPLIT_KNOBS = {
    "rounds1": dict(repair_rounds=1),
    "budget0": dict(repair_budget_frames=0),
    "overlap_off": dict(overlap_fallback=False),
    "frontier_off": dict(frontier_reuse=False),
    "frontier_uncounted": dict(frontier_min_frames=1 << 30),
    "chunk64": dict(chunk_frames=64),
    "chunk256": dict(chunk_frames=256),
    "mode1": dict(mode=1),
    "repair_threads128": dict(repair_threads=128, threads=128),
    # no stored frontier (chunks under 32 frames, frontier reuse off): the
    # banded early fallback starts at frame 0
    "chunk16_frontier_off": dict(chunk_frames=16, frontier_reuse=False),
}


@pytest.mark.parametrize("family", sorted(SPLIT_KNOBS))
def test_knobs_on_the_split_path(family):
    es, ys = _batch(2, MIXED)
    knobs = RC.knob_vector(**SPLIT_KNOBS[family])
    print(f"split tail knobs {family}", flush=True)
    got, want = _run(es, ys, knobs)
    assert_same(got, want, where=f"split {family} ")
    assert (got["repair_passes"] > 0).any()
    if family == "chunk16_frontier_off":
        assert 2 in got["routing_stats"][:, 0].tolist()  # an early fallback ran, from frame 0
