"""GPU parity for the fused tail (optimized mode, log-probability input, no
split tail, at most 16 states per thread, at most 1,024 chunks).

There the chunk kernel's last workgroup of each record runs the record's tail
itself, after a hand-off through agent-scope stores (greedy chunks) or an
agent-scope release (chunks that ran a DP), counted on a per-record arrival
counter that the library keeps per stream and that every call leaves at zero.
These tests drive the hand-off's paths against the CPU oracle, all ten outputs
bit for bit:

* the fast path (every seam legal) and the full tail (repairs, fallbacks,
  rejected records) in one call, many calls in a row (the counters must be
  zero again after each call);
* several streams with calls in flight at once (each stream has its own
  counters);
* records of more than 64 chunks (no fast path) and of more than 512 chunks
  (slots in global memory, no repair rounds so that the tail is not split).
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


def _dev(batch):
    return ([torch.from_numpy(e).cuda() for e in batch.emissions],
            [torch.from_numpy(np.ascontiguousarray(y, dtype=np.int64)).cuda() for y in batch.targets])


def _np(result):
    return {f: getattr(result, f).cpu().numpy() for f in FIELDS}


def _batches():
    """Greedy-dominated (C2, C4), repaired whole (C1) and mixed with tight,
    infeasible and flat rows (C5) batches, all below the fused-tail limits."""
    return {"c2": workloads.c2(batch=16), "c1": workloads.c1(), "c5": workloads.c5(batch=64),
            "c4": workloads.c4(batch=16)}


def test_repeated_calls_leave_the_counters_at_zero():
    """Thirty calls in a row of each batch; every one must equal the oracle (a
    counter left nonzero would hand the tail to the wrong workgroup or to none,
    and the record's outputs would be stale)."""
    for name, b in _batches().items():
        es, ys = _dev(b)
        want = O.align(b.emissions, b.targets, mode="optimized", threads=8)
        print(f"fused tail, repeated: {name}", flush=True)
        results = [ffa.align(es, ys, mode="optimized") for _ in range(30)]
        for i, r in enumerate(results):
            assert_same(_np(r), want, where=f"{name} call {i} ")
        if name in ("c1", "c5"):
            assert (want["repair_passes"] > 0).any()  # the full tail ran in the fused kernel


def test_streams_in_flight_at_once():
    """Four streams, each with its own batch, enqueued round-robin ten times
    without any synchronization in between."""
    batches = _batches()
    wants = {k: O.align(b.emissions, b.targets, mode="optimized", threads=8) for k, b in batches.items()}
    inputs = {k: _dev(b) for k, b in batches.items()}
    streams = {k: torch.cuda.Stream() for k in batches}
    for s in streams.values():
        s.wait_stream(torch.cuda.current_stream())
    print("fused tail, four streams", flush=True)
    results = {k: [] for k in batches}
    for _ in range(10):
        for k in batches:
            with torch.cuda.stream(streams[k]):
                results[k].append(ffa.align(*inputs[k], mode="optimized"))
    for s in streams.values():
        torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for k, rs in results.items():
        for i, r in enumerate(rs):
            assert_same(_np(r), wants[k], where=f"{k} stream call {i} ")


def _noisy_record(rng, T, V, tokens, spans):
    y = rng.integers(1, V, size=tokens).astype(np.int64)
    e = workloads.peaky(rng, y, T, V)
    for start, width, kind in spans:
        if kind == "ties":
            e[start:start + width] = rng.integers(-2, 1, (width, V)).astype(np.float32)
        else:
            e[start:start + width] = workloads._log_softmax(2 * rng.standard_normal((width, V)).astype(np.float32))
    return e, y


@pytest.mark.parametrize("rounds", [0, 1, 2])
def test_more_than_64_chunks(rounds):
    """chunk_frames = 16 and 2,000 frames: 125 chunks, past the tail's one-wave
    fast path, slots in LDS; a tied span and a noisy span make illegal seams."""
    rng = np.random.default_rng(125 + rounds)
    e, y = _noisy_record(rng, 2000, 8, 160, [(600, 30, "ties"), (1300, 50, "noise")])
    short = workloads.peaky(rng, y[:20], 150, 8)
    es, ys = [e, short], [y, y[:20]]
    knobs = RC.knob_vector(chunk_frames=16, repair_rounds=rounds)
    print(f"fused tail, 125 chunks, rounds {rounds}", flush=True)
    got = _op(es, ys, knobs)
    want = O.align(es, ys, blank_id=[0, 0], options=RC.oracle_options(knobs), threads=8)
    assert_same(got, want, where=f"125 chunks rounds {rounds} ")
    if rounds:
        assert got["repair_passes"][0] > 0


def test_more_than_512_chunks_without_repair_rounds():
    """chunk_frames = 16 and 9,000 frames with no repair rounds (so the tail is
    fused, not split): 563 chunks, slots in global memory, illegal seams and
    the full fallback."""
    rng = np.random.default_rng(563)
    e, y = _noisy_record(rng, 9000, 8, 700, [(2000, 40, "ties"), (5000, 60, "noise")])
    short = workloads.peaky(rng, y[:50], 300, 8)
    es, ys = [e, short], [y, y[:50]]
    knobs = RC.knob_vector(chunk_frames=16, repair_rounds=0)
    print("fused tail, 563 chunks, no repair rounds", flush=True)
    got = _op(es, ys, knobs)
    want = O.align(es, ys, blank_id=[0, 0], options=RC.oracle_options(knobs), threads=8)
    assert_same(got, want, where="563 chunks ")
    assert got["stitched"][0] == 0 and got["status"][0] == 0  # seams failed; the fallback aligned it


def _op(es, ys, k):
    ffa.load_extension()
    e = [torch.from_numpy(x).cuda() for x in es]
    y = [torch.from_numpy(x).cuda() for x in ys]
    with torch.inference_mode():
        tensors, _ = torch.ops.fast_forced_aligner_cuda.align(
            e, y, [0] * len(es), k["chunk_frames"], k["mode"], k["threads"], k["repair_rounds"],
            k["optimization_pass"], k["variant"], k["repair_budget_frames"], k["repair_threads"],
            k["compact_alphabet"], k["parallel_traceback"], k["overlap_fallback"], k["trace_min_frames"],
            k["repair_min_frames"], k["frontier_reuse"], k["frontier_min_frames"], None, True)
    return {f: t.cpu().numpy() for f, t in zip(FIELDS, tensors)}
