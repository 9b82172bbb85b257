"""GPU parity for the operator's knob space, called the way a reference-shaped
Python layer calls it: torch.ops.fast_forced_aligner_cuda.align with the
schema of alignment.cu:1065-1068.

* The hand-derived repair, budget and frontier cases of repair_cases.py run
  through the HIP path and must give the values derived on paper.
* Every knob family the operator accepts (alignment.cu:919-941) runs on a
  mixed batch against the CPU oracle with the same options, all ten outputs
  bit for bit.
* A record of more than 512 chunks takes the tail kernel's global-memory slot
  path (chunk_frames = 16, 9,000 frames; chunk_frames = 32, 16,500 frames with
  a saved frontier per chunk, counted in reuse_stats or not).
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
DEV = "cuda"


def op_align(emissions, targets, blanks, knobs, check_inputs=True):
    """The reference-schema operator with an explicit knob vector; returns the
    ten outputs as numpy arrays plus lengths."""
    ffa.load_extension()  # registers the fast_forced_aligner_cuda operators
    es = [torch.from_numpy(np.ascontiguousarray(e)).to(DEV) for e in emissions]
    ys = [torch.from_numpy(np.ascontiguousarray(y, dtype=np.int64)).to(DEV) for y in targets]
    k = knobs
    with torch.inference_mode():
        tensors, lengths = torch.ops.fast_forced_aligner_cuda.align(
            es, ys, list(blanks), k["chunk_frames"], k["mode"], k["threads"], k["repair_rounds"],
            k["optimization_pass"], k["variant"], k["repair_budget_frames"], k["repair_threads"],
            k["compact_alphabet"], k["parallel_traceback"], k["overlap_fallback"], k["trace_min_frames"],
            k["repair_min_frames"], k["frontier_reuse"], k["frontier_min_frames"], None, check_inputs)
    out = {f: t.cpu().numpy() for f, t in zip(FIELDS, tensors)}
    out["lengths"] = tuple(int(x) for x in lengths)
    return out


def oracle_align(emissions, targets, blanks, knobs):
    return O.align(emissions, targets, blank_id=list(blanks), options=RC.oracle_options(knobs), threads=8)


@pytest.mark.parametrize("case", RC.all_cases(), ids=lambda c: c["name"])
def test_hand_derived_repair_cases(case):
    knobs = RC.knob_vector(**case["knobs"])
    print(f"hand-derived {case['name']}", flush=True)
    got = op_align([case["emissions"]], [case["targets"]], [0], knobs)
    RC.check_expected(got, case)


def test_hand_derived_cases_in_one_batch():
    """The public-knob cases batched together (ragged T from 256 to 2,048, V 4
    and 8): batch-level gating turns budget, overlap and frontier reuse on for
    every record (the longest is 2,048 frames), so the short cases must keep
    their per-record results (their T < repair_min_frames and frontier_min_frames
    exempts them, alignment.cu:175, :374)."""
    cases = [c for c in RC.all_cases() if not c["knobs"]]
    knobs = RC.knob_vector()
    got = op_align([c["emissions"] for c in cases], [c["targets"] for c in cases], [0] * len(cases), knobs)
    want = oracle_align([c["emissions"] for c in cases], [c["targets"] for c in cases], [0] * len(cases), knobs)
    assert_same(got, want, where="hand-derived batch ")
    offsets = np.cumsum([0] + [len(c["emissions"]) for c in cases])
    for i, c in enumerate(cases):
        np.testing.assert_array_equal(got["labels"][offsets[i]:offsets[i + 1]], c["expect"]["labels"])
        assert got["repair_passes"][i] == c["expect"]["repair_passes"][0]


def _mixed_batch():
    """C1, peaky and tie-heavy records, a noisy long record (budget, early
    fallback, frontier reuse at T >= 2048) and the hand-derived records."""
    rng = np.random.default_rng(2026)
    b = workloads.c1()
    es, ys, blanks = list(b.emissions), list(b.targets), [0, 0]
    for T, kind in ((300, "peaky"), (700, "peaky"), (420, "ties"), (260, "flat"), (1000, "peaky")):
        y = rng.integers(1, 32, size=max(1, T // 4)).astype(np.int64)
        if kind == "peaky":
            e = workloads.peaky(rng, y, T, 32)
        elif kind == "ties":
            e = rng.integers(-3, 1, (T, 32)).astype(np.float32)
        else:
            e = np.log(rng.dirichlet(np.ones(32) * 50, T)).astype(np.float32)
        es.append(e)
        ys.append(y)
        blanks.append(0)
    T = 2305
    y = rng.integers(1, 32, size=600).astype(np.int64)
    e = workloads.peaky(rng, y, T, 32)
    e[700:1000] = workloads._log_softmax(3 * rng.standard_normal((300, 32)).astype(np.float32))
    e[1500:2200] = workloads._log_softmax(3 * rng.standard_normal((700, 32)).astype(np.float32))
    es.append(e)
    ys.append(y)
    blanks.append(0)
    for case in (RC.one_seam(), RC.second_round(), RC.frontier_resume()):
        es.append(case["emissions"])
        ys.append(case["targets"])
        blanks.append(0)
    return es, ys, blanks


KNOB_FAMILIES = {
    "api_optimized": {},
    "mode1": dict(mode=1),
    "mode0_conventional": dict(mode=0, repair_budget_frames=0, overlap_fallback=False, frontier_reuse=False),
    "rounds0": dict(repair_rounds=0),
    "rounds1": dict(repair_rounds=1),
    "chunk64": dict(chunk_frames=64),
    "chunk256": dict(chunk_frames=256),
    "chunk512": dict(chunk_frames=512),
    "chunk100_mode1": dict(chunk_frames=100, mode=1),
    "budget0": dict(repair_budget_frames=0),
    "overlap_off": dict(overlap_fallback=False),
    "budget0_overlap_off": dict(repair_budget_frames=0, overlap_fallback=False),
    "budget_small": dict(repair_budget_frames=200),
    "frontier_off": dict(frontier_reuse=False),
    "frontier_min0": dict(frontier_min_frames=0),
    "repair_min0": dict(repair_min_frames=0),
    "repair_min_huge": dict(repair_min_frames=1 << 30),
    "pass3": dict(optimization_pass=3),
    "threads128": dict(threads=128),
    "threads256": dict(threads=256),
    "variant0": dict(variant=0),
    "variant1": dict(variant=1),
    "compact": dict(compact_alphabet=True),
    "serial_traceback": dict(parallel_traceback=False),
    "trace_min1": dict(trace_min_frames=1),
    "repair_threads128": dict(repair_threads=128, threads=128),
    "repair_threads256_no_overlap": dict(repair_threads=256, overlap_fallback=False),
}


@pytest.mark.parametrize("family", sorted(KNOB_FAMILIES))
def test_knob_family_matches_oracle(family):
    es, ys, blanks = _mixed_batch()
    knobs = RC.knob_vector(**KNOB_FAMILIES[family])
    print(f"knobs {family}", flush=True)
    got = op_align(es, ys, blanks, knobs)
    want = oracle_align(es, ys, blanks, knobs)
    assert got["lengths"] == want["lengths"]
    assert_same(got, want, where=f"{family} ")
    if family not in ("mode0_conventional", "rounds0", "chunk512"):
        assert (got["repair_passes"] > 0).any()  # the repair rounds ran


@pytest.mark.parametrize("chunk_frames", [0, 513, 1 << 20])
def test_chunk_frames_outside_the_supported_range_is_rejected(chunk_frames):
    """chunk_frames must be 1..512 here (the reference takes any positive int32,
    alignment.cu:947-948): larger values are refused with a RuntimeError before
    anything is allocated or launched."""
    b = workloads.c1()
    with pytest.raises(RuntimeError, match="chunk size or mode"):
        op_align(b.emissions, b.targets, [0, 0], RC.knob_vector(chunk_frames=chunk_frames))


@pytest.mark.parametrize("knobs", [dict(), dict(repair_budget_frames=0), dict(frontier_reuse=False, mode=1)],
                         ids=["api", "budget0", "mode1_no_frontier"])
def test_more_than_512_chunks_use_global_slots(knobs):
    """A 9,000-frame record at chunk_frames = 16 has 563 chunks, more than the
    tail kernel's 512 LDS slots: its repair planning, seams and frontier
    bookkeeping run on slots in global memory. A tied span and a noisy span
    make illegal seams. With the public knobs round 1 merges (8,760 frames)
    and round 2's budget preflight sends the record to the early fallback;
    without a budget two rounds repair 12,040 frames and the record stitches."""
    rng = np.random.default_rng(563)
    T, V = 9000, 8
    y = rng.integers(1, V, size=700).astype(np.int64)
    e = workloads.peaky(rng, y, T, V)
    e[2000:2040] = rng.integers(-2, 1, (40, V)).astype(np.float32)  # ties: chunk DPs
    e[5000:5060] = workloads._log_softmax(2 * rng.standard_normal((60, V)).astype(np.float32))
    short = workloads.peaky(rng, y[:50], 300, V)
    es, ys = [e, short], [y, y[:50]]
    k = RC.knob_vector(chunk_frames=16, **knobs)
    print(f"global slots {knobs}", flush=True)
    got = op_align(es, ys, [0, 0], k)
    want = oracle_align(es, ys, [0, 0], k)
    assert_same(got, want, where="global-slots ")
    assert got["repair_passes"][0] > 0 or got["routing_stats"][0, 0] == 2
    if knobs == dict(repair_budget_frames=0):
        assert got["repair_passes"][0] == 2 and got["stitched"][0] == 1


@pytest.mark.parametrize("knobs", [dict(repair_budget_frames=0), dict(repair_budget_frames=0, frontier_min_frames=1 << 30)],
                         ids=["counted", "uncounted"])
def test_global_slots_resume_from_saved_frontiers(knobs):
    """chunk_frames = 32 and 16,500 frames: 516 chunks in global-memory slots,
    each with a saved frontier (every optimized-mode record keeps them at
    chunk_frames >= 32). The repairs resume from them whether or not the
    reference's reuse gating counts the record in reuse_stats."""
    rng = np.random.default_rng(516)
    T, V = 16500, 8
    y = rng.integers(1, V, size=1200).astype(np.int64)
    e = workloads.peaky(rng, y, T, V)
    e[3000:3040] = rng.integers(-2, 1, (40, V)).astype(np.float32)
    e[9000:9060] = workloads._log_softmax(2 * rng.standard_normal((60, V)).astype(np.float32))
    k = RC.knob_vector(chunk_frames=32, **knobs)
    print(f"global slots with frontiers {knobs}", flush=True)
    got = op_align([e], [y], [0], k)
    want = oracle_align([e], [y], [0], k)
    assert_same(got, want, where="global-slot frontiers ")
    assert got["repair_passes"][0] > 0
    if "frontier_min_frames" in knobs:
        assert got["reuse_stats"].shape == (0, 4)
    else:
        assert got["reuse_stats"][0, 0] > 0  # frames resumed by the repairs
