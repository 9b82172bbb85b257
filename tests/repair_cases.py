"""Hand-derived optimized-mode cases: inputs whose repair-round, budget and
frontier diagnostics follow, on paper, from the reference's rules.

Every expected value below is derived from src/fast_forced_aligner/csrc/
alignment.cu by hand, not by running an implementation:

  * greedy_shortcuts (:29-153): a chunk is a shortcut when every frame has a
    unique finite maximum over the transcript alphabet and the pattern of
    label changes has exactly one legal placement;
  * chunk DP (:400-523): relaxed start for a > 0 (every state starts at
    e[a][l[s]]), strict '>' so ties keep stay > advance > skip, chunk terminal
    = lowest-index argmax, record terminal = S-2 when alpha[S-2] >= alpha[S-1];
  * legal_seam (:157-161), plan_repairs with its budget preflight (:163-228),
    frontier resume (:374-385), validate_seams (:561-592) and the fallbacks
    (:534-559, :767-780).

Emission rows are "<label>-frames": the named label scores 0 and every other
column -10, except for the per-case overrides noted. Values are small
integers, so every fp32 sum is exact. Blank is 0 and V = 4 (8 for the
five-token case), so the chunk kernel's register fast path (V <= 32,
V % 4 == 0) takes the greedy chunks on the GPU.

Each case is a dict: emissions [T, V] fp32, targets, knobs (overrides of the
public API's vector, alignment.py:496-501) and `expect`, the ten outputs'
values (labels/scores as arrays; diagnostics as lists).
"""
from __future__ import annotations

import numpy as np

V = 4


def _rows(spec, T, overrides=(), vocab=V):
    """spec: list of (first_frame, label) runs; overrides: (frame, column, value)."""
    e = np.full((T, vocab), -10.0, np.float32)
    bounds = [a for a, _ in spec] + [T]
    for (a, label), b in zip(spec, bounds[1:]):
        e[a:b, label] = 0.0
    for frame, column, value in overrides:
        e[frame, column] = value
    return e


def one_seam():
    """(i) T = 512, targets [1, 2, 3] (S = 7, l = b 1 b 2 b 3 b), H = 128.
    Frames 0..255 are 1-frames, 256..511 are 3-frames; '2' scores -1 on every
    frame, so the per-frame argmax never shows it.

    Greedy: chunks 0 and 1 place at state 1 (start = end = 1), chunks 2 and 3
    at state 5 (chunk 3 ends the record: 5 >= S-2). All four are shortcuts
    with objective 0: shortcut_stats = [4, 512, 0].
    Seams: 1->1 legal, 1->5 (jump 4) illegal, 5->5 legal. Round 1 merges
    chunk 2 into chunk 1: interval [128, 384), repair_passes 1,
    repaired_frames 256 (T < 2048: no budget, no frontier).
    Repair DP over [128, 384) (relaxed start): '2' must sit on one frame at
    -1; frame 255 (path A) and frame 256 (path B) tie at -1, and at frame 257
    state 5 keeps 'stay' (A) over the equal skip (B). Terminal = unique argmax
    state 5 (-1), start state 1. Round 2 finds every seam legal and merges
    nothing. validate: objective 0 + (-1) + 0 = -1, stitched 1.
    Labels: 1 x 255, 2, 3 x 256; scores 0 except -1 at frame 255. The same as
    conventional DP (the same tie at frame 257)."""
    T = 512
    e = _rows([(0, 1), (256, 3)], T)
    e[:, 2] = -1.0
    labels = np.array([1] * 255 + [2] + [3] * 256, np.int64)
    scores = np.zeros(T, np.float32)
    scores[255] = -1.0
    return dict(name="one_seam", emissions=e, targets=np.array([1, 2, 3], np.int64), knobs={},
                expect=dict(labels=labels, scores=scores, status=[0], objective=[-1.0], stitched=[1],
                            repair_passes=[1], repaired_frames=[256], shortcut_stats=[[4, 512, 0]],
                            routing_stats=[[0, 0, 0]], reuse_rows=0))


def two_merges():
    """(ii-a) T = 1024, V = 8, targets [1, 2, 3, 4, 5] (S = 11), H = 128. Frames
    0..255 are 1-frames, 256..767 3-frames, 768..1023 5-frames; '2' and '4'
    score -1 on every frame.

    All eight chunks are shortcuts (start = end = 1, 1, 5, 5, 5, 5, 9, 9):
    shortcut_stats = [8, 1024, 0]. Seams 1->5 (chunk 1|2) and 5->9 (chunk 5|6)
    are illegal, so one round makes two disjoint merges, [128, 384) and
    [640, 896): repair_passes 1, repaired_frames 256 + 256 = 512.
    Repair DP [128, 384): '4' (state 7) reaches only -2 at frame 383 (skip
    from state 5 then -1 per frame), so state 5 at -1 is the unique argmax;
    start 1, '2' at frame 255 as in one_seam. Repair DP [640, 896): the same
    shifted by four states: start 5, end 9, '4' at frame 767, objective -1.
    Round 2 merges nothing. objective = 0 - 1 + 0 + 0 - 1 + 0 = -2, stitched 1."""
    T = 1024
    e = _rows([(0, 1), (256, 3), (768, 5)], T, vocab=8)  # columns 6, 7 unused (-10)
    e[:, 2] = -1.0
    e[:, 4] = -1.0
    labels = np.array([1] * 255 + [2] + [3] * 511 + [4] + [5] * 256, np.int64)
    scores = np.zeros(T, np.float32)
    scores[[255, 767]] = -1.0
    return dict(name="two_merges", emissions=e,
                targets=np.array([1, 2, 3, 4, 5], np.int64), knobs={},
                expect=dict(labels=labels, scores=scores, status=[0], objective=[-2.0], stitched=[1],
                            repair_passes=[1], repaired_frames=[512], shortcut_stats=[[8, 1024, 0]],
                            routing_stats=[[0, 0, 0]], reuse_rows=0))


def second_round():
    """(ii-b) T = 640, targets [1, 2] (S = 5, l = b 1 b 2 b), H = 128.
    Frames 0..255 1-frames, 256..383 blank-frames, 384..511 1-frames with
    blank -3 and '2' -7, 512..639 2-frames.

    Chunks 0, 1, 3 place at state 1, chunk 4 at state 3 (record end: 3 >= S-2).
    Chunk 2 (all blank) has three placements (states 0, 2, 4): ambiguous,
    shortcut_stats = [4, 512, 1]; its relaxed chunk DP ends at the lowest
    tied argmax, state 0, start 0.
    Round 1 seams: 1->1 legal, 1->0 illegal, 0->1 legal, 1->3 legal skip.
    Merge [128, 384); its repair DP ends at the unique argmax state 2 (0;
    state 4 and state 3 are -10), start 1. Round 2 sees the new end 2 before
    chunk 3's start 1 (jump -1): merge [128, 512), repair_passes 2,
    repaired_frames 256 + 384 = 640. That DP's best is state 2 at -3 x 128 =
    -384 (entering '2' costs at least -7 then blank -3: states 3 and 4 reach
    -388), start 1. Seams 1->1 and 2->3 are legal: stitched 1, objective
    0 + (-384) + 0 = -384. Labels 1 x 256, blank x 256, 2 x 128 (= conventional)."""
    T = 640
    e = _rows([(0, 1), (256, 0), (384, 1), (512, 2)], T)
    e[384:512, 0] = -3.0
    e[384:512, 2] = -7.0
    labels = np.array([1] * 256 + [0] * 256 + [2] * 128, np.int64)
    scores = np.zeros(T, np.float32)
    scores[384:512] = -3.0
    return dict(name="second_round", emissions=e, targets=np.array([1, 2], np.int64), knobs={},
                expect=dict(labels=labels, scores=scores, status=[0], objective=[-384.0], stitched=[1],
                            repair_passes=[2], repaired_frames=[640], shortcut_stats=[[4, 512, 1]],
                            routing_stats=[[0, 0, 0]], reuse_rows=0))


def blank_skip_seam():
    """(i') T = 256, targets [1, 2] (S = 5), H = 128. Frames 0..191 are
    blank-frames, 192..255 2-frames; '1' scores -1 on every frame, so the
    argmax never shows it.

    Chunk 0 (a = 0: start state 0 or 1) places its all-blank pattern only at
    state 0: start = end = 0. Chunk 1's pattern blank -> '2' ends the record
    (terminal >= S-2 = 3), which leaves state 2 (state 0 would end at 1, state
    4 past S): start 2, end 3. shortcut_stats = [2, 256, 0].
    The seam 0 -> 2 is a jump of two into a blank state: illegal, so round 1
    merges the record into [0, 256): repair_passes 1, repaired_frames 256.
    Its DP (standard start) is conventional DP: state 1 advances from state 0
    at every frame (0 > -1), state 2 enters at frame 1 (-1) and then keeps
    stay on the tie with state 1; frame 192 enters '2' from state 2. Path:
    '1' at frame 0 (-1), blank 1..191, '2' 192..255; objective -1, stitched 1."""
    T = 256
    e = _rows([(0, 0), (192, 2)], T)
    e[:, 1] = -1.0
    labels = np.array([1] + [0] * 191 + [2] * 64, np.int64)
    scores = np.zeros(T, np.float32)
    scores[0] = -1.0
    return dict(name="blank_skip_seam", emissions=e, targets=np.array([1, 2], np.int64), knobs={},
                expect=dict(labels=labels, scores=scores, status=[0], objective=[-1.0], stitched=[1],
                            repair_passes=[1], repaired_frames=[256], shortcut_stats=[[2, 256, 0]],
                            routing_stats=[[0, 0, 0]], reuse_rows=0))


def frontier_resume():
    """(iii) T = 2048 (budget 512, overlap and frontier reuse active: T >=
    2048), targets [1, 2, 3] (S = 7), H = 128. Frames 0..255 1-frames, frame
    200 also scores 0 on the blank (a tie), frames 256..2047 3-frames with '2'
    at -1 (so '2' costs -10 before frame 256 and -1 from it).

    Chunk 1 has a tied frame: no shortcut, relaxed chunk DP over [128, 256):
    state 1 stays at 0, unique argmax: start = end = 1; it saves its frontier
    (reuse[2] += S). The other 15 chunks are shortcuts: shortcut_stats =
    [15, 1920, 0]. Seam 1->5 between chunks 1 and 2 is illegal.
    Preflight: the proposed region [128, 384) spans 256 <= 512 frames: no
    rejection. Round 1 merges [128, 384): repair_passes 1, repaired_frames
    256. Its DP resumes from chunk 1's frontier at frame 256 (saved end 256 in
    (128, 384]): reuse[0] += 256 - 128, reuse[3] += S, reuse[2] += S. From
    frame 256: '2' at frame 256 (-1, skip from state 1), '3' from 257;
    terminal state 5 at -1, start 1. Round 2 merges nothing.
    reuse_stats = [128, 0, 14, 7]; objective -1, stitched 1; labels 1 x 256,
    2, 3 x 1791 (= conventional)."""
    T = 2048
    e = _rows([(0, 1), (256, 3)], T, overrides=[(200, 0, 0.0)])
    e[256:, 2] = -1.0
    labels = np.array([1] * 256 + [2] + [3] * 1791, np.int64)
    scores = np.zeros(T, np.float32)
    scores[256] = -1.0
    return dict(name="frontier_resume", emissions=e, targets=np.array([1, 2, 3], np.int64), knobs={},
                expect=dict(labels=labels, scores=scores, status=[0], objective=[-1.0], stitched=[1],
                            repair_passes=[1], repaired_frames=[256], shortcut_stats=[[15, 1920, 0]],
                            routing_stats=[[0, 0, 0]], reuse_stats=[[128, 0, 14, 7]], reuse_rows=1))


def _budget_rows():
    """T = 2048, targets [1, 2, 3], H = 128. Chunk k holds 1-frames for
    k in {0, 2, 4} and 3-frames otherwise; chunk 0's frame 50 ties the blank
    with '1' (so chunk 0 takes the chunk DP); on the 3-frames of chunks 1 and 3
    '1' scores -1; on chunks 5..15 '2' scores -5."""
    T = 2048
    e = _rows([(0, 1), (128, 3), (256, 1), (384, 3), (512, 1), (640, 3)], T, overrides=[(50, 0, 0.0)])
    e[128:256, 1] = -1.0
    e[384:512, 1] = -1.0
    e[640:, 2] = -5.0
    labels = np.array([1] * 640 + [2] + [3] * 1407, np.int64)
    scores = np.zeros(T, np.float32)
    scores[128:256] = -1.0
    scores[384:512] = -1.0
    scores[640] = -5.0
    return e, labels, scores


def budget_reject_no_overlap():
    """(iv) The _budget_rows record with overlap_fallback = False.

    Chunk 0 is a chunk DP (standard start at a = 0): state 1 at 0 is the
    unique argmax, start = end = 1, frontier saved (reuse[2] = S). Chunks 1..15
    are shortcuts (states 5, 1, 5, 1, then 5): shortcut_stats = [15, 1920, 0].
    Seams 0|1 .. 4|5 are all illegal (jumps +4 / -4), 5|6 on are legal.
    Budget preflight (T >= 2048, budget 512): begin stays 0 and the proposed
    span grows 256, 384, 512, 640 (> 512: reject), 768. Each of the two
    rounds rejects: routing_stats = [0, 2, 768]; without overlap nothing is
    queued and no interval merges (repair_passes 0, repaired_frames 0).
    validate_seams: illegal seams, stitched 0. The ordinary fallback DP then
    resumes from chunk 0's frontier at frame 128: reuse[1] = 128, reuse[3] = S.
    Its unique optimum keeps '1' through frame 639 (-1 on the 256 3-frames of
    chunks 1 and 3), '2' at frame 640 (-5), '3' after: objective -261."""
    e, labels, scores = _budget_rows()
    return dict(name="budget_reject_no_overlap", emissions=e, targets=np.array([1, 2, 3], np.int64),
                knobs=dict(overlap_fallback=False),
                expect=dict(labels=labels, scores=scores, status=[0], objective=[-261.0], stitched=[0],
                            repair_passes=[0], repaired_frames=[0], shortcut_stats=[[15, 1920, 0]],
                            routing_stats=[[0, 2, 768]], reuse_stats=[[0, 128, 7, 7]], reuse_rows=1))


def budget_reject_overlap():
    """(iv') The same record with the public API's knobs (overlap on): the
    round-1 rejection queues the record (routing 1) and the repair launch runs
    the full fallback at once, resuming from chunk 0's frontier (reuse[1] 128,
    reuse[3] S), then marks it done (routing 2); round 2, validate_seams and
    the final fallback skip it. routing_stats = [2, 1, 768]."""
    e, labels, scores = _budget_rows()
    return dict(name="budget_reject_overlap", emissions=e, targets=np.array([1, 2, 3], np.int64), knobs={},
                expect=dict(labels=labels, scores=scores, status=[0], objective=[-261.0], stitched=[0],
                            repair_passes=[0], repaired_frames=[0], shortcut_stats=[[15, 1920, 0]],
                            routing_stats=[[2, 1, 768]], reuse_stats=[[0, 128, 7, 7]], reuse_rows=1))


def one_seam_chunks_only():
    """one_seam in mode 1 (chunks without greedy, alignment.cu:3): every chunk
    takes the relaxed chunk DP. Chunk 1's DP keeps state 1 (0) over state 3
    (-1); chunk 2's keeps state 5; chunk 3 ends the record at S-2 = 5 (0 vs
    the trailing blank's -10). Same seams, same merge and repair as in mode 2,
    so the same outputs, except that no chunk is a shortcut."""
    case = one_seam()
    case.update(name="one_seam_mode1", knobs=dict(mode=1))
    case["expect"] = dict(case["expect"], shortcut_stats=[[0, 0, 0]])
    return case


def one_seam_no_repairs():
    """one_seam with repair_rounds = 0: validate_seams (repairs off) checks the
    original chunks, finds the 1->5 seam illegal (stitched 0) and the record
    takes the full fallback DP: the conventional path and objective -1;
    repair_passes and repaired_frames stay 0."""
    case = one_seam()
    case.update(name="one_seam_rounds0", knobs=dict(repair_rounds=0))
    case["expect"] = dict(case["expect"], stitched=[0], repair_passes=[0], repaired_frames=[0])
    return case


def second_round_one_round():
    """second_round with repair_rounds = 1: after the first merge the seam
    2->1 before chunk 3 stays illegal, so validate_seams leaves the record
    unstitched and the full fallback DP gives the conventional result
    (objective -384): repair_passes 1, repaired_frames 256."""
    case = second_round()
    case.update(name="second_round_rounds1", knobs=dict(repair_rounds=1))
    case["expect"] = dict(case["expect"], stitched=[0], repair_passes=[1], repaired_frames=[256])
    return case


def all_cases():
    return [one_seam(), two_merges(), second_round(), blank_skip_seam(), frontier_resume(), budget_reject_no_overlap(),
            budget_reject_overlap(), one_seam_chunks_only(), one_seam_no_repairs(), second_round_one_round()]


# The public API's knob vector (alignment.py:496-501) in optimized mode, by
# the operator's argument names (alignment.cu:1066-1068).
API_KNOBS = dict(chunk_frames=128, mode=2, threads=512, repair_rounds=2, optimization_pass=2, variant=2,
                 repair_budget_frames=512, repair_threads=0, compact_alphabet=False, parallel_traceback=True,
                 overlap_fallback=True, trace_min_frames=2048, repair_min_frames=2048, frontier_reuse=True,
                 frontier_min_frames=2048)


def knob_vector(**overrides):
    knobs = dict(API_KNOBS)
    unknown = set(overrides) - set(knobs)
    if unknown:
        raise KeyError(f"unknown knobs {sorted(unknown)}")
    knobs.update(overrides)
    return knobs


def oracle_options(knobs):
    """The oracle's Options for an operator knob vector (the knobs that change
    results; the rest choose geometry or a result-identical variant)."""
    from oracle import oracle as O

    return O.Options(chunk_frames=knobs["chunk_frames"], mode=knobs["mode"], repair_rounds=knobs["repair_rounds"],
                     repair_budget_frames=knobs["repair_budget_frames"],
                     overlap_fallback=int(knobs["overlap_fallback"]), repair_min_frames=knobs["repair_min_frames"],
                     frontier_reuse=int(knobs["frontier_reuse"]), frontier_min_frames=knobs["frontier_min_frames"],
                     check_inputs=1)


def check_expected(out, case):
    """Assert the outputs `out` (dict of numpy arrays) equal the case's
    hand-derived values, bit for bit."""
    x = case["expect"]
    name = case["name"]
    np.testing.assert_array_equal(out["labels"], x["labels"], err_msg=f"{name} labels")
    np.testing.assert_array_equal(np.asarray(out["scores"], np.float32).view(np.int32),
                                  np.asarray(x["scores"], np.float32).view(np.int32), err_msg=f"{name} scores")
    np.testing.assert_array_equal(np.asarray(out["objective"], np.float32).view(np.int32),
                                  np.asarray(x["objective"], np.float32).view(np.int32), err_msg=f"{name} objective")
    for field in ("status", "stitched", "repair_passes", "repaired_frames", "shortcut_stats", "routing_stats"):
        assert np.asarray(out[field]).tolist() == x[field], f"{name} {field}: {np.asarray(out[field]).tolist()}"
    assert np.asarray(out["reuse_stats"]).shape == (x["reuse_rows"], 4), f"{name} reuse rows"
    if x["reuse_rows"]:
        assert np.asarray(out["reuse_stats"]).tolist() == x["reuse_stats"], \
            f"{name} reuse_stats: {np.asarray(out['reuse_stats']).tolist()}"
