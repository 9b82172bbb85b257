"""GPU parity for the banded DP: conventional mode on batches with transcripts
of more than 1,024 states, where every record's states are cut into bands of
256 (one wave each) that run as workgroups of their own and hand the last
state of each frame to the next band through global memory.

Every output is compared with the CPU oracle bit for bit:
* wide records of 18 and 19 bands (the second with a last band of one state,
  so the terminal candidates S-1 and S-2 sit in different bands);
* a batch mixing a wide record with narrow and one-band records, an empty
  transcript, a tight record, an infeasible one (status 4), one with an
  out-of-vocabulary token (status 3) and one whose DP has no finite path
  (status 1);
* more than 64 records (the record table uploaded instead of passed in the
  kernel arguments);
* integer ties and near-flat rows across band boundaries;
* repeated calls on one stream and calls on two streams in flight (the edge
  arrays are zeroed per call in each call's own workspace).
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


def _wide(rng, U, T, V=32, kind="peaky"):
    y = rng.integers(1, V, size=U).astype(np.int64)
    if kind == "peaky":
        return workloads.peaky(rng, y, T, V), y
    if kind == "ties":
        return rng.integers(-3, 1, (T, V)).astype(np.float32), y
    return workloads._log_softmax((0.01 * rng.standard_normal((T, V))).astype(np.float32)), y


def _run(es, ys, blanks=0, check_inputs=True):
    e = [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in es]
    y = [torch.from_numpy(np.ascontiguousarray(x, dtype=np.int64)).cuda() for x in ys]
    r = ffa.align(e, y, blank_id=blanks, mode="conventional", check_inputs=check_inputs)
    out = {f: getattr(r, f).cpu().numpy() for f in FIELDS}
    out["lengths"] = r.lengths
    return out


def _check(es, ys, blanks=0, check_inputs=True, where=""):
    got = _run(es, ys, blanks, check_inputs)
    want = O.align(es, ys, blank_id=blanks, mode="conventional", check_inputs=check_inputs, threads=8)
    assert got["lengths"] == want["lengths"]
    assert_same(got, want, where=where)
    return got


def test_wide_records():
    rng = np.random.default_rng(4401)
    a = _wide(rng, 2200, 3000)          # S = 4401: 18 bands
    b = _wide(rng, 2304, 3100)          # S = 4609: 19 bands, the last holds state 4608 only
    print("band: 18 and 19 bands", flush=True)
    got = _check([a[0], b[0]], [a[1], b[1]], where="wide ")
    assert (got["status"] == 0).all()


def test_mixed_batch_statuses():
    rng = np.random.default_rng(77)
    V = 32
    recs = [_wide(rng, 2500, 4000)]
    recs.append(_wide(rng, 100, 400))                  # one band
    recs.append(_wide(rng, 400, 900))                  # four bands
    recs.append((workloads._log_softmax(rng.standard_normal((50, V)).astype(np.float32)), np.zeros(0, np.int64)))
    y = rng.integers(1, V, size=2100).astype(np.int64)
    R = int((y[1:] == y[:-1]).sum())
    recs.append((workloads.peaky(rng, y, 2100 + R, V), y))                                       # tight
    recs.append((workloads._log_softmax(rng.standard_normal((2100 + R - 1, V)).astype(np.float32)), y))  # status 4
    bad = y.copy()
    bad[1500] = V
    recs.append((workloads.peaky(rng, y, 3000, V), bad))                                        # status 3
    # no finite path: the first token's column is -inf in every frame
    e = workloads.peaky(rng, y, 3000, V)
    e[:, y[0]] = -np.inf
    recs.append((e, y))
    print("band: mixed batch", flush=True)
    got = _check([r[0] for r in recs], [r[1] for r in recs], where="mixed ")
    assert got["status"].tolist() == [0, 0, 0, 0, 0, 4, 3, 1]


def test_uploaded_table():
    rng = np.random.default_rng(70)
    recs = [_wide(rng, int(rng.integers(20, 200)), int(rng.integers(500, 800))) for _ in range(69)]
    recs.insert(33, _wide(rng, 2100, 2600))
    print("band: 70 records", flush=True)
    _check([r[0] for r in recs], [r[1] for r in recs], where="uploaded ")


@pytest.mark.parametrize("kind", ["ties", "flat"])
def test_ties_across_bands(kind):
    rng = np.random.default_rng(5 if kind == "ties" else 6)
    e, y = _wide(rng, 2300, 2800, kind=kind)
    e2, y2 = _wide(rng, 2050, 2400, V=300)
    print(f"band: {kind}", flush=True)
    _check([e, e2], [y, y2], blanks=[0, 7], where=f"{kind} ")


def test_repeated_calls_and_two_streams():
    rng = np.random.default_rng(12)
    b1 = [_wide(rng, 2200, 2700), _wide(rng, 300, 700)]
    b2 = [_wide(rng, 2600, 3300)]
    w1 = O.align([r[0] for r in b1], [r[1] for r in b1], mode="conventional", threads=8)
    w2 = O.align([r[0] for r in b2], [r[1] for r in b2], mode="conventional", threads=8)
    dev = lambda b: ([torch.from_numpy(r[0]).cuda() for r in b], [torch.from_numpy(r[1]).cuda() for r in b])
    i1, i2 = dev(b1), dev(b2)
    print("band: repeated calls", flush=True)
    for i in range(8):
        r = ffa.align(*i1, mode="conventional")
        assert_same({f: getattr(r, f).cpu().numpy() for f in FIELDS}, w1, where=f"call {i} ")
    print("band: two streams", flush=True)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for s in (s1, s2):
        s.wait_stream(torch.cuda.current_stream())
    out1, out2 = [], []
    for _ in range(4):
        with torch.cuda.stream(s1):
            out1.append(ffa.align(*i1, mode="conventional"))
        with torch.cuda.stream(s2):
            out2.append(ffa.align(*i2, mode="conventional"))
    torch.cuda.synchronize()
    for r in out1:
        assert_same({f: getattr(r, f).cpu().numpy() for f in FIELDS}, w1, where="stream 1 ")
    for r in out2:
        assert_same({f: getattr(r, f).cpu().numpy() for f in FIELDS}, w2, where="stream 2 ")


def _op(es, ys, knobs):
    import repair_cases as RC  # noqa: F401  (knob vectors)
    e = [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in es]
    y = [torch.from_numpy(np.ascontiguousarray(x, dtype=np.int64)).cuda() for x in ys]
    k = knobs
    with torch.inference_mode():
        tensors, _ = torch.ops.fast_forced_aligner_cuda.align(
            e, y, [0] * len(es), k["chunk_frames"], k["mode"], k["threads"], k["repair_rounds"],
            k["optimization_pass"], k["variant"], k["repair_budget_frames"], k["repair_threads"],
            k["compact_alphabet"], k["parallel_traceback"], k["overlap_fallback"], k["trace_min_frames"],
            k["repair_min_frames"], k["frontier_reuse"], k["frontier_min_frames"], None, True)
    return {f: t.cpu().numpy() for f, t in zip(FIELDS, tensors)}


@pytest.mark.parametrize("knobs", [dict(repair_rounds=0), dict(overlap_fallback=False)],
                         ids=["no_repair_rounds", "overlap_off"])
def test_optimized_fallback_after_failed_seams(knobs):
    """Optimized mode, transcripts of more than 4,096 states (K = 32) whose
    seams still fail after the repair rounds: the fallback (cu:552-559) runs
    as a banded DP after the tail, without the split tail (no repair rounds)
    and with it (overlap fallback off)."""
    import repair_cases as RC
    rng = np.random.default_rng(552)
    es, ys = [], []
    for T, U in ((4600, 2200), (4300, 2100)):
        e, y = _wide(rng, U, T)
        # noisy spans: illegal seams around them; the 700-frame one makes any repair
        # region exceed the 512-frame budget, so with overlap off no round repairs it
        for start, width in ((900, 700), (2800, 150), (3700, 150)):
            e[start:start + width] = workloads._log_softmax(2 * rng.standard_normal((width, 32)).astype(np.float32))
        es.append(e)
        ys.append(y)
    e, y = _wide(rng, 150, 600)
    es.append(e)
    ys.append(y)
    k = RC.knob_vector(**knobs)
    print(f"band: optimized fallback after failed seams {knobs}", flush=True)
    got = _op(es, ys, k)
    want = O.align(es, ys, blank_id=[0] * len(es), options=RC.oracle_options(k), threads=8)
    assert_same(got, want, where=f"fallback {knobs} ")
    assert (got["stitched"][:2] == 0).all() and (got["status"][:2] == 0).all()  # the fallback aligned them

