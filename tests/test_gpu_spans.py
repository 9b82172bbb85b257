"""GPU token spans (spans_kernel via the package's token_spans) against the
oracle restatement of the reference README's timestamp rule, on the outputs of
real alignments: every configuration's records, failed records, per-record
blanks, empty targets, transcripts holding the blank id, and long records."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import fast_forced_aligner as ffa
from fast_forced_aligner import workloads
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def check(emissions, targets, blank=0, mode="optimized", check_inputs=True):
    es = [torch.from_numpy(np.ascontiguousarray(e)).to(DEV) for e in emissions]
    ys = [torch.from_numpy(np.ascontiguousarray(y, dtype=np.int64)).to(DEV) for y in targets]
    result = ffa.align(es, ys, blank_id=blank, mode=mode, check_inputs=check_inputs)
    spans = ffa.token_spans(result, ys, blank_id=blank)
    labels = result.labels.cpu().numpy()
    status = result.status.cpu().numpy()
    want = O.token_spans(labels, result.lengths, [y.size for y in targets], status, blank)
    got = spans.spans.cpu().numpy()
    assert got.shape == want.shape and np.array_equal(got, want)
    # invariant: successful records have one run per token, labelled with that token
    for path, span, y, st in zip(np.split(labels, np.cumsum(result.lengths)[:-1]), spans.split(), targets, status):
        if st == 0 and (np.asarray(y) != (blank if isinstance(blank, int) else 0)).all():
            s = span.cpu().numpy()
            assert (s[:, 0] < s[:, 1]).all()
            assert path[s[:, 0]].tolist() == list(y)
    return spans, status


@pytest.mark.parametrize("config", ["c1", "c2", "c5"])
def test_spans_on_configs(config):
    b = workloads.make(config)
    print(f"spans {config}", flush=True)
    spans, status = check(b.emissions, b.targets)
    assert spans.lengths == tuple(int(y.size) for y in b.targets)
    if config == "c5":
        assert (status == 4).any()  # infeasible rows produce -1 spans


def test_spans_ragged_blanks_empty_and_long():
    rng = np.random.default_rng(21)
    es, ys, blanks = [], [], []
    for i in range(20):
        V = int(rng.choice([5, 32, 40]))
        blank = int(rng.integers(0, V))
        vocab = np.array([v for v in range(V) if v != blank])
        U = 0 if i % 7 == 0 else int(rng.integers(1, 80))
        y = rng.choice(vocab, U).astype(np.int64)
        T = int(rng.integers(2 * U + 2, 2 * U + 3000))
        es.append(workloads.peaky(rng, y, T, V, blank) if U else np.log(rng.dirichlet(np.ones(V), T)).astype(np.float32))
        ys.append(y)
        blanks.append(blank)
    print("spans ragged", flush=True)
    check(es, ys, blanks)


def test_spans_blank_inside_targets_unchecked():
    e = np.full((300, 32), -9.0, dtype=np.float32)
    e[:150, 0] = 0.0
    e[150:, 5] = 0.0
    spans, status = check([e], [np.array([0, 5])], check_inputs=False)
    assert spans.spans.cpu().tolist()[-1] == [-1, -1]  # one run for two tokens


def test_spans_seconds_and_no_host_sync():
    b = workloads.c1()
    es = [torch.from_numpy(e).to(DEV) for e in b.emissions]
    ys = [torch.from_numpy(y).to(DEV) for y in b.targets]
    result = ffa.align(es, ys)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        spans = ffa.token_spans(result, ys)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    seconds = spans.seconds(0.02)
    assert seconds.dtype == torch.float64
    assert torch.equal(seconds, spans.spans.double() * 0.02)
