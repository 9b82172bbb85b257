"""Fused logits path (``align_logits``) and the materialized ``log_softmax``.

Parity contract: ``align_logits(x)`` returns every output of
``align(log_softmax(x))`` bit for bit (``log_softmax`` materializes exactly the
values the fused kernels compute), and through that the CPU oracle's outputs on
those values; ``log_softmax`` itself matches a float64 log-softmax within
``atol=3e-5, rtol=1e-6`` (the fp32 rounding of ``(x - m) - log(sum)``; a dropped
max or normalizer term is off by O(1)).
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
DEV = "cuda"
MODES = ["conventional", "optimized"]


def dev(arrays, dtype=None):
    return [torch.from_numpy(np.ascontiguousarray(a, dtype=dtype)).to(DEV) for a in arrays]


def same_bits(a, b, where):
    """Equal tensors, NaN payloads aside (NaN positions must agree)."""
    assert a.shape == b.shape and a.dtype == b.dtype, where
    if a.dtype.is_floating_point:
        nan = torch.isnan(a)
        assert torch.equal(nan, torch.isnan(b)), where
        a, b = a.masked_fill(nan, 0), b.masked_fill(nan, 0)
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), where
    else:
        assert torch.equal(a, b), where


def fused_equals_materialized(logits, targets, blank=0, mode="optimized", **kw):
    fused = ffa.align_logits(logits, targets, blank_id=blank, mode=mode, **kw)
    log_probs = ffa.log_softmax(logits)
    plain = ffa.align(log_probs, targets, blank_id=blank, mode=mode, **kw)
    assert fused.lengths == plain.lengths
    for f in FIELDS:
        same_bits(getattr(fused, f), getattr(plain, f), f"{mode}:{f}")
    return fused, log_probs


@pytest.mark.parametrize("vocab", [1, 2, 3, 4, 7, 31, 32, 33, 64, 65, 127, 300, 1024, 8192])
def test_log_softmax_matches_float64(vocab):
    generator = torch.Generator(device=DEV).manual_seed(vocab)
    frames = 300 if vocab <= 1024 else 40
    x = torch.randn(frames, vocab, generator=generator, device=DEV) * 6 + 3
    x[::7, ::3] = -torch.inf  # masked vocabulary entries
    x[5] = 80.0  # a constant row
    ours = ffa.log_softmax([x])[0]
    ref = torch.log_softmax(x.double(), -1)
    finite = torch.isfinite(ref)
    assert torch.equal(finite, torch.isfinite(ours))
    torch.testing.assert_close(ours.double()[finite], ref[finite], atol=3e-5, rtol=1e-6)
    assert torch.equal(torch.isneginf(ours), torch.isneginf(ref))
    # rows are normalized: logsumexp of the output is 0 up to fp32 rounding
    rows = ~torch.isnan(ref).any(-1)  # an all -inf row is NaN, as in torch
    lse = torch.logsumexp(ours.double()[rows], -1)
    assert lse.abs().max().item() < 1e-5
    # a constant row is -log(V) in every column
    assert torch.equal(ours[5], ours[5, :1].expand(vocab))
    assert abs(ours[5, 0].item() + np.log(vocab)) < 1e-5


def test_log_softmax_special_rows_follow_torch():
    x = torch.randn(6, 16, device=DEV)
    x[0, 3] = torch.nan
    x[1, 4] = torch.inf
    x[2] = -torch.inf
    x[3, :8] = -torch.inf
    x[4] = 0.0
    x[4, 0] = -0.0
    ours = ffa.log_softmax([x])[0]
    ref = torch.log_softmax(x, -1)
    assert torch.equal(torch.isnan(ours), torch.isnan(ref))
    keep = ~torch.isnan(ref)
    torch.testing.assert_close(ours[keep], ref[keep], atol=1e-6, rtol=1e-6)


def test_log_softmax_ragged_batch_and_views():
    generator = torch.Generator(device=DEV).manual_seed(3)
    storage = torch.randn(40 * 33 + 1, generator=generator, device=DEV)
    xs = [torch.randn(t, v, generator=generator, device=DEV) for t, v in ((1, 5), (129, 32), (700, 40), (3, 1024))]
    xs.append(storage[1:].view(40, 33))  # 4 bytes off 16-byte alignment
    outs = ffa.log_softmax(xs)
    for x, y in zip(xs, outs):
        assert y.shape == x.shape and y.is_contiguous()
        torch.testing.assert_close(y.double(), torch.log_softmax(x.double(), -1), atol=3e-5, rtol=1e-6)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("config", ["c1", "c2", "c4", "c5"])
def test_fused_equals_materialized_on_configs(mode, config):
    kwargs = {"c4": {"batch": 32}, "c5": {"batch": 256}}.get(config, {})
    b = workloads.make(config, raw=True, **kwargs)
    print(f"{config} {mode}", flush=True)
    logits, targets = dev(b.emissions), dev(b.targets, np.int64)
    fused, _ = fused_equals_materialized(logits, targets, mode=mode)
    if config != "c5":
        assert (fused.status == 0).all()
    fused_equals_materialized(logits, targets, mode=mode, check_inputs=False)


@pytest.mark.parametrize("mode", MODES)
def test_fused_matches_the_oracle(mode):
    b = workloads.c2(batch=16, raw=True)
    logits, targets = dev(b.emissions), dev(b.targets, np.int64)
    fused = ffa.align_logits(logits, targets, mode=mode)
    log_probs = [x.cpu().numpy() for x in ffa.log_softmax(logits)]
    want = O.align(log_probs, b.targets, blank_id=0, mode=mode, threads=8)
    got = {f: getattr(fused, f).cpu().numpy() for f in FIELDS}
    assert fused.lengths == want["lengths"]
    assert_same(got, want, where=f"logits[{mode}] ")


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("seed", [0, 1])
def test_fused_random_ragged_batches(mode, seed):
    """Ragged batches over vocabularies that take every read path (greedy fast
    path with and without quads past V, general greedy, LDS-staged and
    gathered DP), ties, per-record blanks, empty targets and rows off 16-byte
    alignment."""
    rng = np.random.default_rng(300 + seed)
    logits, targets, blanks = [], [], []
    for i in range(20):
        V = int(rng.choice([3, 6, 12, 28, 32, 40, 300]))
        blank = int(rng.integers(0, V))
        vocab = np.array([v for v in range(V) if v != blank])
        U = int(rng.integers(0, 50))
        y = rng.choice(vocab, U).astype(np.int64)
        R = int((y[1:] == y[:-1]).sum())
        T = int(rng.integers(max(1, U + R), U + R + 400))
        if i % 3 == 0 or U == 0:
            x = np.round(rng.standard_normal((T, V)) * 2).astype(np.float32)  # integer logits: many ties
        else:
            x = workloads.peaky(rng, y, T, V, blank, raw=True)
        t = torch.from_numpy(x).to(DEV)
        if i % 5 == 1:  # a contiguous view one float past a 16-byte boundary
            holder = torch.empty(x.size + 1, device=DEV)
            holder[1:] = t.flatten()
            t = holder[1:].view(T, V)
        logits.append(t)
        targets.append(torch.from_numpy(y).to(DEV))
        blanks.append(blank)
    fused_equals_materialized(logits, targets, blank=blanks, mode=mode)


@pytest.mark.parametrize("mode", MODES)
def test_fused_long_records_use_tail_statistics(mode):
    """T >= 2048: repairs, frontier reuse and the full fallback DP read the row
    statistics the chunk kernel stored (optimized) or the pre-pass (conventional)."""
    b = workloads.c3(batch=2, frames=6000, tokens=1800, raw=True)
    logits, targets = dev(b.emissions), dev(b.targets, np.int64)
    fused, _ = fused_equals_materialized(logits, targets, mode=mode)
    assert (fused.status == 0).all()
    if mode == "optimized":
        assert fused.reuse_stats.shape == (2, 4)


@pytest.mark.parametrize("mode", MODES)
def test_fused_widest_transcripts(mode):
    """More than 8,192 states (K = 32): the chunk DP, repairs and fallback run
    in the non-inlined DP function, which reads the row statistics through the
    record view (from LDS in the chunk kernel, from global memory in the tail)."""
    b = workloads.c3(batch=2, frames=8300, tokens=2500, raw=True)
    print(f"K = 32 logits {mode}", flush=True)
    logits, targets = dev(b.emissions), dev(b.targets, np.int64)
    fused, _ = fused_equals_materialized(logits, targets, mode=mode)
    assert (fused.status == 0).all()


def test_fused_mask_and_statuses():
    b = workloads.c5(batch=64, raw=True)
    logits, targets = dev(b.emissions), dev(b.targets, np.int64)
    poisoned = b.notes["kinds"].index("peaky")
    logits[poisoned][0, 0] = torch.nan
    mask = ffa.emission_validity(logits)
    assert not mask[poisoned].item()
    for mode in MODES:
        fused, _ = fused_equals_materialized(logits, targets, mode=mode, emission_validity=mask)
        assert fused.status[poisoned].item() == 2
