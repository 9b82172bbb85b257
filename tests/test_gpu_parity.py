"""GPU parity: every output of the HIP path equals the CPU oracle, bit for bit.

Labels, scores, statuses and all diagnostics are compared exactly (integer
and index outputs bit-exact; fp32 scores/objectives compared as bit patterns,
which is stricter than the 1e-5 relative tolerance the specification allows).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import fast_forced_aligner as ffa
from fast_forced_aligner import capi, workloads
from helpers import FIELDS, assert_same, collapse, golden_cases, split
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def run_gpu(emissions, targets, blank=0, mode="optimized", check_inputs=True, validity=None):
    es = [torch.from_numpy(np.ascontiguousarray(e)).to(DEV) for e in emissions]
    ys = [torch.from_numpy(np.ascontiguousarray(y, dtype=np.int64)).to(DEV) for y in targets]
    mask = None if validity is None else torch.tensor(validity, dtype=torch.bool, device=DEV)
    r = ffa.align(es, ys, blank_id=blank, mode=mode, check_inputs=check_inputs, emission_validity=mask)
    out = {f: getattr(r, f).cpu().numpy() for f in FIELDS}
    out["lengths"] = r.lengths
    return out


def compare(emissions, targets, blank=0, mode="optimized", check_inputs=True, validity=None, where=""):
    got = run_gpu(emissions, targets, blank, mode, check_inputs, validity)
    want = O.align(emissions, targets, blank_id=blank, mode=mode, check_inputs=check_inputs,
                   emission_validity=validity, threads=8)
    assert got["lengths"] == want["lengths"]
    assert_same(got, want, where=f"{where}[{mode}] ")
    return got


@pytest.mark.parametrize("mode", ["conventional", "optimized"])
def test_c1_plumbing(mode):
    b = workloads.c1()
    print(f"c1 {mode}", flush=True)
    got = compare(b.emissions, b.targets, mode=mode, where="c1")
    for p, y in zip(split(got["labels"], got["lengths"]), b.targets):
        assert collapse(p, 0).tolist() == y.tolist()


@pytest.mark.parametrize("mode", ["conventional", "optimized"])
def test_golden_vectors(mode):
    for name, e, y, blank, labels, scores in golden_cases():
        got = run_gpu([e], [y], blank, mode)
        if mode == "conventional" or name.startswith(("c1", "adapters", "example")):
            np.testing.assert_array_equal(got["labels"], labels, err_msg=name)
            np.testing.assert_array_equal(got["scores"].view(np.int32), scores.view(np.int32), err_msg=name)
        want = O.align([e], [y], blank_id=blank, mode=mode)
        assert_same(got, want, where=f"{name} ")


@pytest.mark.parametrize("mode", ["conventional", "optimized"])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_ragged_batches(mode, seed):
    """Ragged batches with ties, per-record blanks, empty targets, repeats and
    rows shorter than a chunk, over several vocabulary sizes."""
    rng = np.random.default_rng(100 + seed)
    es, ys, blanks = [], [], []
    for i in range(24):
        V = int(rng.choice([3, 6, 32, 40, 300]))
        blank = int(rng.integers(0, V))
        vocab = np.array([v for v in range(V) if v != blank])
        U = int(rng.integers(0, 60))
        y = rng.choice(vocab, U).astype(np.int64)
        if U > 3 and i % 4 == 0:
            y[1] = y[0]
        R = int((y[1:] == y[:-1]).sum())
        T = int(rng.integers(max(1, U + R), U + R + 400))
        kind = i % 3
        if kind == 0:
            e = rng.integers(-4, 1, (T, V)).astype(np.float32)
        elif kind == 1 and U:
            e = workloads.peaky(rng, y, T, V, blank)
        else:
            e = np.log(rng.dirichlet(np.ones(V), T)).astype(np.float32)
        es.append(e)
        ys.append(y)
        blanks.append(blank)
    print(f"random seed {seed} {mode}", flush=True)
    compare(es, ys, blanks, mode=mode, where=f"seed{seed}")


@pytest.mark.parametrize("mode", ["conventional", "optimized"])
def test_fast_path_narrow_vocabularies(mode):
    """The chunk kernel's register fast path (V <= 32, V % 4 == 0) for every V
    it takes: rows narrower than 32 columns leave quads past V, which must read
    as -inf. Targets sit near the top of the vocabulary, so the last real
    column often holds a row's maximum; integer rows add ties."""
    rng = np.random.default_rng(404)
    es, ys, blanks = [], [], []
    for i in range(24):
        V = (4, 8, 12, 16, 20, 24, 28, 32)[i % 8]
        blank = 0 if i % 3 else V - 1
        vocab = np.array([v for v in range(V) if v != blank])
        U = int(rng.integers(1, 80))
        y = rng.choice(vocab[-3:] if i % 2 else vocab, U).astype(np.int64)
        R = int((y[1:] == y[:-1]).sum())
        T = int(rng.integers(U + R, U + R + 500))
        if i % 4 == 3:
            e = rng.integers(-3, 1, (T, V)).astype(np.float32)
        else:
            e = workloads.peaky(rng, y, T, V, blank)
        es.append(e)
        ys.append(y)
        blanks.append(blank)
    print(f"narrow vocabularies {mode}", flush=True)
    got = compare(es, ys, blanks, mode=mode, where="narrow-V")
    if mode == "optimized":
        peaky = [i for i in range(24) if i % 4 != 3]
        assert (got["shortcut_stats"][peaky, 0] > 0).any()  # the fast path accepted chunks


@pytest.mark.parametrize("config", ["c2", "c4", "c5"])
@pytest.mark.parametrize("mode", ["conventional", "optimized"])
def test_config_parity(config, mode):
    b = workloads.make(config)
    print(f"{config} {mode}", flush=True)
    got = compare(b.emissions, b.targets, mode=mode, where=config)
    if config == "c5":
        kinds = b.notes["kinds"]
        status = got["status"]
        assert all(s == 4 for s, k in zip(status, kinds) if k == "infeasible")
        assert all(s == 0 for s, k in zip(status, kinds) if k != "infeasible")


@pytest.mark.parametrize("mode", ["conventional", "optimized"])
def test_c3_long_form_parity(mode):
    """Config C3 (4 x 30,000 frames, 9,000 tokens: 18,001 states, beyond the
    reference's 4,096-state limit): all ten outputs bit-exact with the oracle,
    including the T >= 2048 features (repair budget, early fallback, frontier
    reuse) and the windowed traceback over 30,000 frames."""
    b = workloads.make("c3")
    print(f"c3 {mode}", flush=True)
    got = compare(b.emissions, b.targets, mode=mode, where="c3")
    assert (got["status"] == 0).all()
    for p, y in zip(split(got["labels"], got["lengths"]), b.targets):
        assert collapse(p, 0).tolist() == y.tolist()


@pytest.mark.parametrize("config", ["c2", "c4", "c5"])
def test_optimized_equals_conventional(config):
    """Optimized mode equals conventional DP on the non-adversarial configs
    (labels, scores and statuses; objectives differ only in summation order)."""
    b = workloads.make(config)
    opt = run_gpu(b.emissions, b.targets, mode="optimized")
    conv = run_gpu(b.emissions, b.targets, mode="conventional")
    np.testing.assert_array_equal(opt["labels"], conv["labels"])
    np.testing.assert_array_equal(opt["scores"], conv["scores"])
    np.testing.assert_array_equal(opt["status"], conv["status"])


def test_unchecked_inputs_and_mask():
    rng = np.random.default_rng(5)
    es = [np.log(rng.dirichlet(np.ones(6), n)).astype(np.float32) for n in (7, 257, 130)]
    ys = [np.array([1, 1, 2]), np.array([2, 3]), np.array([1, 1])]
    es[2][:] = 0
    for mode in ("conventional", "optimized"):
        compare(es, ys, mode=mode, check_inputs=False, where="unchecked")
        compare(es, ys, mode=mode, validity=[True, False, True], where="mask")


def test_blank_inside_targets_unchecked():
    """Targets holding the blank id (accepted only with check_inputs=False). The
    greedy placement must follow the reference's literal state loop
    (alignment.cu:119-134): a blank target sits at an odd state, so e.g. an
    all-blank first chunk has two legal starts (0 and 1) and is ambiguous.
    Covers the two-wave fast path (V=32) and the general path (V=40, V=6)."""
    rng = np.random.default_rng(77)
    es, ys = [], []
    for i in range(18):
        V = (32, 40, 6)[i % 3]
        U = int(rng.integers(2, 40))
        y = rng.integers(1, V, size=U).astype(np.int64)
        y[rng.random(U) < 0.3] = 0
        if i % 6 == 0:
            y[0] = 0  # transcript starts with the blank: all-blank opening chunk
        T = int(rng.integers(2 * U + 2, 420))
        es.append(workloads.peaky(rng, y, T, V, 0))
        ys.append(y)
    print("blank inside targets", flush=True)
    for mode in ("optimized", "conventional"):
        compare(es, ys, mode=mode, check_inputs=False, where="blank-in-targets")
    # a hand-built case: targets [0, 5], the first 130 frames peaky on the blank
    e = np.full((300, 32), -9.0, dtype=np.float32)
    e[:200, 0] = 0.0
    e[200:, 5] = 0.0
    got = compare([e], [np.array([0, 5])], mode="optimized", check_inputs=False, where="[0,5]")
    assert got["shortcut_stats"][0, 2] >= 1  # the all-blank opening chunk is ambiguous


@pytest.mark.parametrize("mode", ["conventional", "optimized"])
def test_reference_operator_matches_package_entry(mode):
    """The operator with the reference schema (alignment.cu:1064-1070), called
    the way the reference's Python layer calls it (alignment.py:496-501),
    returns the same ten tensors and lengths as the package's direct entry."""
    b = workloads.c2(batch=12)
    es = [torch.from_numpy(e).to(DEV) for e in b.emissions]
    ys = [torch.from_numpy(y).to(DEV) for y in b.targets]
    ys[3] = torch.tensor([1, 40], device=DEV)  # a rejected record (status 3)
    optimized = mode == "optimized"
    got = ffa.align(es, ys, mode=mode)
    with torch.inference_mode():
        tensors, lengths = torch.ops.fast_forced_aligner_cuda.align(
            es, ys, [0] * len(es), 128, 2 if optimized else 0, 512, 2, 2, 2, 512 if optimized else 0, 0, False,
            True, optimized, 2048, 2048, optimized, 2048, None, True)
    assert tuple(lengths) == got.lengths
    for name, tensor in zip(FIELDS, tensors):
        mine = getattr(got, name)
        assert mine.dtype == tensor.dtype and mine.shape == tensor.shape, name
        assert torch.equal(mine, tensor), name
    assert got.status.tolist()[3] == 3


def test_c_abi_direct_call():
    """Drive the HIP library through its C entry points (ctypes), with caller-
    allocated device buffers, and compare with the oracle."""
    lib = capi.load()
    b = workloads.c1()
    es = [torch.from_numpy(e).to(DEV) for e in b.emissions]
    ys = [torch.from_numpy(y).to(DEV) for y in b.targets]
    recs = (capi.Record * 2)()
    for i, (e, y) in enumerate(zip(es, ys)):
        recs[i] = capi.Record(e.data_ptr(), y.data_ptr(), e.shape[0], e.shape[1], y.numel(), 0)
    for optimized in (False, True):
        o = capi.default_options(lib, optimized)
        plan = capi.Plan()
        capi.check(lib, lib.ffa_align_plan_batch(recs, 2, ctypes.byref(o), ctypes.byref(plan)))
        host = torch.empty(plan.table_bytes, dtype=torch.uint8)
        capi.check(lib, lib.ffa_align_describe(ctypes.byref(plan), recs, host.data_ptr(), plan.table_bytes))
        N, B = plan.total_frames, 2
        outs = {"labels": torch.empty(N, dtype=torch.int64, device=DEV),
                "scores": torch.empty(N, dtype=torch.float32, device=DEV),
                "status": torch.empty(B, dtype=torch.int32, device=DEV),
                "objective": torch.empty(B, dtype=torch.float32, device=DEV),
                "stitched": torch.empty(B, dtype=torch.int32, device=DEV),
                "repair_passes": torch.empty(B, dtype=torch.int32, device=DEV),
                "repaired_frames": torch.empty(B, dtype=torch.int64, device=DEV),
                "shortcut_stats": torch.empty(B, 3, dtype=torch.int64, device=DEV),
                "routing_stats": torch.empty(B, 3, dtype=torch.int32, device=DEV),
                "reuse_stats": torch.empty(plan.reuse_rows, 4, dtype=torch.int64, device=DEV)}
        out = capi.Outputs(*[outs[f].data_ptr() if outs[f].numel() else None for f in FIELDS])
        ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=DEV)
        stream = torch.cuda.current_stream().cuda_stream
        capi.check(lib, lib.ffa_align_launch(ctypes.byref(plan), ctypes.byref(o), host.data_ptr(), None,
                                             ctypes.byref(out), ws.data_ptr(), stream))
        torch.cuda.synchronize()
        got = {f: outs[f].cpu().numpy() for f in FIELDS}
        want = O.align(b.emissions, b.targets, mode="optimized" if optimized else "conventional")
        assert_same(got, want, where="capi ")


def test_emission_validity_scan():
    rng = np.random.default_rng(9)
    es = [np.log(rng.dirichlet(np.ones(7), n)).astype(np.float32) for n in (1, 5, 257, 3000)]
    es[1][2, 3] = np.nan
    es[2][0, 0] = np.inf
    es[3][-1, -1] = -np.inf
    mask = ffa.emission_validity([torch.from_numpy(e).to(DEV) for e in es])
    assert mask.dtype == torch.bool
    assert mask.cpu().tolist() == [O.emission_valid(e) for e in es] == [True, False, False, True]


def test_launch_floor_hook_runs_on_the_current_stream():
    """The measurement hook launches its empty kernel without error and leaves
    the stream usable; an alignment enqueued after it is unaffected."""
    lib = capi.load()
    stream = torch.cuda.current_stream().cuda_stream
    for shape in ((1, 64), (568, 192), (1024, 256)):
        assert lib.ffa_launch_floor(shape[0], shape[1], stream) == 0, lib.ffa_last_error()
    b = workloads.c1()
    got = run_gpu(b.emissions, b.targets, mode="optimized")
    torch.cuda.synchronize()
    want = O.align(b.emissions, b.targets, blank_id=0, mode="optimized")
    assert_same(got, want, where="after-floor ")


@pytest.mark.parametrize("mode", ["conventional", "optimized"])
def test_dp_wave_selection_boundaries(mode):
    """Records on both sides of the one-wave DP loop's limit (S = 255 and 257
    states with K = 4 states per thread, i.e. 64 and 65 threads) in a batch
    whose widest record (S = 1023) makes four-wave workgroups: the chunk DP,
    the repairs and the fallback of optimized mode and the conventional DP
    must agree with the oracle whichever loop each record takes."""
    rng = np.random.default_rng(2560)
    es, ys = [], []
    for U, kind in [(127, "ties"), (128, "ties"), (127, "peaky"), (128, "flat"), (256, "ties"), (511, "peaky"),
                    (130, "flat"), (64, "ties")]:
        V = 32
        y = rng.integers(1, V, U).astype(np.int64)
        R = int((y[1:] == y[:-1]).sum())
        T = int(rng.integers(U + R + 2, U + R + 600))
        if kind == "ties":
            e = rng.integers(-3, 1, (T, V)).astype(np.float32)
        elif kind == "flat":
            e = np.log(rng.dirichlet(np.ones(V) * 50, T)).astype(np.float32)
        else:
            e = workloads.peaky(rng, y, T, V, 0)
        es.append(e)
        ys.append(y)
    print(f"dp wave boundaries {mode}", flush=True)
    got = compare(es, ys, mode=mode, where="wave-boundary")
    if mode == "optimized":  # the tie and flat records take chunk DPs and repair rounds
        assert (got["repair_passes"] > 0).sum() >= 4 and (got["shortcut_stats"][:, 0] == 0).sum() >= 5


@pytest.mark.parametrize("mode", ["conventional", "optimized"])
@pytest.mark.parametrize("case", ["k16", "gather_k4", "gather_k8"])
def test_state_widths_and_gathered_rows(mode, case):
    """The DP at every state width and read path the configs leave out: K = 16
    (transcripts of 1,024 to 2,047 tokens, three-wave workgroups) with staged
    rows, and the gathered-row path (V > 64) in multi-wave workgroups at K = 4
    and K = 8, whose cross-wave exchange differs from the staged path's loops.
    Tie, flat and peaky rows make optimized mode run chunk DPs, repairs and
    fallbacks as well as greedy shortcuts."""
    rng = np.random.default_rng({"k16": 1600, "gather_k4": 1601, "gather_k8": 1602}[case])
    V, widest = {"k16": (32, 1300), "gather_k4": (100, 200), "gather_k8": (80, 600)}[case]
    es, ys = [], []
    for U, kind in [(widest, "peaky"), (widest - 7, "ties"), (widest // 2, "flat"), (widest // 3, "peaky"),
                    (40, "ties")]:
        y = rng.integers(1, V, U).astype(np.int64)
        R = int((y[1:] == y[:-1]).sum())
        T = int(rng.integers(U + R + 2, 2 * (U + R) + 300))
        if kind == "ties":
            e = rng.integers(-3, 1, (T, V)).astype(np.float32)
        elif kind == "flat":
            e = np.log(rng.dirichlet(np.ones(V) * 50, T)).astype(np.float32)
        else:
            e = workloads.peaky(rng, y, T, V, 0)
        es.append(e)
        ys.append(y)
    S = 2 * widest + 1
    K = 4
    while K < 32 and (S + K - 1) // K > 256:
        K *= 2
    assert K == {"k16": 16, "gather_k4": 4, "gather_k8": 8}[case] and (S + K - 1) // K > 64  # several waves
    print(f"state widths {case} {mode}", flush=True)
    compare(es, ys, mode=mode, where=case)


@pytest.mark.parametrize("mode", ["conventional", "optimized"])
def test_vocabulary_and_length_limits(mode):
    """The edges of the supported shapes in one ragged batch: a blank-only
    vocabulary (V = 1, empty transcript), single-frame records, the blank in
    the last column, the widest vocabulary (V = 8,192) with a peaky and a flat
    record, and V = 65 / 64 on either side of the LDS emission blocks."""
    rng = np.random.default_rng(8192)
    es, ys, blanks = [], [], []

    def add(e, y, blank):
        es.append(np.ascontiguousarray(e, dtype=np.float32))
        ys.append(np.asarray(y, dtype=np.int64))
        blanks.append(blank)

    add(workloads._log_softmax(rng.standard_normal((40, 1)).astype(np.float32)), [], 0)  # V = 1
    add(workloads._log_softmax(rng.standard_normal((1, 5)).astype(np.float32)), [3], 0)  # T = 1
    add(workloads._log_softmax(rng.standard_normal((1, 5)).astype(np.float32)), [], 4)   # T = 1, U = 0
    y = rng.integers(0, 39, size=60)
    add(workloads.peaky(rng, y, 300, 40, blank=39), y, 39)                              # blank = V - 1
    y = rng.integers(1, 8192, size=90)
    add(workloads.peaky(rng, y, 400, 8192), y, 0)                                       # V = 8192
    add(workloads._log_softmax(0.1 * rng.standard_normal((150, 8192)).astype(np.float32)),
        rng.integers(1, 8192, size=40), 0)
    for V in (64, 65):
        y = rng.integers(1, V, size=70)
        add(workloads.peaky(rng, y, 260, V), y, 0)
    print(f"shape limits {mode}", flush=True)
    got = compare(es, ys, blank=blanks, mode=mode, where="limits")
    assert (got["status"][[0, 1, 2, 3, 4, 6, 7]] == 0).all()
