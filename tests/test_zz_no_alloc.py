"""The allocation-free entry point (ffa_align_launch_noalloc): its outputs
equal ffa_align_launch's bit for bit, on calls in a row whose later batches
are smaller (the shared device array keeps the first call's contents): a
1,024-record batch (chunk and tail kernels), then a batch with a transcript of
more than 1,024 states (the banded DP, whose control words and edge arrays sit
in the fixed array too; near-flat rows, so that optimized mode sends it to the
early full fallback), then two batches that run as one launch with the fused
tail, whose arrival counters live in a second fixed array (12 C2 records, then
C1, whose records are repaired); and a batch beyond its fixed scratch is
refused."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from fast_forced_aligner import capi, workloads
from helpers import FIELDS, assert_same

DEV = "cuda"


def _records(es, ys):
    recs = (capi.Record * len(es))()
    for i, (e, y) in enumerate(zip(es, ys)):
        recs[i] = capi.Record(e.data_ptr(), y.data_ptr() if y.numel() else None, e.shape[0], e.shape[1],
                              y.numel(), 0)
    return recs


def _outputs(plan, count):
    N = plan.total_frames
    outs = {"labels": torch.full((N,), -7, dtype=torch.int64, device=DEV),
            "scores": torch.full((N,), 7.0, dtype=torch.float32, device=DEV),
            "status": torch.full((count,), 7, dtype=torch.int32, device=DEV),
            "objective": torch.full((count,), 7.0, dtype=torch.float32, device=DEV),
            "stitched": torch.full((count,), 7, dtype=torch.int32, device=DEV),
            "repair_passes": torch.full((count,), 7, dtype=torch.int32, device=DEV),
            "repaired_frames": torch.full((count,), 7, dtype=torch.int64, device=DEV),
            "shortcut_stats": torch.full((count, 3), 7, dtype=torch.int64, device=DEV),
            "routing_stats": torch.full((count, 3), 7, dtype=torch.int32, device=DEV),
            "reuse_stats": torch.full((plan.reuse_rows, 4), 7, dtype=torch.int64, device=DEV)}
    ptrs = capi.Outputs(*[outs[f].data_ptr() if outs[f].numel() else None for f in FIELDS])
    return outs, ptrs


def _run(lib, es, ys, optimized, noalloc):
    recs = _records(es, ys)
    o = capi.default_options(lib, optimized)
    plan = capi.Plan()
    capi.check(lib, lib.ffa_align_plan_batch(recs, len(es), ctypes.byref(o), ctypes.byref(plan)))
    host = torch.empty(plan.table_bytes, dtype=torch.uint8).pin_memory()
    capi.check(lib, lib.ffa_align_describe(ctypes.byref(plan), recs, host.data_ptr(), plan.table_bytes))
    outs, ptrs = _outputs(plan, len(es))
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        capi.check(lib, lib.ffa_align_launch_noalloc(ctypes.byref(plan), ctypes.byref(o), host.data_ptr(), None,
                                                     ctypes.byref(ptrs), stream))
    else:
        ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=DEV)
        capi.check(lib, lib.ffa_align_launch(ctypes.byref(plan), ctypes.byref(o), host.data_ptr(), None,
                                             ctypes.byref(ptrs), ws.data_ptr(), stream))
    torch.cuda.synchronize()
    return {f: outs[f].cpu().numpy() for f in FIELDS}


def _device(batch):
    return ([torch.from_numpy(e).to(DEV) for e in batch.emissions],
            [torch.from_numpy(y).to(DEV) for y in batch.targets])


@pytest.mark.gpu
@pytest.mark.parametrize("optimized", [True, False], ids=["optimized", "conventional"])
def test_noalloc_matches_launch_on_two_calls(optimized):
    lib = capi.load()
    big = _device(workloads.make("c5"))        # 1,024 records: ~11 MiB of scratch
    small = _device(workloads.c2(batch=12))    # then a smaller batch over the stale contents
    tiny = _device(workloads.c1())             # fused tail with repairs, counters left by the last call
    rng = np.random.default_rng(2100)
    y = rng.integers(1, 32, size=2100).astype(np.int64)
    flat = workloads._log_softmax((0.01 * rng.standard_normal((2300, 32))).astype(np.float32))
    y2 = rng.integers(1, 32, size=100).astype(np.int64)
    wide = ([torch.from_numpy(flat).to(DEV), torch.from_numpy(workloads.peaky(rng, y2, 600, 32)).to(DEV)],
            [torch.from_numpy(y).to(DEV), torch.from_numpy(y2).to(DEV)])  # S = 4201: 17 bands
    for name, (es, ys) in (("c5", big), ("wide", wide), ("c2x12", small), ("c1", tiny)):
        print(f"noalloc {name} optimized={optimized}", flush=True)
        want = _run(lib, es, ys, optimized, noalloc=False)
        got = _run(lib, es, ys, optimized, noalloc=True)
        assert_same(got, want, where=f"noalloc {name} ")
        assert not (got["labels"] == -7).all()
        if name == "wide" and optimized:
            assert want["routing_stats"][0, 0] == 2  # the early full fallback ran (banded)


def test_noalloc_rejects_batches_beyond_its_scratch():
    """Host-side size check before any device work: four 30,000-frame records of
    9,000 tokens need ~580 MiB of workspace. No GPU needed (fake addresses are
    never dereferenced)."""
    lib = capi.load()
    recs = (capi.Record * 4)()
    for i in range(4):
        recs[i] = capi.Record(0x1000 * (i + 1), 0x9000 * (i + 1), 30000, 32, 9000, 0)
    o = capi.default_options(lib, True)
    plan = capi.Plan()
    capi.check(lib, lib.ffa_align_plan_batch(recs, 4, ctypes.byref(o), ctypes.byref(plan)))
    host = (ctypes.c_uint8 * plan.table_bytes)()
    capi.check(lib, lib.ffa_align_describe(ctypes.byref(plan), recs, host, plan.table_bytes))
    outs = capi.Outputs(*([0x1000] * 10))
    assert lib.ffa_align_launch_noalloc(ctypes.byref(plan), ctypes.byref(o), host, None, ctypes.byref(outs),
                                        None) == -3
    assert "at most 33554432" in lib.ffa_last_error().decode()
