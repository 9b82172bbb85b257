"""CPU checks of the drop-in boundary: the C ABI library loads and exports what
include/ffa.h declares, host-side planning validates like the reference's
TORCH_CHECKs, the torch operators register the reference's schemas, and the
Python API's host-side contracts (loader errors, metadata errors, status
messages) behave like the reference's. No GPU compute runs here."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

import fast_forced_aligner as ffa
from fast_forced_aligner import alignment, capi

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "ffa.h"

REFERENCE_SCHEMAS = {
    "emission_validity": "fast_forced_aligner_cuda::emission_validity(Tensor[] emissions) -> Tensor",
    "align": ("fast_forced_aligner_cuda::align(Tensor[] emissions, Tensor[] targets, int[] blanks, "
              "int chunk_frames, int mode, int threads, int repair_rounds, int optimization_pass, "
              "int variant, int repair_budget_frames, int repair_threads, bool compact_alphabet, "
              "bool parallel_traceback, bool overlap_fallback, int trace_min_frames, int repair_min_frames, "
              "bool frontier_reuse, int frontier_min_frames, Tensor? emission_validity=None, "
              "bool check_inputs=True) -> (Tensor[], int[])"),
}


@pytest.fixture(scope="module")
def lib():
    if not capi.HIP_LIBRARY.exists():
        pytest.fail("libffa_hip.so is not built: run __graft_entry__.build()")
    return capi.load()


def test_header_symbols_are_exported(lib):
    declared = set(re.findall(r"^(?:int|void|const char\*)\s+(ffa_\w+)\(", HEADER.read_text(), re.M))
    assert declared == set(capi.EXPORTED)
    for name in declared:
        assert hasattr(lib, name), name


def test_default_options_are_the_public_knob_vector(lib):
    o = capi.default_options(lib, True)
    assert (o.chunk_frames, o.mode, o.threads, o.repair_rounds, o.optimization_pass, o.variant,
            o.repair_budget_frames, o.repair_threads, o.compact_alphabet, o.parallel_traceback,
            o.overlap_fallback, o.trace_min_frames, o.repair_min_frames, o.frontier_reuse,
            o.frontier_min_frames, o.check_inputs) == (128, 2, 512, 2, 2, 2, 512, 0, 0, 1, 1, 2048, 2048, 1,
                                                        2048, 1)
    c = capi.default_options(lib, False)
    assert (c.mode, c.repair_budget_frames, c.overlap_fallback, c.frontier_reuse) == (0, 0, 0, 0)


def _records(shapes):
    """Host-only records with fake (never dereferenced) device addresses."""
    recs = (capi.Record * len(shapes))()
    for i, (T, V, U, blank) in enumerate(shapes):
        recs[i] = capi.Record(0x1000 * (i + 1), 0x9000 * (i + 1) if U else 0, T, V, U, blank)
    return recs


def _plan(lib, shapes, optimized=True, **changes):
    o = capi.default_options(lib, optimized)
    for k, v in changes.items():
        setattr(o, k, v)
    plan = capi.Plan()
    recs = _records(shapes)
    rc = lib.ffa_align_plan_batch(recs, len(shapes), ctypes.byref(o), ctypes.byref(plan))
    return rc, plan, recs


def test_plan_sizes_and_gating(lib):
    rc, plan, recs = _plan(lib, [(500, 32, 4, 0), (320, 32, 3, 0)])
    assert rc == 0
    assert plan.count == 2 and plan.total_frames == 820
    # 64-byte record descriptors, passed as a kernel argument
    assert plan.table_bytes == 2 * 64 and plan.table_uploaded == 0
    assert plan.reuse_rows == 0
    # more than 64 records: descriptors plus one 16-byte entry per chunk, uploaded
    rc, big, _ = _plan(lib, [(500, 32, 4, 0)] * 65)
    assert rc == 0 and big.table_uploaded == 1 and big.table_bytes == 65 * 64 + 65 * 4 * 16
    assert big.workspace_bytes >= big.table_bytes
    rc, plan, _ = _plan(lib, [(2048, 32, 4, 0), (320, 32, 3, 0)])
    assert rc == 0 and plan.reuse_rows == 2  # frontier reuse: batch max T >= 2048 (alignment.cu:1002)
    rc, plan, _ = _plan(lib, [(2048, 32, 4, 0)], optimized=False)
    assert rc == 0 and plan.reuse_rows == 0  # never in conventional mode (alignment.cu:935)
    rc, plan, recs = _plan(lib, [(50, 8, 2, 0)])
    buf = (ctypes.c_uint8 * (plan.table_bytes - 1))()
    assert lib.ffa_align_describe(ctypes.byref(plan), recs, buf, plan.table_bytes - 1) == -3
    buf = (ctypes.c_uint8 * plan.table_bytes)()
    assert lib.ffa_align_describe(ctypes.byref(plan), recs, buf, plan.table_bytes) == 0
    words = (ctypes.c_int32 * 16).from_buffer(buf)
    assert (words[4], words[5], words[6], words[7], words[8], words[9]) == (50, 0, 8, 2, 0, 0)  # T, chunk, V, U, frame offset


@pytest.mark.parametrize("shape, changes, message", [
    ([(0, 8, 1, 0)], {}, "shape or blank"),
    ([(10, 0, 1, 0)], {}, "shape or blank"),
    ([(10, 8193, 1, 0)], {}, "shape or blank"),
    ([(10, 8, 1, 8)], {}, "shape or blank"),
    ([(10, 8, 10240, 0)], {}, "shape or blank"),
    ([(10, 8, 1, 0)], {"threads": 100}, "invalid block size"),
    ([(10, 8, 1, 0)], {"repair_rounds": 3}, "invalid repair rounds"),
    ([(10, 8, 1, 0)], {"variant": 3}, "variant must be"),
    ([(10, 8, 1, 0)], {"optimization_pass": 4}, "optimization pass"),
    ([(10, 8, 1, 0)], {"repair_threads": 64, "overlap_fallback": 0}, "repair threads"),
    ([(10, 8, 1, 0)], {"repair_threads": 128}, "overlap preserves fallback geometry"),
    ([(10, 8, 1, 0)], {"trace_min_frames": 0}, "trace_min_frames"),
    ([(10, 8, 1, 0)], {"chunk_frames": 0}, "chunk size or mode"),
    ([(10, 8, 1, 0)], {"chunk_frames": 513}, "chunk size or mode"),
    ([(10, 8, 1, 0)], {"mode": 3}, "chunk size or mode"),
])
def test_plan_rejects_like_the_reference(lib, shape, changes, message):
    rc, _, _ = _plan(lib, shape, **changes)
    assert rc == -1
    assert message in lib.ffa_last_error().decode()


@pytest.mark.parametrize("address", [0x9004, 1 << 48])
def test_plan_rejects_target_addresses_the_chunk_entries_cannot_hold(lib, address):
    """Chunk entries carry the targets' address / 8 in 45 bits: the plan
    rejects a pointer that is not 8-byte aligned or not below 2^48."""
    o = capi.default_options(lib, True)
    plan = capi.Plan()
    recs = (capi.Record * 1)(capi.Record(0x1000, address, 50, 8, 2, 0))
    assert lib.ffa_align_plan_batch(recs, 1, ctypes.byref(o), ctypes.byref(plan)) == -1
    assert "48-bit" in lib.ffa_last_error().decode()


def test_chunk_entries_hold_targets_address_and_counts(lib):
    """Uploaded tables (more than 64 records) carry one 16-byte entry per chunk
    after the record descriptors; tables passed as kernel arguments have none."""
    rc, small, _ = _plan(lib, [(300, 32, 5, 0)])
    assert rc == 0 and small.table_uploaded == 0 and small.table_bytes == 64
    rc, plan, recs = _plan(lib, [(300, 32, 5, 0)] + [(10, 8, 1, 0)] * 64)
    assert rc == 0 and plan.table_uploaded == 1
    buf = (ctypes.c_uint8 * plan.table_bytes)()
    assert lib.ffa_align_describe(ctypes.byref(plan), recs, buf, plan.table_bytes) == 0
    entries = (ctypes.c_uint64 * 6).from_buffer(buf, 65 * 64)  # after the 65 record descriptors
    for c in range(3):  # 300 frames: chunks of 128, 128, 44
        lo, hi = entries[2 * c], entries[2 * c + 1]
        assert (lo & ((1 << 45) - 1)) << 3 == recs[0].targets
        assert (lo >> 45) & 0x3FFF == 5  # U
        assert (lo >> 59) & 1 == 1 and ((lo >> 60) & 7) + 1 == 8  # fast path, V/4
        assert hi & 0xFFFF == 0 and ((hi >> 16) & 0x1FF) + 1 == (128, 128, 44)[c] and hi >> 25 == c


def _descriptors(lib, plan, recs):
    buf = (ctypes.c_uint8 * plan.table_bytes)()
    assert lib.ffa_align_describe(ctypes.byref(plan), recs, buf, plan.table_bytes) == 0
    q = (ctypes.c_int64 * (8 * plan.count)).from_buffer(buf)
    w = (ctypes.c_int32 * (16 * plan.count)).from_buffer(buf)
    # 64-byte records: frontier offset at byte 48, the counted-reuse flag at byte 60
    return [(q[8 * i + 6], w[16 * i + 15]) for i in range(plan.count)]


def test_frontier_storage_and_reuse_counting(lib):
    """Optimized mode with chunks of at least 32 frames keeps S floats per
    chunk for every record (repairs and fallbacks resume from them); only the
    records the reference runs with frontier reuse (batch max T >= 2048 and the
    record's T >= frontier_min_frames, alignment.cu:374, :1002) carry the flag
    that makes reuse_stats count. Conventional mode and short chunks keep none
    beyond the reference's."""
    shapes = [(2048, 32, 4, 0), (300, 32, 5, 0), (500, 32, 2, 0)]
    rc, plan, recs = _plan(lib, shapes)
    assert rc == 0 and plan.reuse_rows == 3
    # 2048 frames: 16 chunks x 9 states; 300: 3 x 11; 500: 4 x 5
    assert _descriptors(lib, plan, recs) == [(0, 1), (144, 0), (177, 0)]
    rc, plan, recs = _plan(lib, shapes[1:])  # no record reaches 2048 frames: nothing counted
    assert rc == 0 and plan.reuse_rows == 0
    assert _descriptors(lib, plan, recs) == [(0, 0), (33, 0)]
    rc, plan, recs = _plan(lib, shapes, frontier_reuse=0)  # reference reuse off: storage stays
    assert rc == 0 and plan.reuse_rows == 0
    assert _descriptors(lib, plan, recs) == [(0, 0), (144, 0), (177, 0)]
    rc, plan, recs = _plan(lib, shapes, chunk_frames=16)  # short chunks: the reference's records only
    assert rc == 0 and plan.reuse_rows == 3
    assert _descriptors(lib, plan, recs) == [(0, 1), (-1, 0), (-1, 0)]
    rc, plan, recs = _plan(lib, shapes, optimized=False)
    assert rc == 0 and plan.reuse_rows == 0
    assert _descriptors(lib, plan, recs) == [(-1, 0), (-1, 0), (-1, 0)]


def test_operator_schemas_match_the_reference():
    torch.ops.load_library(str(alignment.TORCH_LIBRARY))
    for name, schema in REFERENCE_SCHEMAS.items():
        assert str(getattr(torch.ops.fast_forced_aligner_cuda, name).default._schema) == schema


@pytest.fixture
def fresh_loader():
    ffa.load_extension.cache_clear()
    yield
    ffa.load_extension.cache_clear()


def test_loader_requires_rocm_torch(monkeypatch, fresh_loader):
    monkeypatch.setattr(torch.version, "hip", None)
    with pytest.raises(RuntimeError, match="ROCm-enabled PyTorch"):
        ffa.load_extension()


def test_loader_requires_gpu(monkeypatch, fresh_loader):
    monkeypatch.setattr(torch.version, "hip", "7.0")
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    with pytest.raises(RuntimeError, match="accessible AMD GPU"):
        ffa.load_extension()


def test_loader_reports_missing_toolkit(monkeypatch, tmp_path, fresh_loader):
    monkeypatch.setattr(torch.version, "hip", "7.0")
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(alignment, "HIP_LIBRARY", tmp_path / "missing.so")
    monkeypatch.setattr(alignment, "_rocm_home", lambda: None)
    with pytest.raises(RuntimeError, match="including hipcc"):
        ffa.load_extension()


def test_metadata_errors_raise_before_native_code():
    e = torch.zeros(12, 6)
    t = torch.tensor([1])
    with pytest.raises(ValueError, match="mode must be"):
        ffa.align([e], [t], mode="unknown")
    with pytest.raises(TypeError, match="check_inputs must be bool"):
        ffa.align([e], [t], check_inputs=1)
    with pytest.raises(ValueError, match="1..65535"):
        ffa.align([], [])
    with pytest.raises(ValueError, match="contiguous CUDA"):
        ffa.align([e], [t])
    with pytest.raises(ValueError, match="one blank ID per record"):
        ffa.align([e], [t], blank_id=[0, 1])
    with pytest.raises(ValueError):
        ffa.emission_validity([])
    with pytest.raises(ValueError, match="contiguous CUDA"):
        ffa.emission_validity([e])


def _batch(status):
    z = torch.zeros(len(status))
    return ffa.AlignmentBatch((1,) * len(status), z, z, torch.tensor(status, dtype=torch.int32), z, z, z, z,
                              z, z, z)


def test_raise_for_status_messages():
    _batch([0, 0]).raise_for_status()
    with pytest.raises(ValueError) as error:
        _batch([3, 4, 2, 3, 1]).raise_for_status()
    text = str(error.value)
    parts = ["invalid emissions at batch indices [2]", "no finite complete CTC path for batch indices [4]",
             "invalid target IDs at batch indices [0, 3]", "insufficient CTC frames at batch indices [1]"]
    assert text == "; ".join(parts)
    with pytest.raises(RuntimeError, match="unknown alignment status"):
        _batch([0, 99]).raise_for_status()


def test_logits_option_plans_statistics(lib):
    shapes = [(500, 32, 4, 0), (320, 32, 3, 0)]
    for optimized in (True, False):
        rc, plain, _ = _plan(lib, shapes, optimized=optimized)
        assert rc == 0
        rc, fused, _ = _plan(lib, shapes, optimized=optimized, logits=1)
        assert rc == 0
        # 8 bytes of row statistics per frame, 256-byte aligned; same table
        assert fused.workspace_bytes == plain.workspace_bytes + (8 * 820 + 255) // 256 * 256
        assert fused.table_bytes == plain.table_bytes
    rc, _, _ = _plan(lib, shapes, logits=2)
    assert rc == -1 and "logits must be 0 or 1" in lib.ffa_last_error().decode()


def test_banded_dp_plans_control_words_and_edge_arrays(lib):
    """Transcripts of more than 1,024 states run the banded DP (bands of 256
    states) in conventional mode and, under the split tail, for optimized
    mode's fallbacks; without the split tail, transcripts of more than 4,096
    states; log-probability input only. The plan adds control
    words (64 + B ints and two floats per record, 256-byte aligned) and 8 bytes
    per frame and band boundary of the widest record to the workspace."""
    wide = [(3000, 32, 2200, 0), (500, 32, 100, 0)]   # S = 4401 (18 bands) and 201 (1 band)
    band = -(-(-(-(4 * (64 + 2) + 8 * 2) // 256) * 256 + 8 * 3500 * 17) // 256) * 256
    stats = -(-8 * 3500 // 256) * 256
    rc, conv, _ = _plan(lib, wide, optimized=False)
    rc2, conv_lg, _ = _plan(lib, wide, optimized=False, logits=1)   # logits keep the one-workgroup DP
    assert rc == 0 and rc2 == 0
    assert conv.workspace_bytes - conv_lg.workspace_bytes == band - stats
    rc, opt, _ = _plan(lib, wide)                     # T_max >= 2048: split tail, banded early fallbacks
    rc2, opt_lg, _ = _plan(lib, wide, logits=1)       # logits: one-workgroup DPs
    assert rc == 0 and rc2 == 0
    assert opt.workspace_bytes - opt_lg.workspace_bytes == band - stats
    # no repair rounds (no split tail): K = 32 transcripts still hand their fallback to the
    # banded DP, through one 112-byte tail state per record
    rc, opt_r0, _ = _plan(lib, wide, repair_rounds=0)
    rc2, opt_r0_lg, _ = _plan(lib, wide, repair_rounds=0, logits=1)
    assert rc == 0 and rc2 == 0
    assert opt_r0.workspace_bytes - opt_r0_lg.workspace_bytes == 256 + band - stats
    k16 = [(3000, 32, 1500, 0), (500, 32, 100, 0)]   # S = 3001: K = 16, no banded DP without the split tail
    rc, a, _ = _plan(lib, k16, repair_rounds=0)
    rc2, b, _ = _plan(lib, k16, repair_rounds=0, logits=1)
    assert rc == 0 and rc2 == 0 and b.workspace_bytes - a.workspace_bytes == stats
    narrow = [(3000, 32, 500, 0), (500, 32, 100, 0)]  # S = 1001: K = 4, one workgroup per record
    rc, conv, _ = _plan(lib, narrow, optimized=False)
    rc2, conv_lg, _ = _plan(lib, narrow, optimized=False, logits=1)
    assert rc == 0 and rc2 == 0 and conv_lg.workspace_bytes - conv.workspace_bytes == stats


def test_logits_entry_points_check_arguments_on_the_host(lib):
    assert lib.ffa_log_softmax_launch(None, 1, 10, None) == -1
    assert "null record" in lib.ffa_last_error().decode()
    assert lib.ffa_log_softmax_launch(None, 0, 10, None) == -1
    assert lib.ffa_log_softmax_launch(None, 1, 0, None) == -1
    e = torch.zeros(12, 6)
    t = torch.tensor([1])
    with pytest.raises(ValueError, match="contiguous CUDA"):
        ffa.align_logits([e], [t])
    with pytest.raises(ValueError, match="mode must be"):
        ffa.align_logits([e], [t], mode="fast")
    with pytest.raises(ValueError, match="1..65535"):
        ffa.log_softmax([])
    with pytest.raises(ValueError, match="contiguous CUDA"):
        ffa.log_softmax([e])


@pytest.mark.parametrize("workgroups, threads", [(0, 64), (-1, 64), (8, 0), (8, 1025)])
def test_launch_floor_checks_its_shape_on_the_host(lib, workgroups, threads):
    assert lib.ffa_launch_floor(workgroups, threads, None) == -1
    assert "threads 1..1024" in lib.ffa_last_error().decode()
