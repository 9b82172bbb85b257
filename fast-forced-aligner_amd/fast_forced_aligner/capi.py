"""ctypes binding of the C ABI in ``include/ffa.h``.

This is the binding a non-PyTorch host would write; tests use it to drive the
HIP library through its C entry points with caller-owned device buffers.
Device memory here comes from PyTorch tensors, but nothing in the ABI needs
torch: every argument is a plain pointer, size or stream handle.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

_HERE = Path(__file__).resolve().parent
HIP_LIBRARY = _HERE / "libffa_hip.so"

FFA_OK = 0
FFA_MAX_BATCH = 65535
FFA_MAX_VOCAB = 8192
FFA_MAX_STATES = 20479

EXPORTED = ("ffa_default_options", "ffa_align_plan_batch", "ffa_align_describe", "ffa_align_launch",
            "ffa_align_launch_noalloc", "ffa_emission_validity_launch", "ffa_token_spans_launch", "ffa_log_softmax_launch", "ffa_last_error",
            "ffa_profile_next_launch", "ffa_launch_floor")


class SpanRecord(ctypes.Structure):
    _fields_ = [("frame_offset", ctypes.c_int64), ("frames", ctypes.c_int64), ("span_offset", ctypes.c_int64),
                ("tokens", ctypes.c_int32), ("blank", ctypes.c_int32)]


class Record(ctypes.Structure):
    _fields_ = [("emissions", ctypes.c_void_p), ("targets", ctypes.c_void_p), ("frames", ctypes.c_int64),
                ("vocab", ctypes.c_int64), ("tokens", ctypes.c_int64), ("blank", ctypes.c_int64)]


class Options(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int64) for name in (
        "chunk_frames", "mode", "threads", "repair_rounds", "optimization_pass", "variant",
        "repair_budget_frames", "repair_threads", "trace_min_frames", "repair_min_frames",
        "frontier_min_frames")] + [(name, ctypes.c_int32) for name in (
            "compact_alphabet", "parallel_traceback", "overlap_fallback", "frontier_reuse", "check_inputs",
            "logits")]


class LogitsRecord(ctypes.Structure):
    _fields_ = [("logits", ctypes.c_void_p), ("log_probs", ctypes.c_void_p), ("frames", ctypes.c_int64),
                ("vocab", ctypes.c_int64)]


class Plan(ctypes.Structure):
    _fields_ = [("count", ctypes.c_int64), ("total_frames", ctypes.c_int64), ("table_bytes", ctypes.c_int64),
                ("table_uploaded", ctypes.c_int64), ("workspace_bytes", ctypes.c_int64),
                ("reuse_rows", ctypes.c_int64), ("internal", ctypes.c_int64 * 32)]


class Outputs(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in (
        "labels", "scores", "status", "objective", "stitched", "repair_passes", "repaired_frames",
        "shortcut_stats", "routing_stats", "reuse_stats")]


def load(path: Path | str = HIP_LIBRARY) -> ctypes.CDLL:
    """Load the HIP library (import torch first so both share one HIP runtime)."""
    lib = ctypes.CDLL(str(path), mode=ctypes.RTLD_GLOBAL)
    p = ctypes.c_void_p
    lib.ffa_default_options.restype = None
    lib.ffa_default_options.argtypes = [ctypes.c_int, ctypes.POINTER(Options)]
    lib.ffa_align_plan_batch.restype = ctypes.c_int
    lib.ffa_align_plan_batch.argtypes = [ctypes.POINTER(Record), ctypes.c_int64, ctypes.POINTER(Options),
                                         ctypes.POINTER(Plan)]
    lib.ffa_align_describe.restype = ctypes.c_int
    lib.ffa_align_describe.argtypes = [ctypes.POINTER(Plan), ctypes.POINTER(Record), p, ctypes.c_int64]
    lib.ffa_align_launch.restype = ctypes.c_int
    lib.ffa_align_launch.argtypes = [ctypes.POINTER(Plan), ctypes.POINTER(Options), p, p,
                                     ctypes.POINTER(Outputs), p, p]
    lib.ffa_align_launch_noalloc.restype = ctypes.c_int
    lib.ffa_align_launch_noalloc.argtypes = [ctypes.POINTER(Plan), ctypes.POINTER(Options), p, p,
                                             ctypes.POINTER(Outputs), p]
    lib.ffa_emission_validity_launch.restype = ctypes.c_int
    lib.ffa_emission_validity_launch.argtypes = [p, ctypes.c_int64, p, p]
    lib.ffa_last_error.restype = ctypes.c_char_p
    lib.ffa_last_error.argtypes = []
    lib.ffa_profile_next_launch.restype = ctypes.c_int
    lib.ffa_profile_next_launch.argtypes = [p, p]
    lib.ffa_launch_floor.restype = ctypes.c_int
    lib.ffa_launch_floor.argtypes = [ctypes.c_int32, ctypes.c_int32, p]
    lib.ffa_token_spans_launch.restype = ctypes.c_int
    lib.ffa_token_spans_launch.argtypes = [p, ctypes.c_int64, p, p, p, p]
    lib.ffa_log_softmax_launch.restype = ctypes.c_int
    lib.ffa_log_softmax_launch.argtypes = [p, ctypes.c_int64, ctypes.c_int64, p]
    return lib


def default_options(lib: ctypes.CDLL, optimized: bool) -> Options:
    o = Options()
    lib.ffa_default_options(1 if optimized else 0, ctypes.byref(o))
    return o


def check(lib: ctypes.CDLL, rc: int) -> None:
    if rc != FFA_OK:
        raise RuntimeError(f"ffa call failed ({rc}): {lib.ffa_last_error().decode()}")
