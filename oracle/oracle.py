"""ctypes wrapper for the CPU oracle (``oracle/ffa_oracle.c``).

Test infrastructure only: ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg import this module as the checker. The
product path (``fast_forced_aligner``) never imports it.

``align`` mirrors the reference's ``align`` (alignment.py:346-502) on numpy
arrays, with the same fixed knob vector (alignment.py:496-501), and returns the
same ten fields as ``AlignmentBatch`` plus ``lengths``.
"""
from __future__ import annotations

import ctypes
import subprocess
from collections.abc import Sequence
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libffa_oracle.so"
REF_DIR = HERE / "_ref"


class Options(ctypes.Structure):
    _fields_ = [
        ("chunk_frames", ctypes.c_int64),
        ("mode", ctypes.c_int32),
        ("repair_rounds", ctypes.c_int32),
        ("repair_budget_frames", ctypes.c_int64),
        ("overlap_fallback", ctypes.c_int32),
        ("repair_min_frames", ctypes.c_int64),
        ("frontier_reuse", ctypes.c_int32),
        ("frontier_min_frames", ctypes.c_int64),
        ("check_inputs", ctypes.c_int32),
    ]


def build() -> None:
    """Compile the oracle (and oracle/_ref when the reference tree is mounted)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


_lib = None
_mutants = None
MUTANTS_LIB = HERE / "libffa_oracle_mutants.so"


def _declare(handle: ctypes.CDLL) -> ctypes.CDLL:
    p = ctypes.c_void_p
    handle.orc_align.restype = ctypes.c_int
    handle.orc_align.argtypes = [ctypes.c_int64, p, p, p, p, p, p, p, ctypes.POINTER(Options),
                                 ctypes.c_int32] + [p] * 10 + [p]
    handle.orc_record_status.restype = ctypes.c_int32
    handle.orc_record_status.argtypes = [p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                         ctypes.c_int64, ctypes.c_int32, ctypes.c_int32]
    handle.orc_emission_valid.restype = ctypes.c_int32
    handle.orc_emission_valid.argtypes = [p, ctypes.c_int64]
    return handle


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = _declare(ctypes.CDLL(str(LIB)))
    return _lib


def mutants() -> ctypes.CDLL:
    """The oracle built with planted-mistake hooks (tests only):
    ``orc_set_mutant(n)`` selects mistake n (0 = none); pass the handle to
    ``align(..., library=...)``."""
    global _mutants
    if _mutants is None:
        if not MUTANTS_LIB.exists():
            build()
        _mutants = _declare(ctypes.CDLL(str(MUTANTS_LIB)))
        _mutants.orc_set_mutant.argtypes = [ctypes.c_int]
        _mutants.orc_set_mutant.restype = None
    return _mutants


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def knobs(mode: str) -> Options:
    """The knob vector the public API always passes (alignment.py:496-501)."""
    optimized = mode == "optimized"
    return Options(chunk_frames=128, mode=2 if optimized else 0, repair_rounds=2,
                   repair_budget_frames=512 if optimized else 0, overlap_fallback=int(optimized),
                   repair_min_frames=2048, frontier_reuse=int(optimized), frontier_min_frames=2048,
                   check_inputs=1)


def align(emissions: Sequence[np.ndarray], targets: Sequence[np.ndarray], blank_id=0,
          mode: str = "optimized", check_inputs: bool = True, emission_validity=None,
          threads: int = 1, options: Options | None = None, library: ctypes.CDLL | None = None) -> dict:
    """Run the oracle on host arrays; returns a dict of numpy outputs."""
    count = len(emissions)
    blanks = [blank_id] * count if isinstance(blank_id, (int, np.integer)) else list(blank_id)
    es = [np.ascontiguousarray(e, dtype=np.float32) for e in emissions]
    ys = [np.ascontiguousarray(t, dtype=np.int64).reshape(-1) for t in targets]
    T = np.array([e.shape[0] for e in es], dtype=np.int64)
    V = np.array([e.shape[1] for e in es], dtype=np.int64)
    U = np.array([y.shape[0] for y in ys], dtype=np.int64)
    B = np.array(blanks, dtype=np.int64)
    # a zero-length target still needs a valid address
    ys = [y if y.size else np.zeros(1, dtype=np.int64) for y in ys]
    eptr = np.array([_ptr(e) for e in es], dtype=np.uint64)
    yptr = np.array([_ptr(y) for y in ys], dtype=np.uint64)
    o = options if options is not None else knobs(mode)
    o.check_inputs = int(check_inputs)
    N = int(T.sum())
    out = {
        "labels": np.empty(N, dtype=np.int64), "scores": np.empty(N, dtype=np.float32),
        "status": np.empty(count, dtype=np.int32), "objective": np.empty(count, dtype=np.float32),
        "stitched": np.empty(count, dtype=np.int32), "repair_passes": np.empty(count, dtype=np.int32),
        "repaired_frames": np.empty(count, dtype=np.int64),
        "shortcut_stats": np.empty((count, 3), dtype=np.int64),
        "routing_stats": np.empty((count, 3), dtype=np.int32),
        "reuse_stats": np.zeros((count, 4), dtype=np.int64),
    }
    validity = None
    if emission_validity is not None:
        validity = np.ascontiguousarray(emission_validity, dtype=np.uint8)
    rows = ctypes.c_int64(0)
    rc = (library or lib()).orc_align(count, _ptr(eptr), _ptr(T), _ptr(V), _ptr(yptr), _ptr(U), _ptr(B),
                         None if validity is None else _ptr(validity), ctypes.byref(o), threads,
                         *[_ptr(out[k]) for k in ("labels", "scores", "status", "objective", "stitched",
                                                  "repair_passes", "repaired_frames", "shortcut_stats",
                                                  "routing_stats", "reuse_stats")],
                         ctypes.addressof(rows))
    if rc != 0:
        raise MemoryError("oracle allocation failed")
    out["reuse_stats"] = out["reuse_stats"][: rows.value]
    out["lengths"] = tuple(int(x) for x in T)
    return out


def record_status(targets: np.ndarray, frames: int, vocab: int, blank: int,
                  check_inputs: bool = True, masked: bool = False) -> int:
    y = np.ascontiguousarray(targets, dtype=np.int64).reshape(-1)
    holder = y if y.size else np.zeros(1, dtype=np.int64)
    return int(lib().orc_record_status(_ptr(holder), y.size, frames, vocab, blank,
                                       int(check_inputs), int(masked)))


def emission_valid(emission: np.ndarray) -> bool:
    e = np.ascontiguousarray(emission, dtype=np.float32)
    return bool(lib().orc_emission_valid(_ptr(e), e.size))


def token_spans(labels: np.ndarray, lengths: Sequence[int], tokens: Sequence[int], status: np.ndarray,
                blank_id=0) -> np.ndarray:
    """Token spans of aligned paths, restating the reference README's
    "Converting frame labels to timestamps" (README.md:509-517; no code in the
    reference): split each path into equal-label runs, discard blank runs, keep
    each remaining run's [start, end) frames. Rows per record = its target
    length: records with nonzero status are all -1; missing runs are -1 and
    extra runs are dropped (only possible for a transcript holding the blank id)."""
    blanks = [blank_id] * len(lengths) if isinstance(blank_id, int) else list(blank_id)
    out = np.full((int(sum(tokens)), 2), -1, dtype=np.int64)
    frame = span = 0
    for T, U, st, b in zip(lengths, tokens, status, blanks):
        p = np.asarray(labels[frame:frame + T])
        if st == 0 and U > 0:
            edges = np.flatnonzero(np.r_[True, p[1:] != p[:-1]])
            ends = np.r_[edges[1:], T]
            keep = p[edges] != b
            runs = np.stack([edges[keep], ends[keep]], axis=1)[:U]
            out[span:span + len(runs)] = runs
        frame += T
        span += U
    return out


def reference_comparator():
    """The reference's own CPU comparator compiled into oracle/_ref, or None.

    It exists only where the reference tree was mounted at build time (this
    container); tests that use it skip elsewhere.
    """
    import importlib.util
    for path in sorted(REF_DIR.glob("ffa_corrected_ctc_cpp*.so")):
        spec = importlib.util.spec_from_file_location("ffa_corrected_ctc_cpp", path)
        module = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(module)
        return module
    return None
