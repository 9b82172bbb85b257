"""Public API of the MI355X alignment path: a drop-in for the reference package.

Same names, arguments, result type, statuses and error messages as the
reference's ``src/fast_forced_aligner/alignment.py`` (cited as ``py:<line>``);
the native operators ``fast_forced_aligner_cuda.align`` / ``.emission_validity``
come from this package's HIP build instead of a CUDA JIT build.
"""
from __future__ import annotations

import ctypes
import os
from collections.abc import Sequence
from dataclasses import dataclass, fields
from functools import lru_cache
from pathlib import Path
from typing import Literal

import torch
from torch import Tensor

Mode = Literal["optimized", "conventional"]

_HERE = Path(__file__).resolve().parent
HIP_LIBRARY = _HERE / "libffa_hip.so"
TORCH_LIBRARY = _HERE / "_ffa_torch.so"


def _rocm_home() -> Path | None:
    from torch.utils import cpp_extension

    home = getattr(cpp_extension, "ROCM_HOME", None) or os.environ.get("ROCM_PATH")
    return Path(home) if home else None


_native = None  # the _ffa_torch module once load_extension() succeeded


@lru_cache(maxsize=1)
def load_extension() -> None:
    """Load the bundled HIP extension (build it first if it is absent).

    Mirrors the reference loader (py:15-63) for ROCm: the libraries are built
    in place by ``fast-forced-aligner_amd/build.py`` for gfx950; the first call
    loads them and registers the ``fast_forced_aligner_cuda`` operators.
    Successful calls are memoized for the process.

    Raises:
        RuntimeError: PyTorch lacks ROCm support, no AMD GPU is accessible, the
            libraries are missing and no ROCm toolkit (hipcc) can build them,
            or loading fails.
    """
    if torch.version.hip is None:
        raise RuntimeError("fast_forced_aligner requires a ROCm-enabled PyTorch installation")
    if not torch.cuda.is_available():
        raise RuntimeError("fast_forced_aligner requires an accessible AMD GPU and compatible driver")
    if not (HIP_LIBRARY.is_file() and TORCH_LIBRARY.is_file()):
        home = _rocm_home()
        if home is None or not (home / "bin" / "hipcc").is_file():
            raise RuntimeError(
                "fast_forced_aligner ships HIP source and its gfx950 libraries are not built. "
                "Install the ROCm development toolkit (including hipcc) or run "
                "fast-forced-aligner_amd/build.py; set ROCM_PATH if ROCm is outside /opt/rocm."
            )
        import importlib.util

        spec = importlib.util.spec_from_file_location("_ffa_build", _HERE.parent / "build.py")
        module = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(module)
        module.build()
    # the HIP library first, so the operator library resolves against it;
    # importing _ffa_torch registers the fast_forced_aligner_cuda operators
    ctypes.CDLL(str(HIP_LIBRARY), mode=ctypes.RTLD_GLOBAL)
    global _native
    from . import _ffa_torch

    _native = _ffa_torch


@dataclass(frozen=True)
class AlignmentBatch:
    """Packed frame alignments and per-record diagnostics returned by ``align``.

    Field meaning follows the reference (py:66-148): ``labels`` int64 ``(N,)``,
    ``scores`` float32 ``(N,)`` (the selected input emission per frame; ``-1`` /
    ``-inf`` for failed records), ``status`` int32 ``(B,)`` (0 ok, 1 no finite
    path, 2 rejected by the emission mask, 3 invalid target ids, 4 insufficient
    frames), ``objective`` float32 ``(B,)``, ``stitched``, ``repair_passes``,
    ``repaired_frames``, ``shortcut_stats`` ``(B, 3)``, ``routing_stats``
    ``(B, 3)`` and ``reuse_stats`` ``(B, 4)`` or ``(0, 4)``. All tensors stay on
    the input device; reading them on the host synchronizes.
    """

    lengths: tuple[int, ...]
    labels: Tensor
    scores: Tensor
    status: Tensor
    objective: Tensor
    stitched: Tensor
    repair_passes: Tensor
    repaired_frames: Tensor
    shortcut_stats: Tensor
    routing_stats: Tensor
    reuse_stats: Tensor

    @property
    def paths(self) -> tuple[Tensor, ...]:
        """Per-record views into ``labels`` (no copy, no synchronization)."""
        return self.labels.split(self.lengths)

    def raise_for_status(self) -> None:
        """Raise if any record failed (py:163-230); reading status synchronizes.

        Raises:
            ValueError: some record has status 1, 2, 3 or 4; the message lists
                the zero-based indices per category.
            RuntimeError: a status outside 0..4.
        """
        statuses = self.status.cpu().tolist()
        if not any(statuses):
            return
        unknown = [i for i, value in enumerate(statuses) if value not in (0, 1, 2, 3, 4)]
        if unknown:
            raise RuntimeError(f"unknown alignment status at batch indices {unknown}")
        groups = {code: [i for i, value in enumerate(statuses) if value == code] for code in (1, 2, 3, 4)}
        messages = []
        for code, text in ((2, "invalid emissions at batch indices"),
                           (1, "no finite complete CTC path for batch indices"),
                           (3, "invalid target IDs at batch indices"),
                           (4, "insufficient CTC frames at batch indices")):
            if groups[code]:
                messages.append(f"{text} {groups[code]}")
        raise ValueError("; ".join(messages))


_BATCH_FIELDS = tuple(f.name for f in fields(AlignmentBatch))


def _batch(lengths: tuple[int, ...], tensors: Sequence[Tensor]) -> AlignmentBatch:
    """``AlignmentBatch(lengths, *tensors)`` with one dict update instead of the
    frozen dataclass's eleven ``object.__setattr__`` calls (the same instance;
    the per-call host cost of ``align`` is a few microseconds)."""
    out = object.__new__(AlignmentBatch)
    out.__dict__.update(zip(_BATCH_FIELDS, (lengths, *tensors)))
    return out


def _metadata(emissions: Sequence[Tensor], targets: Sequence[Tensor],
              blank_id: int | Sequence[int]) -> list[int]:
    """Host-only metadata checks (py:233-252). Returns one blank per record.

    The target-length limit follows the native state limit of this build
    (2U+1 <= 20479, i.e. U <= 10239) instead of the reference's 2047.
    """
    count = len(emissions)
    if not 0 < count <= 65535 or len(targets) != count:
        raise ValueError("provide 1..65535 matching emissions and targets")
    blanks = [blank_id] * count if type(blank_id) is int else list(blank_id)
    if len(blanks) != count:
        raise ValueError("provide one blank ID per record")
    device = emissions[0].device
    for e, t, blank in zip(emissions, targets, blanks, strict=True):
        if (e.device.type != "cuda" or e.device != device or t.device != device
                or e.dtype != torch.float32 or t.dtype != torch.int64
                or e.ndim != 2 or t.ndim != 1
                or not e.is_contiguous() or not t.is_contiguous()):
            raise ValueError("inputs must be contiguous CUDA float32 [T,V] and int64 [U] on one device")
        if (not 0 < e.shape[0] <= 2**31 - 1 or not 0 < e.shape[1] <= 8192
                or t.numel() > MAX_TOKENS or type(blank) is not int or not 0 <= blank < e.shape[1]):
            raise ValueError("unsupported frame count, vocabulary, target length, or blank ID")
    return blanks


MAX_TOKENS = 10239


@torch.inference_mode()
def validate_inputs(emissions: Sequence[Tensor], targets: Sequence[Tensor], *,
                    blank_id: int | Sequence[int] = 0) -> None:
    """Check metadata, target ids and CTC frame feasibility; synchronizes (py:255-309).

    Raises:
        ValueError: metadata violations, or the batch indices whose targets are
            invalid or need more frames than available.
    """
    blanks = _metadata(emissions, targets, blank_id)
    valid = []
    for e, t, blank in zip(emissions, targets, blanks, strict=True):
        tokens_ok = ((t >= 0) & (t < e.shape[1]) & (t != blank)).all()
        frames_ok = t.numel() + (t[1:] == t[:-1]).sum() <= e.shape[0]
        valid.append(tokens_ok & frames_ok)
    failures = [i for i, ok in enumerate(torch.stack(valid).cpu().tolist()) if not ok]
    if failures:
        raise ValueError(f"invalid target IDs or insufficient CTC frames at batch indices {failures}")


@torch.inference_mode()
def emission_validity(emissions: Sequence[Tensor]) -> Tensor:
    """Device bool mask, false for any record holding NaN or +inf (py:312-343).

    No value is read by the host; the scan runs on the current stream.
    """
    if not 0 < len(emissions) <= 65535:
        raise ValueError("provide 1..65535 emission tensors")
    if not (isinstance(emissions[0], Tensor) and emissions[0].is_cuda):
        raise ValueError("emissions must be contiguous CUDA float32 [T,V] with supported dimensions on one device")
    load_extension()
    # the native entry checks every record with the same message (O(B) in C++)
    return _native.emission_validity(emissions)


def align(emissions: Sequence[Tensor], targets: Sequence[Tensor], *,
          blank_id: int | Sequence[int] = 0, mode: Mode = "optimized",
          check_inputs: bool = True, emission_validity: Tensor | None = None) -> AlignmentBatch:
    """Align known CTC targets to resident emissions on the GPU (py:346-502).

    Args:
        emissions: ``B`` contiguous float32 ``(T_i, V_i)`` device tensors.
        targets: ``B`` contiguous int64 ``(U_i,)`` device tensors, no blanks.
        blank_id: one int, or one int per record.
        mode: ``"optimized"`` (128-frame chunks, greedy shortcuts, two repair
            rounds, full-DP fallback) or ``"conventional"`` (full fp32 DP).
        check_inputs: validate target ids and frame feasibility on the GPU.
        emission_validity: optional device bool ``(B,)`` mask; False rejects
            a record with status 2 unless its targets are invalid (3, 4).

    Returns:
        AlignmentBatch; failures are reported in ``status``, never raised here.
        Its tensors are inference tensors, as under the reference's
        ``torch.inference_mode``.

    Raises:
        ValueError: invalid mode, metadata, blank ids or mask metadata.
        TypeError: ``check_inputs`` is not a bool.
        RuntimeError: the HIP extension is unavailable or a launch fails.
    """
    if mode not in ("optimized", "conventional"):
        raise ValueError("mode must be 'optimized' or 'conventional'")
    if type(check_inputs) is not bool:
        raise TypeError("check_inputs must be bool")
    if not (emissions and isinstance(emissions[0], Tensor) and emissions[0].is_cuda):
        _metadata(emissions, targets, blank_id)  # raises the reference's ValueError for these inputs
    if _native is None:
        load_extension()
    # the native entry checks every record's metadata with the same messages
    # (O(B) in C++) and passes the fixed knob vector of py:496-501
    tensors, lengths = _native.align(emissions, targets, blank_id, mode == "optimized", check_inputs,
                                     emission_validity)
    return _batch(lengths, tensors)


def align_logits(logits: Sequence[Tensor], targets: Sequence[Tensor], *,
                 blank_id: int | Sequence[int] = 0, mode: Mode = "optimized",
                 check_inputs: bool = True, emission_validity: Tensor | None = None) -> AlignmentBatch:
    """``align`` on raw logits, with the row log-softmax fused into the kernels.

    The producer step of the reference's callers
    (examples/transformers_ctc/align.py:55-56, ``logits.float().log_softmax(-1)``)
    moves inside the alignment: each frame's log-softmax is computed where the
    row is read, so the normalized ``(T, V)`` tensors are never written or read
    back. The result equals ``align(log_softmax(logits), ...)`` bit for bit
    (``log_softmax`` below materializes the same values); ``scores`` are those
    log-probabilities. Same arguments, statuses and exceptions as ``align``,
    with ``logits`` in place of ``emissions``.
    """
    if mode not in ("optimized", "conventional"):
        raise ValueError("mode must be 'optimized' or 'conventional'")
    if type(check_inputs) is not bool:
        raise TypeError("check_inputs must be bool")
    if not (logits and isinstance(logits[0], Tensor) and logits[0].is_cuda):
        _metadata(logits, targets, blank_id)
    if _native is None:
        load_extension()
    tensors, lengths = _native.align(logits, targets, blank_id, mode == "optimized", check_inputs,
                                     emission_validity, True)
    return _batch(lengths, tensors)


def log_softmax(logits: Sequence[Tensor]) -> list[Tensor]:
    """Row log-softmax of ``B`` contiguous CUDA float32 ``(T_i, V_i)`` logits.

    Per row, with ``m = max(x)`` and ``ls = log(sum(exp(x - m)))`` summed in
    one fixed order, returns ``(x - m) - ls`` (torch's formula; within a few
    ulp of ``torch.log_softmax``): exactly the values ``align_logits`` aligns.
    Enqueued on the current stream; no host synchronization.
    """
    if not 0 < len(logits) <= 65535:
        raise ValueError("provide 1..65535 logit tensors")
    if not (isinstance(logits[0], Tensor) and logits[0].is_cuda):
        raise ValueError("logits must be contiguous CUDA float32 [T,V] with supported dimensions on one device")
    load_extension()
    return _native.log_softmax(logits)


@dataclass(frozen=True)
class TokenSpans:
    """Token spans of an alignment: ``spans`` int64 ``(sum(lengths), 2)`` holds,
    per record and in transcript order, the ``[start, end)`` frames of each
    non-blank run of the path (``-1`` rows for records whose status is not 0);
    ``lengths`` the target length of each record."""

    lengths: tuple[int, ...]
    spans: Tensor

    def split(self) -> tuple[Tensor, ...]:
        """Per-record ``(U_i, 2)`` views (no copy, no synchronization)."""
        return self.spans.split(self.lengths)

    def seconds(self, frame_stride: float) -> Tensor:
        """Span boundaries in seconds: frames times the model's frame stride
        (for Transformers CTC models ``inputs_to_logits_ratio / sample_rate``)."""
        return self.spans.to(torch.float64) * frame_stride


def token_spans(batch: AlignmentBatch, targets: Sequence[Tensor] | Sequence[int], *,
                blank_id: int | Sequence[int] = 0) -> TokenSpans:
    """Token spans of ``align``'s paths, computed on the GPU without a host sync.

    Follows the reference README's "Converting frame labels to timestamps":
    split each path into equal-label runs, discard blank runs, and keep each
    remaining run's start and exclusive end frame; blank-separated repeated
    tokens stay separate occurrences. A successful record has exactly one run
    per target token.

    Args:
        batch: the result of ``align``.
        targets: the targets passed to ``align`` (tensors) or their lengths.
        blank_id: the blank id(s) passed to ``align``.

    Raises:
        ValueError: the batch, targets and blanks do not belong together.
    """
    tokens = [t if type(t) is int else int(t.numel()) for t in targets]
    load_extension()
    spans = _native.token_spans(batch.labels, batch.status, batch.lengths, tokens, blank_id)
    return TokenSpans(tuple(tokens), spans)
