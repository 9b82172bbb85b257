"""CTC forced alignment on MI355X (gfx950): drop-in for ``fast_forced_aligner``.

``token_spans`` / ``TokenSpans`` extend the reference API with the GPU form of
its documented frame-label-to-timestamp conversion.
"""
from .alignment import AlignmentBatch, TokenSpans, align, emission_validity, load_extension, token_spans, validate_inputs

__all__ = ["AlignmentBatch", "TokenSpans", "align", "emission_validity", "load_extension", "token_spans",
           "validate_inputs"]
