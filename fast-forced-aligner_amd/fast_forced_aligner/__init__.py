"""CTC forced alignment on MI355X (gfx950): drop-in for ``fast_forced_aligner``."""
from .alignment import AlignmentBatch, align, emission_validity, load_extension, validate_inputs

__all__ = ["AlignmentBatch", "align", "emission_validity", "load_extension", "validate_inputs"]
