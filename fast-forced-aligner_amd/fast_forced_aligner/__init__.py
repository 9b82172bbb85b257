"""CTC forced alignment on MI355X (gfx950): drop-in for ``fast_forced_aligner``.

``token_spans`` / ``TokenSpans`` extend the reference API with the GPU form of
its documented frame-label-to-timestamp conversion; ``align_logits`` and
``log_softmax`` fuse its callers' log-softmax producer step into the alignment.
"""
from .alignment import (AlignmentBatch, TokenSpans, align, align_logits, emission_validity, load_extension,
                        log_softmax, token_spans, validate_inputs)

__all__ = ["AlignmentBatch", "TokenSpans", "align", "align_logits", "emission_validity", "load_extension",
           "log_softmax", "token_spans", "validate_inputs"]
