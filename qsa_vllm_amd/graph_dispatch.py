"""Decode logits-width buckets for QSA selection.

Restates the column policy of the reference ``graph_dispatch.py:313-342``:
decode rows whose compressed length fits 32768 columns share one short
logits width; longer batches use the full page-table capacity. Graph capture
pins the width through ``capture_column_scope``. The vLLM graph-manager
patches of the reference (``install_short_decode_dispatch``) belong to the
serving runtime and are not part of this package.
"""

from __future__ import annotations

from contextlib import contextmanager

SHORT_DECODE_COLUMNS = 32768
_capture_columns = None


def decode_column_bucket(max_seq_len: int, compress_ratio: int = 4) -> int:
    """Zero denotes the full page-table capacity; short rows use one selector."""
    return SHORT_DECODE_COLUMNS if max_seq_len // compress_ratio <= SHORT_DECODE_COLUMNS else 0


def decode_logits_columns(max_seq_len: int, compress_ratio: int, capacity: int) -> int:
    columns = (_capture_columns if _capture_columns is not None
               else decode_column_bucket(max_seq_len, compress_ratio))
    return min(columns, capacity) if columns else capacity


@contextmanager
def capture_column_scope(columns):
    """Fix the decode logits width (0 = capacity) while capturing a graph."""
    global _capture_columns
    previous = _capture_columns
    _capture_columns = columns
    try:
        yield
    finally:
        _capture_columns = previous
