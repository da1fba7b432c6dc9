"""Logits-width policy of QSA selection.

Decode scoring writes one fp32 logit per compressed key into a
``[rows, columns]`` buffer, so the column count decides the buffer and the
top-k kernel instance. The reference (``graph_dispatch.py:26-34``) uses two
width classes so captured graphs stay valid across batches: a short class of
32768 columns whenever the longest sequence's compressed length fits it, and
the full page-table capacity otherwise. A graph capture pins the class with
:func:`capture_column_scope`. Prefill sizes its logits by the longest
sequence, rounded up to 64 columns (``ops/indexer.py:320-321``).

The reference also patches vLLM's graph manager to key graphs by this class;
that belongs to the serving runtime, not to this package.
"""

from __future__ import annotations

from contextlib import contextmanager

SHORT_DECODE_COLUMNS = 32768
_pinned_columns: int | None = None


def decode_column_bucket(max_seq_len: int, compress_ratio: int = 4) -> int:
    """Width class of a decode batch: SHORT_DECODE_COLUMNS when its longest
    compressed length fits in it, else 0, meaning the page-table capacity."""
    fits_short = max_seq_len // compress_ratio <= SHORT_DECODE_COLUMNS
    return SHORT_DECODE_COLUMNS if fits_short else 0


def decode_logits_columns(max_seq_len: int, compress_ratio: int, capacity: int) -> int:
    """Logits columns of a decode call, never more than ``capacity`` (the
    compressed page table's width times keys per compressed page)."""
    bucket = _pinned_columns
    if bucket is None:
        bucket = decode_column_bucket(max_seq_len, compress_ratio)
    return capacity if bucket == 0 else min(bucket, capacity)


def prefill_logits_width(max_seq_len: int, compress_ratio: int, capacity: int) -> int:
    """Logits columns of a prefill call: the longest compressed length rounded
    up to a multiple of 64, at least 64, at most ``capacity``."""
    keys = -(-max_seq_len // compress_ratio)
    rounded = -(-keys // 64) * 64
    return min(max(rounded, 64), capacity)


@contextmanager
def capture_column_scope(columns: int):
    """Pin the decode width class (0 = capacity) while a graph is captured."""
    global _pinned_columns
    saved = _pinned_columns
    _pinned_columns = columns
    try:
        yield
    finally:
        _pinned_columns = saved


def check_decode_graph_batch(batch, num_tokens: int, columns: int, compress_ratio: int) -> None:
    """Raise ValueError unless ``batch`` (a ``QSABatch``) may replay a decode
    graph captured for ``num_tokens`` one-token requests under width class
    ``columns``: a batch whose longest compressed length exceeds the captured
    class belongs to the other class's graph (``graph_dispatch.py:26-34``)."""
    if batch.num_tokens != num_tokens or batch.main.max_query_len != 1:
        raise ValueError("batch is not a uniform decode batch of the captured size")
    if columns and batch.compressed.max_seq_len // compress_ratio > columns:
        raise ValueError(
            f"batch needs {batch.compressed.max_seq_len // compress_ratio} logits columns; the "
            f"graph was captured for the {columns}-column width class")

