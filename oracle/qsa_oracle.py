"""Eager-PyTorch CPU restatement of the YuLan QSA sparse-attention path.

TEST INFRASTRUCTURE ONLY: this module is what the HIP kernels are tested against and
the timed CPU baseline. Nothing under ``qsa_vllm_amd`` imports it.

Every function cites the reference lines it restates (paths relative to the
``yulan_qsa_vllm`` package of clotholza/qsa_vllm). Integer rules (top-k order,
expansion, slot mapping, counts) are restated exactly; floating-point work is
fp32 math on bf16 inputs, as the reference accumulates.

Pinning (how each function is checked independently of its own formula;
``tests/test_oracle_mutants.py`` plants a mistake in each function's source
and requires its pin to fail):

* ``visible_blocks``, ``*_logits_*`` - closed forms on hand-built rows.
* ``indexer_scores_*``    - pure-Python brute-force loops (one and two rows per
                            decode request); ReLU/positivity, positive
                            homogeneity, unit-vector closed forms; prefill rows
                            equal decode rows of the same request.
* ``uint32_keys``, ``topk_ids`` - pure-Python rank counting over (uint32 key
                            desc, id asc); hand-written known answers for ties,
                            -0.0, negatives, inf and NaN bit patterns.
* ``topk_expand``, ``expand_blocks`` - a column-wise restatement of the second
                            statement of the rule in the reference (the Triton
                            expansion kernel, ``ops/qsa.py:18-106``) on the same
                            blocks; hand-built physical mappings;
                            prefix/dup/causal invariants.
* ``store_cache_rows``, ``compress_groups`` - closed form; a walk over member
                            positions.
* ``select_paged_tokens`` - a mixed batch (two rows per decode request, ragged
                            prefill chunks, padding rows) against each row's own
                            selection by loops, rank counting and column-wise
                            expansion, logical and physical.
* ``sparse_attention``    - dense causal GQA through
                            ``torch.nn.functional.scaled_dot_product_attention``
                            when every token is selected; pure-Python softmax
                            loops; one-slot and empty-row closed forms;
                            permutation invariance; duplicate weighting.
* ``sparse_attention_partials``, ``merge_splits`` - LSE identity: split +
                            merge equals one pass.
* ``decode_step``         - slots and counts against each row's selection by
                            loops, the output against softmax loops over the
                            K/V rows at those slots, and against the same tokens
                            given as logical ids through the block table.

Parity unpinned: the un-vendored upstream metadata builder
(``vllm.models.qwen4_exp.common.qsa_cache``, vllm 0.30.0) that produces
``visible_blocks`` / compressed tables in serving. Its outputs are synthesised
from their consumers' contracts here.
"""

from __future__ import annotations

import torch

__all__ = [
    "visible_blocks",
    "decode_logits_columns",
    "prefill_logits_width",
    "indexer_scores_decode",
    "indexer_scores_prefill",
    "uint32_keys",
    "topk_ids",
    "topk_expand",
    "expand_blocks",
    "store_cache_rows",
    "compress_groups",
    "select_paged_tokens",
    "sparse_attention",
    "sparse_attention_partials",
    "merge_splits",
    "decode_step",
]


def visible_blocks(query_positions, sequence_lengths, token_to_req, compress_ratio):
    """``ops/indexer.py:363-369``: complete compressed blocks visible to each row."""
    safe_requests = token_to_req.clamp_min(0).long()
    visible = torch.minimum(
        (query_positions.long() + 1) // compress_ratio,
        sequence_lengths.long().index_select(0, safe_requests) // compress_ratio,
    ).to(torch.int32)
    return torch.where(token_to_req >= 0, visible, torch.zeros_like(visible))


def decode_logits_columns(max_seq_len: int, compress_ratio: int, capacity: int) -> int:
    """``graph_dispatch.py:26-34`` outside graph capture: 32768 short bucket or capacity."""
    columns = 32768 if max_seq_len // compress_ratio <= 32768 else 0
    return min(columns, capacity) if columns else capacity


def _cdiv(a: int, b: int) -> int:
    return (a + b - 1) // b


def prefill_logits_width(max_seq_len: int, compress_ratio: int, columns: int) -> int:
    """``ops/indexer.py:321-323``."""
    width = _cdiv(_cdiv(max_seq_len, compress_ratio), 64) * 64
    return min(max(64, width), columns)


def _cache_3d(k_cache):
    """The compressed key cache is ``[blocks, page, (1,) dim]``; drop the singleton head."""
    if k_cache.dim() == 4:
        return k_cache[:, :, 0, :]
    return k_cache


def _row_scores(q_row, keys):
    """``ops/indexer.py:101-107``: D^-0.5 * sum_h relu(q_h . k), fp32 accumulation."""
    dim = q_row.shape[-1]
    dots = q_row.float() @ keys.float().T  # [heads, n]
    return dots.clamp_min(0.0).sum(0) * (dim ** -0.5)


def indexer_scores_decode(q, k_cache, page_table, visible, decode_query_len, columns):
    """``ops/indexer.py:24-114`` (+ launch ``:241-272``).

    Row ``r`` belongs to request ``r // decode_query_len`` and scores compressed
    keys ``c < min(visible[r], table_width * page)``. Columns that the kernel does
    not store are NaN here.
    """
    kc = _cache_3d(k_cache)
    rows = q.shape[0]
    page = kc.shape[1]
    width = page_table.shape[1]
    num_columns = width * page
    out = torch.full((rows, columns), float("nan"), dtype=torch.float32)
    for r in range(rows):
        req = r // decode_query_len
        n = min(int(visible[r]), num_columns, columns)
        if n <= 0:
            continue
        c = torch.arange(n)
        pages = page_table[req, (c // page).clamp_max(width - 1)].long()
        out[r, :n] = _row_scores(q[r], kc[pages, c % page])
    return out


def indexer_scores_prefill(q, k_cache, page_table, query_start_loc, visible,
                           query_offset, num_rows, width):
    """``ops/indexer.py:117-223`` (+ launch ``:282-302``).

    ``q``/``visible`` are indexed by the prefill-relative absolute row; the
    returned logits rows are relative to ``query_offset``.
    """
    kc = _cache_3d(k_cache)
    page = kc.shape[1]
    table_width = page_table.shape[1]
    num_columns = table_width * page
    base = int(query_start_loc[0])
    out = torch.full((num_rows, width), float("nan"), dtype=torch.float32)
    for req in range(page_table.shape[0]):
        start = max(int(query_start_loc[req]) - base, query_offset)
        end = min(int(query_start_loc[req + 1]) - base, query_offset + num_rows)
        for r in range(start, end):
            n = min(int(visible[r]), num_columns, width)
            if n <= 0:
                continue
            c = torch.arange(n)
            pages = page_table[req, (c // page).clamp_max(table_width - 1)].long()
            out[r - query_offset, :n] = _row_scores(q[r], kc[pages, c % page])
    return out


def uint32_keys(scores):
    """The reference orders scores by their raw fp32 bit pattern as uint32
    (``ops/csrc/topk.cu:262, 287, 331-338``)."""
    return scores.contiguous().view(torch.int32).long() & 0xFFFFFFFF


def topk_ids(scores, lengths, k):
    """``ops/csrc/topk.cu:182-350`` selection with ``CompressedWriter`` (``:90-95``).

    Per row with ``L = lengths[r]``: ``L <= k`` -> ids ``0..L-1`` then -1;
    otherwise the k ids with the largest uint32 keys, lowest id first on ties,
    emitted in ascending id order.
    """
    rows = scores.shape[0]
    out = torch.full((rows, k), -1, dtype=torch.int32)
    for r in range(rows):
        length = int(lengths[r])
        if length <= k:
            if length > 0:
                out[r, :length] = torch.arange(length, dtype=torch.int32)
            continue
        assert length <= scores.shape[1], "length beyond the logits row"
        keys = uint32_keys(scores[r, :length])
        order = torch.sort(-keys, stable=True).indices[:k]
        out[r] = torch.sort(order).values.to(torch.int32)
    return out


def topk_expand(scores, lengths, positions, sequence_lengths, token_to_req, table,
                output_width, ratio, page_size, physical):
    """``ops/csrc/topk.cu:97-180, 410-422, 470-525``: select, expand, tail, map, count.

    Returns ``(out[rows, output_width] int32, counts[rows] int32)``.
    """
    k = output_width // ratio
    ids = topk_ids(scores, lengths, k)
    return expand_blocks(ids, positions, sequence_lengths, token_to_req, table, output_width,
                         ratio, page_size, physical, k)


def expand_blocks(block_ids, positions, sequence_lengths, token_to_req, table, output_width,
                  ratio, page_size, physical, k):
    """Expansion of ranked block ids (rank i < k is ``block_ids[:, i]``, any order,
    -1 for none) with the causal tail, mapping and counts: ``ops/csrc/topk.cu:97-180``
    and its Triton twin ``ops/qsa.py:18-106``. Returns ``(out, counts)``."""
    ids = block_ids[:, :k].long()
    rows = ids.shape[0]
    num_requests = sequence_lengths.numel()
    req = token_to_req.long()
    mapped = (req >= 0) & (req < num_requests)
    safe_req = req.clamp(0, max(num_requests - 1, 0))
    seq_len = torch.where(mapped, sequence_lengths.long()[safe_req], torch.zeros_like(req))
    pos = positions.long()
    pos = ((pos + 2**31) % 2**32) - 2**31          # int(positions[row]) truncation
    assert bool((pos >= -1).all()), "negative positions are undefined in the reference"
    p1 = pos + 1                                    # >= 0, so floor == C truncation below
    complete = torch.minimum(torch.minimum(p1 // ratio, seq_len // ratio),
                             torch.full_like(p1, k))
    tail_start = (p1 // ratio) * ratio
    tail_count = p1 - tail_start
    expanded = complete * ratio

    col = torch.arange(output_width)[None, :]
    rank = (col // ratio).clamp_max(k - 1)
    block = torch.gather(ids, 1, rank.expand(rows, -1))
    in_blocks = col < expanded[:, None]
    off = col - expanded[:, None]
    in_tail = (~in_blocks) & (off < tail_count[:, None]) & (off < ratio - 1)
    token = torch.where(in_blocks, block * ratio + col % ratio, tail_start[:, None] + off)
    valid = (in_blocks | in_tail) & (token >= 0) & (token < seq_len[:, None])
    if physical:
        table_width = table.shape[1]
        logical_page = token.clamp_min(0) // page_size
        valid &= logical_page < table_width
        physical_page = table.long()[safe_req[:, None], logical_page.clamp_max(table_width - 1)]
        valid &= physical_page >= 0
        token = physical_page * page_size + token.clamp_min(0) % page_size
    out = torch.where(valid, token, torch.full_like(token, -1)).to(torch.int32)
    counts = torch.minimum(expanded + tail_count, seq_len).to(torch.int32)
    return out, counts


def store_cache_rows(cache, slot_mapping, rows):
    """``qsa_store_cache_rows`` (ops/qsa.py:366-401, 691-706): row r into
    cache[slot // page, slot % page, 0, :width] when 0 <= slot < blocks * page."""
    rows = rows[:, 0] if rows.dim() == 3 else rows
    page, width = cache.shape[1], cache.shape[3]
    for r, slot in enumerate(slot_mapping.tolist()[:rows.shape[0]]):
        if 0 <= slot < cache.shape[0] * page:
            cache[slot // page, slot % page, 0, :width] = rows[r, :width]


def compress_groups(raw_keys, raw_positions, state_cache, state_table, token_to_req,
                    query_start_loc, logical_positions, compressed_slots, ratio, rope_cache=None):
    """``qsa_compress_groups_with_ratio`` (ops/qsa.py:403-549, 709-750). Returns
    ``(pooled [rows, 1, dim] bf16, first_positions [rows, 3] int64)``."""
    rows, dim = token_to_req.numel(), raw_keys.shape[-1]
    keys = raw_keys.reshape(raw_keys.shape[0], -1)[:, :dim].float()
    ring = state_cache.reshape(state_cache.shape[0], state_cache.shape[1], -1)[..., :dim].float()
    S = state_cache.shape[1]
    qsl = query_start_loc.tolist()
    nreq = len(qsl) - 1
    pooled = torch.zeros(rows, 1, dim, dtype=torch.float32)
    first_positions = torch.zeros(rows, 3, dtype=torch.int64)
    for row in range(rows):
        req = int(token_to_req[row])
        end = int(logical_positions[row])
        slot = int(compressed_slots[row])
        req_ok = 0 <= req < nreq
        qs, qe = (qsl[req], qsl[req + 1]) if req_ok else (0, 0)
        block = int(state_table[req, 0]) if req_ok else -1
        ring_ok = 0 <= block < ring.shape[0]
        chunk_start = end - (row - qs)
        valid = req_ok and qs <= row < qe and end >= ratio - 1 and slot >= 0
        acc = torch.zeros(dim, dtype=torch.float32)
        for m in range(ratio):
            position = end - (ratio - 1) + m
            if not valid:
                continue
            if position >= chunk_start:
                raw_row = qs + position - chunk_start
                if qs <= raw_row < qe and raw_row < rows:
                    acc = acc + keys[raw_row]
            elif ring_ok:
                acc = acc + ring[block, position % S]
        pooled[row, 0] = acc / torch.tensor(float(ratio), dtype=torch.float32)
        first = end - ratio + 1
        if rope_cache is None:
            first_positions[row] = first if valid else 0
        elif valid and first >= chunk_start:
            raw_first = qs + first - chunk_start
            if qs <= raw_first < qe and raw_first < rows:
                first_positions[row] = raw_positions.reshape(raw_positions.shape[0], -1)[raw_first, :3]
        elif valid and ring_ok:
            first_positions[row] = rope_cache.reshape(rope_cache.shape[0], rope_cache.shape[1],
                                                      -1)[block, first % S, :3]
    return pooled.to(torch.bfloat16), first_positions


def select_paged_tokens(q, k_cache, page_table, token_to_req, query_positions,
                        sequence_lengths, token_topk, compress_ratio, *, query_start_loc,
                        max_query_len, max_seq_len, num_decodes=0, num_decode_tokens=0,
                        decode_query_len=1, visible_blocks_in=None, main_block_table=None,
                        main_page_size=1):
    """``ops/indexer.py:227-393``: decode rows then prefill rows, scoring + top-k.

    Returns ``(indices, counts, visible)``.
    """
    rows = q.shape[0]
    width = token_topk + compress_ratio - 1
    out = torch.full((rows, width), -1, dtype=torch.int32)
    counts = torch.zeros(rows, dtype=torch.int32)
    if rows == 0:
        return out, counts, torch.zeros(0, dtype=torch.int32)
    if visible_blocks_in is None:
        visible = visible_blocks(query_positions, sequence_lengths, token_to_req, compress_ratio)
    else:
        visible = visible_blocks_in
    kc = _cache_3d(k_cache)
    physical = main_block_table is not None
    table = main_block_table if physical else torch.zeros((1, 1), dtype=torch.int32)
    if num_decode_tokens:
        capacity = page_table.shape[1] * kc.shape[1]
        columns = decode_logits_columns(max_seq_len, compress_ratio, capacity)
        logits = indexer_scores_decode(q[:num_decode_tokens], kc, page_table[:num_decodes],
                                       visible[:num_decode_tokens], decode_query_len, columns)
        o, c = topk_expand(logits, visible[:num_decode_tokens],
                           query_positions[:num_decode_tokens], sequence_lengths,
                           token_to_req[:num_decode_tokens], table, width,
                           compress_ratio, main_page_size, physical)
        out[:num_decode_tokens] = o
        counts[:num_decode_tokens] = c
    if num_decode_tokens < rows:
        columns = page_table.shape[1] * kc.shape[1]
        lw = prefill_logits_width(max_seq_len, compress_ratio, columns)
        n = rows - num_decode_tokens
        logits = indexer_scores_prefill(q[num_decode_tokens:], kc, page_table[num_decodes:],
                                        query_start_loc[num_decodes:],
                                        visible[num_decode_tokens:], 0, n, lw)
        o, c = topk_expand(logits, visible[num_decode_tokens:],
                           query_positions[num_decode_tokens:], sequence_lengths,
                           token_to_req[num_decode_tokens:], table, width,
                           compress_ratio, main_page_size, physical)
        out[num_decode_tokens:] = o
        counts[num_decode_tokens:] = c
    return out, counts, visible


def _gather_valid(indices_row, n, k_cache, v_cache, block_table, request, num_requests,
                  physical):
    """``ops/qsa.py:186-232``: slot validity and the K/V rows of valid slots."""
    num_blocks, page = k_cache.shape[0], k_cache.shape[1]
    tok = indices_row[:n].long()
    safe = tok.clamp_min(0)
    logical_page = safe // page
    offset = safe % page
    if physical:
        physical_page = logical_page
        valid = (tok >= 0) & (physical_page < num_blocks)
    else:
        width = block_table.shape[1]
        req_ok = 0 <= request < num_requests
        safe_req = min(max(request, 0), num_requests - 1)
        valid = (tok >= 0) & (logical_page < width) & req_ok
        physical_page = torch.where(
            valid, block_table[safe_req, logical_page.clamp_max(width - 1)].long(),
            torch.full_like(logical_page, -1))
        valid &= (physical_page >= 0) & (physical_page < num_blocks)
    pp = physical_page[valid]
    off = offset[valid]
    return k_cache[pp, off].float(), v_cache[pp, off].float()


def sparse_attention(q, k_cache, v_cache, indices, block_table, token_to_req, *,
                     output_gate=None, indices_are_physical=False, valid_counts=None):
    """``ops/qsa.py:109-303, 594-688`` as fp32 math; returns fp32 ``[rows, Hq, D]``.

    Head ``h`` attends with kv head ``h // (Hq / Hkv)`` over the valid slots of
    ``indices[r, :n]`` where ``n = min(valid_counts[r], W)`` (decode) or ``W``.
    Empty rows give 0. With a gate the output is ``bf16(o) * sigmoid(gate)``
    (``:257-269``). The reference rounds P to bf16 before P@V (``:242-246``);
    this oracle keeps P in fp32 - the tolerance covers the difference.
    """
    rows, num_q_heads, dim = q.shape
    num_kv_heads = k_cache.shape[2]
    group = num_q_heads // num_kv_heads
    width = indices.shape[1]
    num_requests = block_table.shape[0]
    out = torch.zeros((rows, num_q_heads, dim), dtype=torch.float32)
    scale = dim ** -0.5
    for r in range(rows):
        n = width if valid_counts is None else max(0, min(int(valid_counts[r]), width))
        keys, values = _gather_valid(indices[r], n, k_cache, v_cache, block_table,
                                     int(token_to_req[r]), num_requests,
                                     indices_are_physical)
        if keys.shape[0] == 0:
            continue
        for g in range(num_kv_heads):
            qg = q[r, g * group:(g + 1) * group].float()
            s = (qg @ keys[:, g].T) * scale
            p = torch.softmax(s, dim=-1)
            out[r, g * group:(g + 1) * group] = p @ values[:, g]
    if output_gate is not None:
        out = out.to(torch.bfloat16).float() * torch.sigmoid(output_gate.float())
    return out


def sparse_attention_partials(q, k_cache, v_cache, indices, block_table, token_to_req,
                              num_splits, *, indices_are_physical=False, valid_counts=None,
                              block_n=32):
    """``ops/qsa.py:178-184, 250-303``: per-split normalised output and log2-LSE.

    Split ``s`` covers tiles ``[s*T//S, (s+1)*T//S)`` of ``T = cdiv(n, block_n)``.
    Returns ``(partial_out [S, rows, Hq, D], partial_lse [S, rows, Hq])``.
    """
    rows, num_q_heads, dim = q.shape
    num_kv_heads = k_cache.shape[2]
    group = num_q_heads // num_kv_heads
    width = indices.shape[1]
    num_requests = block_table.shape[0]
    po = torch.zeros((num_splits, rows, num_q_heads, dim), dtype=torch.float32)
    pl = torch.full((num_splits, rows, num_q_heads), float("-inf"), dtype=torch.float32)
    scale_log2 = dim ** -0.5 * 1.4426950408889634
    for r in range(rows):
        n = width if valid_counts is None else max(0, min(int(valid_counts[r]), width))
        tiles = -(-n // block_n)
        for s in range(num_splits):
            lo = min(n, (s * tiles // num_splits) * block_n)
            hi = min(n, ((s + 1) * tiles // num_splits) * block_n)
            sub = indices[r].clone()
            sub[:lo] = -1
            keys, values = _gather_valid(sub, hi, k_cache, v_cache, block_table,
                                         int(token_to_req[r]), num_requests,
                                         indices_are_physical)
            if keys.shape[0] == 0:
                continue
            for g in range(num_kv_heads):
                qg = q[r, g * group:(g + 1) * group].float()
                sc = (qg @ keys[:, g].T) * scale_log2
                m = sc.max(dim=-1).values
                p = torch.exp2(sc - m[:, None])
                l = p.sum(-1)
                po[s, r, g * group:(g + 1) * group] = (p @ values[:, g]) / l[:, None]
                pl[s, r, g * group:(g + 1) * group] = m + torch.log2(l)
    return po, pl


def merge_splits(partial_out, partial_lse, output_gate=None):
    """``ops/qsa.py:306-362``: LSE-weighted (log2 domain) merge of split partials."""
    lse_max = partial_lse.max(dim=0).values
    has = lse_max > float("-inf")
    shifted = torch.where(has[None], partial_lse - lse_max[None],
                          torch.full_like(partial_lse, float("-inf")))
    weights = torch.exp2(shifted)
    denom = weights.sum(0)
    merged = (partial_out * weights[..., None]).sum(0)
    merged = torch.where(denom[..., None] > 0, merged / denom.clamp_min(1e-38)[..., None],
                         torch.zeros_like(merged))
    if output_gate is not None:
        merged = merged.to(torch.bfloat16).float() * torch.sigmoid(output_gate.float())
    return merged


def decode_step(q_idx, k_idx_cache, idx_page_table, q, k_cache, v_cache, block_table,
                positions, seq_lens, token_topk, compress_ratio, *, output_gate=None):
    """One uniform-decode QSA layer step (``attention.py:191-214`` →
    ``backend.py:39-68``): indexer scores → top-k/expand with physical slots and
    counts → sparse attention. Returns ``(out fp32, indices, counts)``."""
    rows = q.shape[0]
    token_to_req = torch.arange(rows, dtype=torch.int32)
    query_start_loc = torch.arange(rows + 1, dtype=torch.int32)
    max_seq_len = int(seq_lens.max()) if rows else 0
    indices, counts, _ = select_paged_tokens(
        q_idx, k_idx_cache, idx_page_table, token_to_req, positions, seq_lens,
        token_topk, compress_ratio, query_start_loc=query_start_loc, max_query_len=1,
        max_seq_len=max_seq_len, num_decodes=rows, num_decode_tokens=rows,
        main_block_table=block_table, main_page_size=k_cache.shape[1])
    out = sparse_attention(q, k_cache, v_cache, indices, block_table, token_to_req,
                           output_gate=output_gate, indices_are_physical=True,
                           valid_counts=counts)
    return out, indices, counts
